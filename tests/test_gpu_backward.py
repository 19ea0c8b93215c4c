"""GPU parity of the differentiable HIP experts (q38.hip.autograd) against CPU autograd of the
reference's eager experts (modeling:769-793, oracle.experts_eager).

The reference's own gradient check (scripts/check_q38_kernels.py:19-27) compares its kernel path
with the eager bf16 autograd. Here both sides are measured against fp32 autograd of the same
bf16-valued inputs: every gradient of the HIP path must lie within relative L2 2.5e-2 of it (the
reference's tolerance, rtol 0.025) and within twice the error of the eager bf16 autograd plus 2e-3
(the HIP path rounds at the same points as bf16 autograd; only fp32 summation order differs).
The forward output keeps the forward tolerance (tests/_util.py).
"""
import pytest
import torch

from _util import assert_bf16_close, assert_gemm_bf16_rounding
from oracle import moe_oracle as orc

pytestmark = pytest.mark.gpu

REL = 2.5e-2


def _inputs(name, T, drop=0):
    from q38 import workloads
    wl = workloads.get(name)
    x, params, _ = workloads.make(wl, tokens=T)
    _, _, idx, w = orc.router(x, params["gate.weight"], wl.topk)
    if drop:
        # Dropped pairs (index E): they contribute nothing and get zero weight gradient.
        g = torch.Generator().manual_seed(7)
        sel = torch.randperm(idx.numel(), generator=g)[:drop]
        idx.view(-1)[sel] = wl.experts
    gdo = torch.Generator().manual_seed(11)
    dout = (torch.randn(T, wl.hidden, generator=gdo) * 0.05).to(torch.bfloat16)
    return wl, x, idx, w, params["experts.gate_up_proj"], params["experts.down_proj"], dout


def _cpu_grads(x, idx, w, wgu, wdn, dout, dtype):
    leaves = [t.detach().to(dtype).requires_grad_(True) for t in (x, w, wgu, wdn)]
    out = orc.experts_eager(leaves[0], idx, *leaves[1:])
    out.backward(dout.to(dtype))
    return out.detach().float(), [t.grad.float() for t in leaves]


def _rel(a, b):
    a, b = a.detach().float().cpu(), b.detach().float().cpu()
    return float((a - b).norm() / b.norm().clamp_min(1e-30))


@pytest.mark.parametrize("name,T,drop", [("c1", 53, 0), ("c1", 700, 40), ("c2", 2048, 0), ("c2", 3001, 97)])
def test_experts_backward(gpu, name, T, drop):
    from q38.hip import autograd
    wl, x, idx, w, wgu, wdn, dout = _inputs(name, T, drop)
    ref_out, ref_g = _cpu_grads(x, idx, w, wgu, wdn, dout, torch.float32)
    _, eager_g = _cpu_grads(x, idx, w, wgu, wdn, dout, torch.bfloat16)
    leaves = [t.to(gpu).requires_grad_(True) for t in (x, w, wgu, wdn)]
    out = autograd.experts(leaves[0], idx.to(gpu), *leaves[1:])
    out.backward(dout.to(gpu))
    torch.cuda.synchronize()
    assert_bf16_close(out, ref_out, what=f"{name} T={T} forward")
    for nm, leaf, r, e in zip(("x", "top_k_weights", "gate_up_proj", "down_proj"), leaves, ref_g, eager_g):
        g = leaf.grad
        assert g is not None and g.dtype == torch.bfloat16 and g.shape == leaf.shape, nm
        assert torch.isfinite(g.float()).all(), f"{nm}: non-finite gradient"
        err, eager_err = _rel(g, r), _rel(e, r)
        assert err <= REL, f"{name} T={T} d{nm}: rel {err:.3e} vs fp32 autograd (<= {REL})"
        assert err <= 2 * eager_err + 2e-3, f"{name} T={T} d{nm}: rel {err:.3e}, eager bf16 {eager_err:.3e}"
    if drop:
        dropped = idx.to(gpu) == wl.experts
        assert bool((leaves[1].grad[dropped] == 0).all()), "dropped pairs must get a zero weight gradient"


def test_experts_backward_partial_grads(gpu):
    """Only some inputs need gradients (frozen experts, or frozen router weights)."""
    from q38.hip import autograd
    _, x, idx, w, wgu, wdn, dout = _inputs("c1", 301)
    _, ref_g = _cpu_grads(x, idx, w, wgu, wdn, dout, torch.float32)
    xg = x.to(gpu).requires_grad_(True)
    wg = w.to(gpu).requires_grad_(True)
    out = autograd.experts(xg, idx.to(gpu), wg, wgu.to(gpu), wdn.to(gpu))
    out.backward(dout.to(gpu))
    assert _rel(xg.grad, ref_g[0]) <= REL and _rel(wg.grad, ref_g[1]) <= REL
    wdg = wdn.to(gpu).requires_grad_(True)
    out = autograd.experts(x.to(gpu), idx.to(gpu), w.to(gpu), wgu.to(gpu), wdg)
    out.backward(dout.to(gpu))
    assert _rel(wdg.grad, ref_g[3]) <= REL


def test_experts_backward_fp32_params_under_autocast(gpu):
    """fp32 leaves under bf16 autocast (the reference's training setup, scripts/check_q38_kernels.py:
    19-26): the kernels run on bf16 casts, the output comes back in fp32 and every gradient arrives
    in fp32, within the reference's bar of fp32 autograd; outside autocast fp32 is refused."""
    from q38.hip import autograd
    from q38.inference import hip_experts_forward
    _, x, idx, w, wgu, wdn, dout = _inputs("c1", 411)
    _, ref_g = _cpu_grads(x, idx, w, wgu, wdn, dout, torch.float32)
    leaves = [t.float().to(gpu).requires_grad_(True) for t in (x, w, wgu, wdn)]
    with torch.autocast("cuda", dtype=torch.bfloat16):
        out = autograd.experts(leaves[0], idx.to(gpu), *leaves[1:])
    assert out.dtype == torch.float32
    out.backward(dout.float().to(gpu))
    for nm, leaf, r in zip(("x", "top_k_weights", "gate_up_proj", "down_proj"), leaves, ref_g):
        assert leaf.grad is not None and leaf.grad.dtype == torch.float32, nm
        assert _rel(leaf.grad, r) <= REL, f"d{nm}: rel {_rel(leaf.grad, r):.3e}"
    # The registered implementation with fp32 module parameters, as a model trains under autocast.

    class Experts(torch.nn.Module):
        def __init__(self):
            super().__init__()
            self.gate_up_proj = torch.nn.Parameter(wgu.float().to(gpu))
            self.down_proj = torch.nn.Parameter(wdn.float().to(gpu))

    m = Experts()
    xg = x.float().to(gpu).requires_grad_(True)
    with torch.autocast("cuda", dtype=torch.bfloat16):
        out = hip_experts_forward(m, xg, idx.to(gpu), w.float().to(gpu))
    out.backward(dout.float().to(gpu))
    assert m.gate_up_proj.grad.dtype == torch.float32 and _rel(m.gate_up_proj.grad, ref_g[2]) <= REL
    assert _rel(xg.grad, ref_g[0]) <= REL and _rel(m.down_proj.grad, ref_g[3]) <= REL
    with pytest.raises(TypeError, match="autocast"):
        autograd.experts(*[t.detach().requires_grad_(True) for t in (leaves[0],)], idx.to(gpu),
                         *[t.detach().requires_grad_(True) for t in leaves[1:]])


def test_registered_experts_train(gpu):
    """The registered ExpertsInterface implementation runs the differentiable path under autograd
    (module parameters with requires_grad) and the plain forward under inference_mode."""
    from q38.inference import hip_experts_forward
    _, x, idx, w, wgu, wdn, dout = _inputs("c1", 257)
    _, ref_g = _cpu_grads(x, idx, w, wgu, wdn, dout, torch.float32)

    class Experts(torch.nn.Module):
        def __init__(self):
            super().__init__()
            self.gate_up_proj = torch.nn.Parameter(wgu.to(gpu))
            self.down_proj = torch.nn.Parameter(wdn.to(gpu))

    m = Experts()
    xg = x.to(gpu).requires_grad_(True)
    out = hip_experts_forward(m, xg, idx.to(gpu), w.to(gpu))
    out.backward(dout.to(gpu))
    assert _rel(xg.grad, ref_g[0]) <= REL
    assert _rel(m.gate_up_proj.grad, ref_g[2]) <= REL and _rel(m.down_proj.grad, ref_g[3]) <= REL
    with torch.inference_mode():
        out2 = hip_experts_forward(m, x.to(gpu), idx.to(gpu), w.to(gpu))
    assert torch.equal(out.detach(), out2)


@pytest.mark.parametrize("E,k,T,h,I,drop", [(64, 5, 2048, 1024, 256, 0), (8, 2, 301, 64, 64, 17),
                                            (16, 3, 999, 192, 320, 50), (4, 1, 5, 128, 64, 0)])
def test_expert_wgrad(gpu, E, k, T, h, I, drop):
    """q38moe_expert_wgrad in both forms against exact per-expert products: every element within
    one bf16 ulp of the exact value plus an fp32 accumulation allowance (one rounding of an fp32
    accumulation); experts without rows get zeros; the permutation equals the oracle's."""
    from q38.hip import ops
    g = torch.Generator().manual_seed(E * 1000 + T)
    idx = torch.randint(0, E, (T, k), generator=g, dtype=torch.int32)
    if E > 4:
        idx[idx == 1] = 2  # expert 1 gets no rows
    if drop:
        idx.view(-1)[torch.randperm(T * k, generator=g)[:drop]] = E
    x = torch.randn(T, h, generator=g).to(torch.bfloat16)
    G = torch.randn(T * k, 2 * I, generator=g).to(torch.bfloat16)
    Gd = torch.randn(T * k, h, generator=g).to(torch.bfloat16)
    Hs = torch.randn(T * k, I, generator=g).to(torch.bfloat16)
    di = idx.to(gpu)
    counts, starts, perm, _, _, _ = ops.permute(di, ops.histogram(di, E), E)
    dgu = ops.expert_wgrad(G.to(gpu), x.to(gpu), starts, counts, k, perm=perm)
    ddn = ops.expert_wgrad(Gd.to(gpu), Hs.to(gpu), starts, counts, k)
    torch.cuda.synchronize()
    assert dgu.shape == (E, 2 * I, h) and ddn.shape == (E, h, I)
    c_ref, s_ref, p_ref = orc.permute_cpu(idx.numpy(), E)
    assert torch.equal(perm.cpu()[: int(c_ref.sum())], torch.from_numpy(p_ref.astype("int32")))
    assert torch.equal(counts.cpu(), torch.from_numpy(c_ref.astype("int32")))
    for e in range(E):
        s0, c = int(s_ref[e]), int(c_ref[e])
        rows = torch.from_numpy(p_ref[s0:s0 + c].astype("int64"))
        if c == 0:
            assert not dgu[e].any() and not ddn[e].any(), f"expert {e} has no rows but a nonzero gradient"
            continue
        assert_gemm_bf16_rounding(dgu[e].cpu(), G[s0:s0 + c].float().T.contiguous(),
                                  x[rows // k].float().T.contiguous(), what=f"d gate_up_proj[{e}]")
        assert_gemm_bf16_rounding(ddn[e].cpu(), Gd[s0:s0 + c].float().T.contiguous(),
                                  Hs[s0:s0 + c].float().T.contiguous(),
                                  what=f"d down_proj[{e}]")


def test_expert_wgrad_no_rows(gpu):
    """T = 0: every expert's gradient is zero (the counts are not read)."""
    from q38.hip import ops
    E, k = 8, 2
    z = torch.zeros(E, dtype=torch.int32, device=gpu)
    dW = ops.expert_wgrad(torch.empty(0, 128, dtype=torch.bfloat16, device=gpu),
                          torch.empty(0, 64, dtype=torch.bfloat16, device=gpu), z, z, k,
                          perm=torch.empty(0, dtype=torch.int32, device=gpu))
    torch.cuda.synchronize()
    assert dW.shape == (E, 128, 64) and not dW.any()


@pytest.mark.parametrize("E,R,C", [(64, 1024, 256), (64, 512, 1024), (3, 64, 192), (1, 320, 64)])
def test_transpose_experts(gpu, E, R, C):
    """q38moe_transpose_experts is a bit-exact per-expert transpose."""
    from q38.hip import ops
    w = torch.randn(E, R, C, generator=torch.Generator().manual_seed(R + C)).to(torch.bfloat16)
    out = ops.transpose_experts(w.to(gpu))
    torch.cuda.synchronize()
    assert out.shape == (E, C, R) and torch.equal(out.cpu(), w.transpose(1, 2).contiguous())


@pytest.mark.parametrize("E,k,T,K,N,drop", [(64, 5, 2048, 1024, 256, 0), (64, 5, 2048, 512, 1024, 37),
                                             (3, 2, 700, 320, 192, 5), (17, 8, 300, 64, 448, 0),
                                             (1, 1, 999, 128, 64, 0)])
def test_down_kn(gpu, E, k, T, K, N, drop):
    """q38moe_down_kn (weights [E, K, N] as stored, read with the transposing LDS read) against
    q38moe_down on the per-expert transposes: bit-identical (same products, K order and rounding;
    T*k > 32 E, so q38moe_down runs the persistent kernel too). And against exact per-expert
    products: each value within one bf16 rounding plus 2^-20 of the sum of |a*w| (fp32
    accumulation). Shapes: configuration 2's dH (K = h, N = I) and input-row (K = 2I, N = h)
    products, N not a multiple of 256, K of one or two slices, a single expert, dropped pairs."""
    from q38.hip import ops
    g = torch.Generator().manual_seed(K * 7 + N)
    idx = torch.stack([torch.randperm(E, generator=g)[:k] for _ in range(T)]).to(torch.int32)
    if drop:
        idx.view(-1)[torch.randperm(T * k, generator=g)[:drop]] = E
    A = (torch.randn(T * k, K, generator=g) * 0.5).to(torch.bfloat16)
    W = (torch.randn(E, K, N, generator=g) * 0.05).to(torch.bfloat16)
    di = idx.to(gpu)
    hist = ops.histogram(di, E)
    counts, starts, perm, inv, tiles, tc = ops.permute(di, hist, E)
    dA, dW = A.to(gpu), W.to(gpu)
    Y = ops.down_kn(dA, dW, tiles, tc, T, k)
    Yt = ops.down(dA, ops.transpose_experts(dW), tiles, tc, T, k)
    torch.cuda.synchronize()
    rows = int(counts.sum())
    assert torch.equal(Y[:rows].cpu(), Yt[:rows].cpu())
    st, ct = starts.cpu().tolist(), counts.cpu().tolist()
    Yc = Y.cpu().double()
    for e in range(E):
        if ct[e] == 0:
            continue
        a = A[st[e]:st[e] + ct[e]].double()
        exact = a @ W[e].double()
        mag = a.abs() @ W[e].double().abs()
        ulp = torch.pow(2.0, torch.floor(torch.log2(exact.abs().clamp_min(1e-38))) - 7)
        err = (Yc[st[e]:st[e] + ct[e]] - exact).abs()
        assert bool((err <= ulp + mag * 2.0 ** -20).all()), f"expert {e}: worst {float((err - ulp - mag * 2.0 ** -20).max()):.3e}"


@pytest.mark.parametrize("name,T,drop,over", [("c2", 2048, 0, {}), ("c1", 700, 40, {}),
                                              ("c2", 333, 9, {"experts": 7, "topk": 3, "hidden": 320, "inter": 192})])
def test_gate_up_save(gpu, name, T, drop, over):
    """q38moe_gate_up_save: H bit-identical to q38moe_gate_up on the same tiles (persistent kernel),
    GU bit-identical to q38moe_gather_gemm's recomputation (the values H is computed from, same K
    order), and GU within one bf16 rounding + fp32 accumulation of the exact products."""
    from q38 import workloads
    from q38.hip import ops
    wl = workloads.get(name, **over)
    x, params, _ = workloads.make(wl, tokens=T)
    k, E = wl.topk, wl.experts
    _, _, idx, _ = orc.router(x, params["gate.weight"], k)
    if drop:
        idx.view(-1)[torch.randperm(idx.numel(), generator=torch.Generator().manual_seed(5))[:drop]] = E
    wgu = params["experts.gate_up_proj"]
    dx, dwgu, di = x.to(gpu), wgu.to(gpu), idx.to(gpu)
    hist = ops.histogram(di, E)
    counts, starts, perm, inv, tiles, tc = ops.permute(di, hist, E)
    H, GU = ops.gate_up_save(dx, dwgu, perm, tiles, tc, k)
    GU2 = ops.gather_gemm(dx, perm, dwgu, tiles, tc, k)
    torch.cuda.synchronize()
    rows = int(counts.sum())
    assert torch.equal(GU[:rows].cpu(), GU2[:rows].cpu())
    if ops.gemm_tiling(T, wl.hidden, E, k, wl.inter, 0) == "persistent":
        H2 = ops.gate_up(dx, dwgu, perm, tiles, tc, k)
        torch.cuda.synchronize()
        assert torch.equal(H[:rows].cpu(), H2[:rows].cpu())
    xs = x[perm[:rows].cpu().long() // k]
    e_of = torch.repeat_interleave(torch.arange(E), counts.cpu().long())
    assert_gemm_bf16_rounding(GU[:rows].cpu()[e_of == 0], xs[e_of == 0], wgu[0], what="GU expert 0")


def test_expert_only_kernels_skip_shared_tiles(gpu):
    """q38moe_down_kn and q38moe_gate_up_save given a tile table that also holds shared-expert rows
    (q38moe_permute with shared_rows = T, through the C ABI: the Python wrappers refuse it): the
    routed rows equal the expert-only table's results and the rows from T*k on stay untouched."""
    from q38 import workloads
    from q38.hip import ops
    wl = workloads.get("c2")
    T, k, E, h, I = 2048, wl.topk, wl.experts, wl.hidden, wl.inter
    x, params, _ = workloads.make(wl, tokens=T)
    _, _, idx, _ = orc.router(x, params["gate.weight"], k)
    dx, di = x.to(gpu), idx.to(gpu)
    dwgu, dwdn = params["experts.gate_up_proj"].to(gpu), params["experts.down_proj"].to(gpu)
    hist = ops.histogram(di, E)
    counts, starts, perm, inv, tiles, tc = ops.permute(di, hist, E)
    _, _, perm_s, _, tiles_s, tc_s = ops.permute(di, hist, E, shared_rows=T)
    P = T * k
    H_ref, GU_ref = ops.gate_up_save(dx, dwgu, perm, tiles, tc, k)
    A = (torch.randn(P, h, generator=torch.Generator().manual_seed(3)) * 0.5).to(torch.bfloat16).to(gpu)
    Y_ref = ops.down_kn(A, dwdn, tiles, tc, T, k)
    pattern = torch.tensor(0x7F7F, dtype=torch.int16).view(torch.bfloat16)  # largest finite bf16
    H = torch.full((P + T, I), float(pattern), dtype=torch.bfloat16, device=gpu)
    GU = torch.full((P + T, 2 * I), float(pattern), dtype=torch.bfloat16, device=gpu)
    Y = torch.full((P + T, I), float(pattern), dtype=torch.bfloat16, device=gpu)
    st = ops._stream(dx.device)
    ops.check(ops.lib.q38moe_gate_up_save(ops._ptr(dx), ops._ptr(dwgu), ops._ptr(perm_s), ops._ptr(tiles_s),
                                          ops._ptr(tc_s), ops._ptr(H), ops._ptr(GU), T, h, E, k, I, st),
              "q38moe_gate_up_save")
    ops.check(ops.lib.q38moe_down_kn(ops._ptr(A), ops._ptr(dwdn), ops._ptr(tiles_s), ops._ptr(tc_s), ops._ptr(Y),
                                     T, h, I, E, k, st), "q38moe_down_kn")
    torch.cuda.synchronize()
    assert int(tc_s.item()) > int(tc.item())  # the table does hold shared-expert tiles
    assert torch.equal(perm_s[:P], perm[:P])
    assert torch.equal(H[:P], H_ref) and torch.equal(GU[:P], GU_ref) and torch.equal(Y[:P], Y_ref)
    for nm, t in (("H", H), ("GU", GU), ("Y", Y)):
        assert bool((t[P:] == pattern).all()), f"{nm}: rows past T*k were written"


@pytest.mark.parametrize("name,T,drop", [("c2", 2048, 0), ("c1", 700, 40)])
def test_pair_dots_rows_fused(gpu, name, T, drop):
    """pair_dots with top_k_weights writes the same routed-row gradient as gather_rows and the same
    weight gradient as pair_dots alone, bit for bit (same roundings, one pass)."""
    from q38.hip import ops
    wl, x, idx, w, wgu, wdn, dout = _inputs(name, T, drop)
    E, k = wl.experts, wl.topk
    di, dw_, dd = idx.to(gpu), w.to(gpu), dout.to(gpu)
    counts, starts, perm, inv, _, _ = ops.permute(di, ops.histogram(di, E), E)
    Y = torch.randn(T * k, wl.hidden, device=gpu).to(torch.bfloat16)
    dw_alone = ops.pair_dots(dd, Y, inv, di, E)
    dw_fused, d_raw = ops.pair_dots(dd, Y, inv, di, E, w=dw_)
    rows = ops.gather_rows(dd, perm, starts, counts, k, w=dw_)
    torch.cuda.synchronize()
    filled = int(counts.sum())
    assert torch.equal(dw_alone, dw_fused)
    assert torch.equal(d_raw[:filled], rows[:filled])


@pytest.mark.parametrize("main", [1.0, 0.0], ids=["main+aux", "aux-only"])
def test_dropin_block_trains_under_autocast(gpu, main):
    """The drop-in Qwen3_8MoeSparseMoeBlock trained as the reference trainer runs it: fp32
    parameters under bf16 autocast, a forward hook on ``gate`` recording the router logits
    (q38/train.py:228-233) and the load-balancing loss over them (modeling:1289-1355) added to the
    main loss (main = 0: the router's gradient from the auxiliary loss alone). Every gradient, of x
    and of the eight parameters, within relative L2 2.5e-2 of fp32 CPU autograd of the reference's
    op sequence (modeling:805-835) and loss on the same selections (the GPU's top-k sets, so that
    bf16 near-ties do not pick other experts)."""
    from q38 import prefill as P
    from q38 import workloads
    from q38.models.qwen3_8_moe import Qwen3_8MoeSparseMoeBlock, new_config
    F = torch.nn.functional
    wl = workloads.get("c2")
    T, h, E, k = 2048, wl.hidden, wl.experts, wl.topk
    x, params, _ = workloads.make(wl, tokens=T)
    x = x.float()
    params = {n: t.float() for n, t in params.items()}
    dout = torch.randn(T, h, generator=torch.Generator().manual_seed(21)) * 0.05
    cfg = new_config(hidden_size=h, num_experts=E, num_experts_per_tok=k, moe_intermediate_size=wl.inter,
                     shared_expert_intermediate_size=wl.shared_inter)
    block = Qwen3_8MoeSparseMoeBlock(cfg)
    block.load_state_dict(params, strict=True)
    block = block.to(gpu)
    seen = []
    block.gate.register_forward_hook(lambda m, a, o: seen.append(o))
    xg = x.to(gpu).requires_grad_(True)
    with torch.autocast("cuda", dtype=torch.bfloat16):
        out = block(xg.view(1, T, h))
        aux = P.load_balancing_loss((seen[0][0],), E, k)
    loss = main * (out.view(T, h).float() * dout.to(gpu)).sum() + aux
    loss.backward()
    torch.cuda.synchronize()
    assert len(seen) == 1 and seen[0][0].dtype == torch.bfloat16 and out.dtype == torch.float32
    idx = seen[0][2].cpu()

    leaves = {n: t.clone().requires_grad_(True) for n, t in params.items()}
    xc = x.clone().requires_grad_(True)
    logits = F.linear(xc, leaves["gate.weight"])
    probs = torch.softmax(logits, dim=-1, dtype=torch.float)
    top = probs.gather(1, idx)
    top = top / top.sum(dim=-1, keepdim=True)
    routed = orc.experts_eager(xc, idx, top, leaves["experts.gate_up_proj"], leaves["experts.down_proj"])
    sh = F.linear(F.silu(F.linear(xc, leaves["shared_expert.gate_proj.weight"]))
                  * F.linear(xc, leaves["shared_expert.up_proj.weight"]), leaves["shared_expert.down_proj.weight"])
    ref = routed + torch.sigmoid(F.linear(xc, leaves["shared_expert_gate.weight"])) * sh
    # The loss's expert counts (its own top-k of the softmax, not differentiated) as the GPU run
    # chose them: a few bf16 near-ties moving a count shift the small per-expert deviations the
    # auxiliary gradient is made of.
    chosen = torch.topk(torch.softmax(seen[0][0].detach().float(), dim=-1), k, dim=-1).indices
    counts = torch.bincount(chosen.reshape(-1), minlength=E).float().cpu()
    ref_aux = E * ((counts / T) * (torch.softmax(logits, dim=-1).sum(0) / T)).sum()
    ref_loss = main * (ref * dout).sum() + ref_aux
    ref_loss.backward()
    assert abs(float(aux.detach()) - float(ref_aux.detach())) < 1e-3
    pairs = [("x", xg.grad, xc.grad)] + [(n, p.grad, leaves[n].grad) for n, p in block.named_parameters()]
    if main == 0.0:
        pairs = [q for q in pairs if q[0] in ("x", "gate.weight")]
    for n, got, want in pairs:
        assert got is not None and got.dtype == torch.float32, n
        r = _rel(got, want)
        print(f"{n}: rel L2 {r:.2e}")
        assert r <= REL, f"{n}: rel L2 {r:.3e}"
