"""GPU parity of the grouped GEMMs, combine, shared expert and the whole MoE block (R0, R5-R9)
against the CPU oracle (fp32 matmuls with the reference's explicit bf16 rounding points).

Tolerance (bf16): max-abs <= 2e-2 and relative L2 <= 1e-2 (tests/_util.py).
"""
import pytest
import torch

from _util import assert_bf16_close, assert_gemm_bf16_rounding, bf16_ulp_diff
from oracle import moe_oracle as orc

pytestmark = pytest.mark.gpu


def _ops():
    from q38.hip import ops
    return ops


def _setup(name, T=None, **over):
    from q38 import workloads
    wl = workloads.get(name, **over) if over else workloads.get(name)
    x, params, bias = workloads.make(wl, tokens=T)
    return wl, x, params, bias


@pytest.mark.parametrize("name,T", [("c1", 2048), ("c2", 4096)])
def test_gate_up_down_stages(gpu, name, T):
    """Each stage against the oracle on identical inputs (oracle routing, GPU permutation)."""
    ops = _ops()
    wl, x, params, _ = _setup(name, T)
    k = wl.topk
    _, _, ridx, rw = orc.router(x, params["gate.weight"], k)
    ref_out, ref_y, ref_H, ref_Y = orc.experts_grouped(x, ridx, rw, params["experts.gate_up_proj"],
                                                       params["experts.down_proj"], return_sorted=True)
    dx, didx, dw = x.to(gpu), ridx.to(gpu), rw.to(gpu)
    wgu, wdn = params["experts.gate_up_proj"].to(gpu), params["experts.down_proj"].to(gpu)
    hist = ops.histogram(didx, wl.experts)
    counts, starts, perm, inv, tiles, tcount = ops.permute(didx, hist, wl.experts)
    H = ops.gate_up(dx, wgu, perm, tiles, tcount, k)
    torch.cuda.synchronize()
    # H in sorted order: bf16 results of identical roundings; fp32 accumulation order differs.
    assert_bf16_close(H.cpu(), ref_H, what="H (gate/up + SwiGLU)")
    assert float((bf16_ulp_diff(H.cpu(), ref_H) > 1).float().mean()) < 1e-3
    Y = ops.down(H, wdn, tiles, tcount, T, k)
    torch.cuda.synchronize()
    assert_bf16_close(Y.cpu(), ref_Y, what="Y (down projection, sorted rows)")
    # Down alone on the oracle's H: isolates the down GEMM.
    Y2 = ops.down(ref_H.to(gpu), wdn, tiles, tcount, T, k)
    torch.cuda.synchronize()
    assert float((bf16_ulp_diff(Y2.cpu(), ref_Y) > 1).float().mean()) < 1e-3
    # Combine on the oracle's sorted rows: weight, k-sum and rounding exactly as the oracle.
    out_exact = ops.combine(ref_Y.to(gpu), inv, dw, wl.experts)
    torch.cuda.synchronize()
    assert float((bf16_ulp_diff(out_exact.cpu(), ref_out) > 1).float().mean()) < 1e-3
    out = ops.combine(Y, inv, dw, wl.experts)
    torch.cuda.synchronize()
    assert_bf16_close(out.cpu(), ref_out, what="routed experts output")


def test_fused_shared_rows(gpu):
    """Routed and shared-expert rows in one grouped launch equal the separate computations."""
    ops = _ops()
    wl, x, params, _ = _setup("c2", 1500)
    T, k = x.shape[0], wl.topk
    _, _, ridx, rw = orc.router(x, params["gate.weight"], k)
    d = {n: p.to(gpu) for n, p in params.items()}
    didx = ridx.to(gpu)
    hist = ops.histogram(didx, wl.experts)
    counts, starts, perm, inv, tiles, tcount = ops.permute(didx, hist, wl.experts, shared_rows=T)
    H = ops.gate_up(x.to(gpu), d["experts.gate_up_proj"], perm, tiles, tcount, k,
                    shared_weights=(d["shared_expert.gate_proj.weight"], d["shared_expert.up_proj.weight"]),
                    shared_rows=T)
    Y = ops.down(H, d["experts.down_proj"], tiles, tcount, T, k, w_shared_down=d["shared_expert.down_proj.weight"],
                 shared_rows=T)
    torch.cuda.synchronize()
    ref_sh = orc.shared_expert(x, params["shared_expert.gate_proj.weight"], params["shared_expert.up_proj.weight"],
                               params["shared_expert.down_proj.weight"])
    assert_bf16_close(Y[T * k:].cpu(), ref_sh, what="shared rows of the fused launch")
    _, _, ref_H, ref_Y = orc.experts_grouped(x, ridx, rw, params["experts.gate_up_proj"],
                                             params["experts.down_proj"], return_sorted=True)
    assert_bf16_close(Y[:T * k].cpu(), ref_Y, what="routed rows of the fused launch")


@pytest.mark.parametrize("name,T", [("c1", 2048), ("c2", 4096), ("c2", 333)])
def test_shared_expert(gpu, name, T):
    ops = _ops()
    wl, x, params, _ = _setup(name, T)
    wg, wu, wd = (params[f"shared_expert.{n}_proj.weight"] for n in ("gate", "up", "down"))
    ref = orc.shared_expert(x, wg, wu, wd)
    out = ops.shared_expert(x.to(gpu), wg.to(gpu), wu.to(gpu), wd.to(gpu))
    torch.cuda.synchronize()
    assert_bf16_close(out.cpu(), ref, what="shared expert")


@pytest.mark.parametrize("name,T", [("c1", 2048), ("c2", 16384), ("c3", 16384), ("c2", 1000)])
def test_block_forward(gpu, name, T):
    """Whole block vs the oracle; routing compared on the GPU's own logits (bit-exact)."""
    ops = _ops()
    wl, x, params, bias = _setup(name, T)
    d = {n: p.to(gpu) for n, p in params.items()}
    out, logits, idx, w = ops.block_forward(
        x.to(gpu), d["gate.weight"], d["experts.gate_up_proj"], d["experts.down_proj"],
        d["shared_expert.gate_proj.weight"], d["shared_expert.up_proj.weight"], d["shared_expert.down_proj.weight"],
        d["shared_expert_gate.weight"], wl.topk, logit_bias=None if bias is None else bias.to(gpu),
        return_router=True)
    torch.cuda.synchronize()
    ref_out, inter = orc.block(x, params, wl.topk, logit_bias=bias)
    assert_gemm_bf16_rounding(logits, x, params["gate.weight"], "router logits")
    _, _, sidx, _ = orc.router(None, None, wl.topk, logit_bias=bias, logits=logits.cpu())
    assert torch.equal(idx.cpu().long(), sidx)
    mx, r = assert_bf16_close(out.cpu(), ref_out, what=f"{name} block output")
    print(f"{name} T={T}: max-abs {mx:.3e} rel {r:.3e}")


@pytest.mark.parametrize("name,T", [("c2", 16384), ("c3", 16384), ("c2", 20000), ("c2", 300)])
def test_block_forward_equals_staged_pipeline(gpu, name, T):
    """The fused block equals bit for bit the same pipeline staged through the separate entry points
    (route, permute with the shared rows, gate_up with the fused shared rows, down, combine with the
    gated shared row): the block adds no arithmetic of its own, whatever the tiling (T = 300: small
    tiles) or the router's block size (T = 20000: 128-token blocks)."""
    ops = _ops()
    wl, x, params, bias = _setup(name, T)
    k, E = wl.topk, wl.experts
    d = {n: p.to(gpu) for n, p in params.items()}
    dx, db = x.to(gpu), (None if bias is None else bias.to(gpu))
    out, _, idx, w = ops.block_forward(
        dx, d["gate.weight"], d["experts.gate_up_proj"], d["experts.down_proj"],
        d["shared_expert.gate_proj.weight"], d["shared_expert.up_proj.weight"], d["shared_expert.down_proj.weight"],
        d["shared_expert_gate.weight"], k, logit_bias=db, return_router=True)
    _, idx2, w2, gate, hist = ops.route(dx, d["gate.weight"], k, w_shared_gate=d["shared_expert_gate.weight"],
                                        logit_bias=db, want_hist=True)
    counts, starts, perm, inv, tiles, tc = ops.permute(idx2, hist, E, shared_rows=T)
    H = ops.gate_up(dx, d["experts.gate_up_proj"], perm, tiles, tc, k,
                    shared_weights=(d["shared_expert.gate_proj.weight"], d["shared_expert.up_proj.weight"]),
                    shared_rows=T)
    Y = ops.down(H, d["experts.down_proj"], tiles, tc, T, k, w_shared_down=d["shared_expert.down_proj.weight"],
                 shared_rows=T)
    out2 = ops.combine(Y[:T * k], inv, w2, E, idx=idx2, shared_out=Y[T * k:], shared_gate_logit=gate)
    torch.cuda.synchronize()
    assert torch.equal(idx.cpu(), idx2.cpu()) and torch.equal(w.cpu(), w2.cpu())
    assert torch.equal(out.cpu(), out2.cpu())


@pytest.mark.parametrize("name,T", [("c1", 3001), ("c2", 16384)])
def test_block_forward_all_tokens_tie(gpu, name, T):
    """Router rows 32..63 copy rows 0..31, so every logit has an equal twin and every token's top-k
    goes through the libstdc++ replay inside the block forward: indices bit-exact, weights within
    1 bf16 ulp, block output within tolerance."""
    ops = _ops()
    wl, x, params, bias = _setup(name, T)
    params = dict(params)
    wr = params["gate.weight"].clone()
    wr[32:] = wr[:32]
    params["gate.weight"] = wr
    d = {n: p.to(gpu) for n, p in params.items()}
    out, logits, idx, w = ops.block_forward(
        x.to(gpu), d["gate.weight"], d["experts.gate_up_proj"], d["experts.down_proj"],
        d["shared_expert.gate_proj.weight"], d["shared_expert.up_proj.weight"], d["shared_expert.down_proj.weight"],
        d["shared_expert_gate.weight"], wl.topk, return_router=True)
    torch.cuda.synchronize()
    lg = logits.cpu()
    assert torch.equal(lg[:, 32:], lg[:, :32])
    _, _, sidx, sw = orc.router(None, None, wl.topk, logits=lg)
    assert torch.equal(idx.cpu().long(), sidx)
    assert int(bf16_ulp_diff(w.cpu(), sw).max()) <= 1
    # A 1-ulp difference between CPU and GPU logits can break a tie the other way, so the reference
    # runs the oracle's experts on the routing of the GPU's own logits.
    routed, _, _ = orc.experts_grouped(x, sidx, sw, params["experts.gate_up_proj"], params["experts.down_proj"])
    sh = orc.shared_expert(x, params["shared_expert.gate_proj.weight"], params["shared_expert.up_proj.weight"],
                           params["shared_expert.down_proj.weight"])
    gl = orc.bf16(orc._f(x) @ orc._f(params["shared_expert_gate.weight"]).reshape(-1))
    ref = orc.bf16(orc._f(routed) + orc._f(orc.bf16(orc._f(orc.bf16(torch.sigmoid(orc._f(gl))))[:, None] * orc._f(sh))))
    assert_bf16_close(out.cpu(), ref, what=f"{name} all-tie block output")


def test_experts_forward_int64(gpu):
    """ExpertsInterface entry (int64 top_k_index, as torch.topk returns) vs the oracle."""
    ops = _ops()
    wl, x, params, _ = _setup("c2", 2048)
    _, _, ridx, rw = orc.router(x, params["gate.weight"], wl.topk)
    ref, _, _ = orc.experts_grouped(x, ridx, rw, params["experts.gate_up_proj"], params["experts.down_proj"])
    out = ops.experts_forward(x.to(gpu), ridx.to(gpu), rw.to(gpu), params["experts.gate_up_proj"].to(gpu),
                              params["experts.down_proj"].to(gpu))
    torch.cuda.synchronize()
    assert_bf16_close(out.cpu(), ref, what="experts_forward")


def test_dropin_module_and_registry(gpu):
    """Drop-in modules load a reference-named state dict; the registered experts implementation
    and the fused block agree with the oracle."""
    from q38.inference import register_experts_implementation
    from q38.models.qwen3_8_moe import Qwen3_8MoeSparseMoeBlock, new_config
    wl, x, params, _ = _setup("c1", 512)
    cfg = new_config(hidden_size=wl.hidden, num_experts=wl.experts, num_experts_per_tok=wl.topk,
                     moe_intermediate_size=wl.inter, shared_expert_intermediate_size=wl.shared_inter)
    block = Qwen3_8MoeSparseMoeBlock(cfg).to(torch.bfloat16)
    missing, unexpected = block.load_state_dict(params, strict=True)
    assert not missing and not unexpected
    block = block.to(gpu)
    ref_out, inter = orc.block(x, params, wl.topk)
    with torch.inference_mode():
        out = block(x.view(1, -1, wl.hidden).to(gpu))
        logits, scores, sel = block.gate(x.to(gpu))
        assert sel.dtype == torch.int64
        assert register_experts_implementation() == "q38_hip"
        routed = block.experts(x.to(gpu), sel, scores)
        hooked = []
        h = block.gate.register_forward_hook(lambda m, i, o: hooked.append(o[0]))
        out2 = block(x.view(1, -1, wl.hidden).to(gpu))
        h.remove()
    torch.cuda.synchronize()
    assert_bf16_close(out.view(-1, wl.hidden).cpu(), ref_out, what="drop-in block")
    assert_bf16_close(out2.view(-1, wl.hidden).cpu(), ref_out, what="drop-in block (hooked router)")
    assert len(hooked) == 1 and hooked[0].shape == (512, wl.experts)
    ref_routed, _, _ = orc.experts_grouped(x, sel.cpu(), scores.cpu(), params["experts.gate_up_proj"],
                                           params["experts.down_proj"])
    assert_bf16_close(routed.cpu(), ref_routed, what="drop-in experts")
    # Training in fp32 without autocast: the HIP experts backward takes bf16 only.
    with pytest.raises(TypeError, match="bf16"):
        block.float().requires_grad_(True)
        block(x.view(1, -1, wl.hidden).to(gpu).float())


# Shapes off the benchmark configs: few or single experts, k = 1 (torch's partial_sort path when
# k*64 <= E), k = 8, the smallest hidden/intermediate sizes (one or two K slices), ragged and single
# tokens, and a shared expert narrower than the routed ones (separate dense shared GEMMs).
EDGE_SHAPES = [
    dict(experts=8, topk=2, hidden=128, inter=64, shared_inter=64, T=100),
    dict(experts=1, topk=1, hidden=64, inter=64, shared_inter=64, T=37),
    dict(experts=64, topk=1, hidden=256, inter=64, shared_inter=64, T=1),
    dict(experts=64, topk=8, hidden=256, inter=128, shared_inter=64, T=300),
    dict(experts=16, topk=4, hidden=512, inter=192, shared_inter=192, T=2000),
]


@pytest.mark.parametrize("shape", EDGE_SHAPES, ids=lambda s: "E{experts}k{topk}h{hidden}I{inter}Is{shared_inter}T{T}".format(**s))
def test_block_forward_edge_shapes(gpu, shape):
    ops = _ops()
    shape = dict(shape)
    T = shape.pop("T")
    wl, x, params, _ = _setup("c2", T, **shape)
    d = {n: p.to(gpu) for n, p in params.items()}
    out, logits, idx, w = ops.block_forward(
        x.to(gpu), d["gate.weight"], d["experts.gate_up_proj"], d["experts.down_proj"],
        d["shared_expert.gate_proj.weight"], d["shared_expert.up_proj.weight"], d["shared_expert.down_proj.weight"],
        d["shared_expert_gate.weight"], wl.topk, return_router=True)
    torch.cuda.synchronize()
    _, _, sidx, _ = orc.router(None, None, wl.topk, logits=logits.cpu())
    assert torch.equal(idx.cpu().long(), sidx)
    ref_out, _ = orc.block(x, params, wl.topk)
    # The oracle block routes on CPU-computed logits; re-run its experts on the GPU's routing.
    _, _, _, rw = orc.router(None, None, wl.topk, logits=logits.cpu())
    routed, _, _ = orc.experts_grouped(x, sidx, rw, params["experts.gate_up_proj"], params["experts.down_proj"])
    sh = orc.shared_expert(x, params["shared_expert.gate_proj.weight"], params["shared_expert.up_proj.weight"],
                           params["shared_expert.down_proj.weight"])
    gl = orc.bf16(orc._f(x) @ orc._f(params["shared_expert_gate.weight"]).reshape(-1))
    ref = orc.bf16(orc._f(routed) + orc._f(orc.bf16(orc._f(orc.bf16(torch.sigmoid(orc._f(gl))))[:, None] * orc._f(sh))))
    assert_bf16_close(out.cpu(), ref, what=f"edge block {shape}")


@pytest.mark.parametrize("name", ["c2", "c3"])
def test_block_forward_deterministic(gpu, name):
    """Two forwards of the same inputs are bit-identical: no floating-point atomics anywhere in the
    path (histograms are integer, the k-sum runs in a fixed order), so outputs, logits, indices and
    weights repeat exactly."""
    ops = _ops()
    wl, x, params, bias = _setup(name, 4096)
    d = {n: p.to(gpu) for n, p in params.items()}
    args = (x.to(gpu), d["gate.weight"], d["experts.gate_up_proj"], d["experts.down_proj"],
            d["shared_expert.gate_proj.weight"], d["shared_expert.up_proj.weight"],
            d["shared_expert.down_proj.weight"], d["shared_expert_gate.weight"], wl.topk)
    kw = dict(logit_bias=None if bias is None else bias.to(gpu), return_router=True)
    first = ops.block_forward(*args, **kw)
    second = ops.block_forward(*args, **kw)
    torch.cuda.synchronize()
    for a, b in zip(first, second):
        assert torch.equal(a, b)


@pytest.mark.parametrize("name,T", [("c2", 16384), ("c3", 16384), ("c2", 20000), ("c2", 300)])
def test_block_forward_router_outputs_change_nothing(gpu, name, T):
    """The two calls the packed prefill makes of one block, ``hip_moe_block_forward_with_router``
    (return_router=True) and ``block(x)`` (return_router=False), over one reused workspace that
    holds another call's data or a byte pattern: out bit-identical in every call; idx, w and the
    logits equal the standalone router's. T = 20000 takes 128-token router blocks, T = 300 the
    small GEMM tiles."""
    ops = _ops()
    wl, x, params, bias = _setup(name, T)
    d = {n: p.to(gpu) for n, p in params.items()}
    dx = x.to(gpu)
    args = (dx, d["gate.weight"], d["experts.gate_up_proj"], d["experts.down_proj"],
            d["shared_expert.gate_proj.weight"], d["shared_expert.up_proj.weight"],
            d["shared_expert.down_proj.weight"], d["shared_expert_gate.weight"], wl.topk)
    lb = None if bias is None else bias.to(gpu)
    nbytes = ops.block_workspace_bytes(T, wl.hidden, wl.experts, wl.topk, wl.inter, wl.shared_inter)
    ws = torch.empty(nbytes, dtype=torch.uint8, device=gpu)
    runs = []
    for fill, want in ((0xFF, False), (0x00, True), (0x7F, False), (None, True), (None, False), (0xFF, True)):
        if fill is not None:
            ws.fill_(fill)  # bf16 0xFFFF is a NaN, 0x7F7F the largest finite value
        res = ops.block_forward(*args, logit_bias=lb, return_router=want, workspace=ws)
        runs.append(res if want else (res,))
    logits, idx, w, _, _ = ops.route(dx, d["gate.weight"], wl.topk, w_shared_gate=d["shared_expert_gate.weight"],
                                     logit_bias=lb, want_logits=True)
    torch.cuda.synchronize()
    out0 = runs[0][0]
    assert torch.isfinite(out0).all()
    for i, r in enumerate(runs):
        assert torch.equal(r[0], out0), f"call {i}: out differs"
        if len(r) == 4:
            assert torch.equal(r[1], logits), f"call {i}: logits differ from the router's"
            assert torch.equal(r[2], idx), f"call {i}: idx differs from the router's"
            assert torch.equal(r[3], w), f"call {i}: w differs from the router's"


def test_dropin_block_with_and_without_router_logits(gpu):
    """The drop-in module's two prefill calls on its cached workspace give the same bits."""
    from q38.inference import hip_moe_block_forward_with_router
    from q38.models.qwen3_8_moe import Qwen3_8MoeSparseMoeBlock, new_config
    wl, x, params, _ = _setup("c2", 4096)
    cfg = new_config(hidden_size=wl.hidden, num_experts=wl.experts, num_experts_per_tok=wl.topk,
                     moe_intermediate_size=wl.inter, shared_expert_intermediate_size=wl.shared_inter)
    block = Qwen3_8MoeSparseMoeBlock(cfg).to(torch.bfloat16)
    block.load_state_dict(params, strict=True)
    block = block.to(gpu)
    xs = x.view(2, -1, wl.hidden).to(gpu)
    with torch.inference_mode():
        plain = block(xs)
        with_router, logits = hip_moe_block_forward_with_router(block, xs)
        again = block(xs)
    torch.cuda.synchronize()
    assert torch.equal(plain, with_router) and torch.equal(plain, again)
    assert logits.shape == (4096, wl.experts)
