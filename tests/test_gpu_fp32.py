"""GPU parity of the fp32 path (configuration 1 and fp32 models): the reference computes fp32 models
with true fp32 products and no intermediate roundings (q38/inference.py:54-57, 172; the eager
module in the parameters' dtype, modeling:769-793), and holds fp32 experts to rtol 1e-4,
atol 2e-8 (scripts/check_q38_kernels.py:26).

Bars: routing indices and fp32 weights bit-exact against the CPU oracle on the same fp32 logits
(the kernel computes torch's CPU softmax bit for bit); router logits within fp32 accumulation of
the CPU's; expert and block outputs within the reference's fp32 bar (torch.allclose with rtol 1e-4,
atol 2e-8) of the reference op sequence run in fp32 torch on the CPU on the same routing; the
intermediate stages (H, Y) within that bar plus an fp32 accumulation allowance.
"""
import numpy as np
import pytest
import torch
import torch.nn.functional as F

from _util import assert_fp32_close as _assert_fp32_close
from oracle import moe_oracle as orc

pytestmark = pytest.mark.gpu


def _c1(T, seed_x=1234, **over):
    from q38 import workloads
    wl = workloads.get("c1", **over)
    x, params, bias = workloads.make(wl, tokens=T, dtype=torch.float32, seed_x=seed_x)
    return wl, x, params, bias


@pytest.mark.parametrize("T,E,k,kind", [(4096, 64, 5, "randn"), (999, 64, 8, "randn"), (1000, 8, 3, "randn"),
                                        (2048, 64, 5, "near"), (513, 17, 4, "near")])
def test_route_from_logits_fp32(gpu, T, E, k, kind):
    """fp32 logits (not bf16 values): indices and fp32 weights bit-exact. "near" rows put several
    logits a few fp32 ulps apart, where exp and the 1/sum scaling merge neighbours."""
    from q38.hip import ops
    rng = np.random.RandomState(T + E)
    z = (rng.randn(T, E) * 0.5).astype(np.float32)
    if kind == "near":
        base = z[:, :1].copy()
        steps = rng.randint(0, 4, size=(T, E)).astype(np.uint32)
        z = (base.view(np.uint32) + steps).view(np.float32)
        z[:, E // 2:] -= 1.0
    logits = torch.from_numpy(z)
    idx, w, hist = ops.route_from_logits(logits.to(gpu), k, want_hist=True)
    torch.cuda.synchronize()
    _, _, ridx, rw = orc.router(None, None, k, logits=logits)
    assert w.dtype == torch.float32 and rw.dtype == torch.float32
    assert torch.equal(idx.cpu().long(), ridx)
    assert torch.equal(w.cpu(), rw)


@pytest.mark.parametrize("T", [2048, 999])
def test_experts_forward_fp32(gpu, T):
    """Routed experts in fp32 (the ExpertsInterface on an fp32 model) against the eager module's
    fp32 forward and transformers' grouped_mm on the CPU, same routing."""
    from q38.hip import ops
    wl, x, p, _ = _c1(T)
    _, _, idx, w = orc.router(x, p["gate.weight"], wl.topk, dtype=torch.float32)
    out = ops.experts_forward(x.to(gpu), idx.to(gpu), w.to(gpu), p["experts.gate_up_proj"].to(gpu),
                              p["experts.down_proj"].to(gpu))
    torch.cuda.synchronize()
    eager = orc.experts_eager(x, idx, w, p["experts.gate_up_proj"], p["experts.down_proj"])
    _assert_fp32_close(out, eager, f"fp32 experts T={T} vs eager")
    gmm = orc.experts_grouped_mm(x, idx, w, p["experts.gate_up_proj"], p["experts.down_proj"])
    _assert_fp32_close(out, gmm, f"fp32 experts T={T} vs grouped_mm")


def test_gemm_stages_fp32(gpu):
    """gate/up + SwiGLU, down and the shared rows alone, each against fp32 torch on the CPU on the
    GPU's own inputs (H of the GPU feeds the down check). Intermediates get the fp32 bar plus an
    accumulation allowance of 2^-20 times the magnitude of their sums: where g, u or a down row
    cancel, two fp32 summation orders differ by more than rtol 1e-4 of the small result."""
    from q38.hip import ops
    wl, x, p, _ = _c1(700)
    T, k, E, I = 700, wl.topk, wl.experts, wl.inter
    _, _, idx, w = orc.router(x, p["gate.weight"], k, dtype=torch.float32)
    d = {n: t.to(gpu) for n, t in p.items()}
    hist = ops.histogram(idx.to(gpu), E)
    counts, starts, perm, inv, tiles, tc = ops.permute(idx.to(gpu), hist, E, shared_rows=T)
    sh = (d["shared_expert.gate_proj.weight"], d["shared_expert.up_proj.weight"])
    H = ops.gate_up(x.to(gpu), d["experts.gate_up_proj"], perm, tiles, tc, k, shared_weights=sh, shared_rows=T)
    Y = ops.down(H, d["experts.down_proj"], tiles, tc, T, k, w_shared_down=d["shared_expert.down_proj.weight"],
                 shared_rows=T)
    torch.cuda.synchronize()
    perm_c = perm.cpu().long()
    ids = idx.reshape(-1)[perm_c]
    tok = perm_c // k
    g = torch.empty(T * k, I)
    u = torch.empty(T * k, I)
    mg = torch.empty(T * k, I)
    mu = torch.empty(T * k, I)
    for e in range(E):
        sel = ids == e
        gu = x[tok[sel]] @ p["experts.gate_up_proj"][e].T
        mgu = x[tok[sel]].abs() @ p["experts.gate_up_proj"][e].abs().T
        g[sel], u[sel] = gu[:, :I], gu[:, I:]
        mg[sel], mu[sel] = mgu[:, :I], mgu[:, I:]
    wsg, wsu = p["shared_expert.gate_proj.weight"], p["shared_expert.up_proj.weight"]
    g, u = torch.cat([g, x @ wsg.T]), torch.cat([u, x @ wsu.T])
    mg, mu = torch.cat([mg, x.abs() @ wsg.abs().T]), torch.cat([mu, x.abs() @ wsu.abs().T])
    refH = F.silu(g) * u
    # |d silu / dg| <= 1.1: an error in g moves H by at most 1.1 |u| times it
    _assert_fp32_close(H, refH, "fp32 gate/up H", allowance=2.0 ** -20 * (1.1 * mg * u.abs() + F.silu(g).abs() * mu))
    Hc = H.cpu()
    refY = torch.empty(T * k + T, wl.hidden)
    magY = torch.empty(T * k + T, wl.hidden)
    for e in range(E):
        sel = torch.nonzero(ids == e).flatten()
        refY[sel] = Hc[sel] @ p["experts.down_proj"][e].T
        magY[sel] = Hc[sel].abs() @ p["experts.down_proj"][e].abs().T
    refY[T * k:] = Hc[T * k:] @ p["shared_expert.down_proj.weight"].T
    magY[T * k:] = Hc[T * k:].abs() @ p["shared_expert.down_proj.weight"].abs().T
    _assert_fp32_close(Y, refY, "fp32 down Y", allowance=2.0 ** -20 * magY)


@pytest.mark.parametrize("T,Is,skew", [(2048, None, False), (777, 128, True)])
def test_block_forward_fp32(gpu, T, Is, skew):
    """The whole block in fp32 (configuration 1 at its own precision): logits within fp32
    accumulation of the CPU's, routing bit-exact on the GPU's logits, output within the reference's
    fp32 bar of the reference op sequence in fp32 on the same routing."""
    from q38.hip import ops
    over = {} if Is is None else {"shared_inter": Is}
    wl, x, p, _ = _c1(T, **over)
    bias = None
    if skew:
        bias = torch.from_numpy(-0.24 * np.log(np.random.RandomState(7).permutation(wl.experts) + 1.0)).float()
    names = ("gate.weight", "experts.gate_up_proj", "experts.down_proj", "shared_expert.gate_proj.weight",
             "shared_expert.up_proj.weight", "shared_expert.down_proj.weight", "shared_expert_gate.weight")
    d = [p[n].to(gpu) for n in names]
    out, logits, idx, w = ops.block_forward(x.to(gpu), *d, wl.topk, return_router=True,
                                            logit_bias=None if bias is None else bias.to(gpu))
    torch.cuda.synchronize()
    assert out.dtype == torch.float32 and w.dtype == torch.float32
    ref_logits = x.double() @ p["gate.weight"].double().T
    mag = x.double().abs() @ p["gate.weight"].double().abs().T
    assert bool(((logits.cpu().double() - ref_logits).abs() <= mag * 2.0 ** -20).all()), "router logits"
    _, _, ridx, rw = orc.router(None, None, wl.topk, logit_bias=bias, logits=logits.cpu())
    assert torch.equal(idx.cpu().long(), ridx) and torch.equal(w.cpu(), rw)
    ref = orc.reference_block_forward(x, p, wl.topk, routing=(ridx, rw))
    _assert_fp32_close(out, ref, f"fp32 block T={T} Is={wl.shared_inter}")
    # the no-allocation entry point computes the same in fp32
    out2 = ops.block_forward_noalloc(x.to(gpu), *d, wl.topk, logit_bias=None if bias is None else bias.to(gpu))
    torch.cuda.synchronize()
    assert torch.equal(out2, out)
