"""GPU parity of the fp8 expert path (R14; this repository's definition, include/q38moe.h):
e4m3 quantisation bit-exact against the CPU quantiser (pinned in test_oracle_fp8.py), the e4m3
grouped GEMMs and the fp8 block against the CPU fake-quant oracle on identical inputs.

Tolerances (the fp8 tolerance the benchmark set asks this repository to state): quantisation
bit-exact (codes and fp32 scales). GEMM stages vs the fake-quant oracle on identical e4m3 inputs:
relative L2 <= 1e-2, max-abs <= 2e-2 scaled by max(1, max|ref|), and beyond 3 bf16 ulps only on
values below 2^-5 of the largest; they differ only in fp32 accumulation order. Block output vs the
fake-quant oracle: max-abs <= 5e-2, relative L2 <= 1e-2 (a bf16 rounding flip in H can move an
e4m3 code of the second quantisation by one step, 1/8 relative, so the bf16 max-abs bar of 2e-2 is
widened). Against the bf16 block the fp8 block is reported, with relative L2 <= 8e-2 for the e4m3
quantisation error itself.
"""
import numpy as np
import pytest
import torch

from _util import assert_bf16_close, bf16_ulp_diff
from oracle import moe_oracle as orc

pytestmark = pytest.mark.gpu


def _ops():
    from q38.hip import ops
    return ops


def _assert_ulps(actual, expected, what):
    """Elementwise: differences beyond 3 bf16 ulps only where the value is small. e4m3 operands
    make near-total cancellation common, and there a different fp32 summation order moves the
    bf16 result by many ulps of a tiny value."""
    a, b = actual.cpu(), expected.cpu()
    sig = b.float().abs() > 2.0 ** -5 * b.float().abs().max()
    frac = float((bf16_ulp_diff(a, b)[sig] > 3).float().mean())
    assert frac < 1e-3, f"{what}: {frac:.2e} of the significant values differ by more than 3 ulps"


@pytest.mark.parametrize("R,C", [(257, 64), (1000, 512), (333, 1024), (64, 2048), (17, 4096), (40, 320)])
def test_quantize_rows_bitexact(gpu, R, C):
    ops = _ops()
    g = torch.Generator().manual_seed(R * 7 + C)
    mag = torch.logspace(-6, 4, R)[:, None]
    x = (torch.randn(R, C, generator=g) * mag).to(torch.bfloat16)
    x[0] = 0                                    # zero row: scale 0, all codes 0
    x[1, :] = 1e-30                             # amax far below the smallest e4m3 subnormal times 448
    x[2, ::3] = 0
    q, s = ops.quantize_rows(x.to(gpu))
    torch.cuda.synchronize()
    rq, rs = orc.quant_e4m3_rows(x)
    assert torch.equal(s.cpu(), rs), float((s.cpu() - rs).abs().max())
    bad = q.cpu() != rq
    assert not bad.any(), f"{int(bad.sum())} codes differ, e.g. x={x[bad][:4].tolist()}"


def test_quantize_rows_nan_row(gpu):
    ops = _ops()
    x = torch.randn(8, 128).to(torch.bfloat16)
    x[5, 7] = float("nan")
    q, s = ops.quantize_rows(x.to(gpu))
    torch.cuda.synchronize()
    assert torch.isnan(s.cpu()[5]) and torch.isfinite(s.cpu()[[0, 1, 2, 3, 4, 6, 7]]).all()
    assert torch.isnan(orc.e4m3_value(q.cpu()[5])).all()
    rq, rs = orc.quant_e4m3_rows(x)
    assert torch.equal(q.cpu()[[0, 1, 2, 3, 4, 6, 7]], rq[[0, 1, 2, 3, 4, 6, 7]])


def _setup(name, T, scale_x=1.0, **shape):
    from q38 import workloads
    wl = workloads.get(name, **shape)
    x, params, bias = workloads.make(wl, tokens=T)
    return wl, x, params, bias


@pytest.mark.parametrize("name,T,kind", [("c1", 1024, "persistent"), ("c4", 2048, "persistent"),
                                         ("c4", 1024, "persistent"), ("c4", 1, "small"), ("c4", 16, "small"),
                                         ("c4", 272, "small"), ("c4", 273, "persistent")])
def test_fp8_gemm_stages(gpu, name, T, kind):
    """gate/up and down on e4m3 vs the fake-quant oracle, stage by stage on identical inputs, on both
    tilings (small e4m3 tiles up to configuration 4's threshold, T = 272; h = 256 has none). At
    configuration 4 the persistent gate/up is the four-wave kernel: T = 2048 (about 72 row tiles of
    more than 128 rows, 288 units) and T = 1024 (rows per expert near 80: units of at most 128 rows)
    both end in a partial round that runs as column halves."""
    _check_fp8_stages(gpu, name, T, kind)


@pytest.mark.parametrize("h,I,T", [(1024, 128, 1500), (1024, 384, 700), (1536, 256, 3000)])
def test_fp8_gemm_stages_four_wave_shapes(gpu, h, I, T):
    """The four-wave e4m3 gate/up at the edges of its rule: h = 1024 (eight 128-byte slices, the
    first and the last iteration only, no steady one), one column tile (I = 128), three (I = 384),
    and h = 1536 (twelve slices: one steady iteration)."""
    _check_fp8_stages(gpu, "c4", T, "persistent", hidden=h, inter=I, shared_inter=I)


def _check_fp8_stages(gpu, name, T, kind, **shape):
    ops = _ops()
    wl, x, params, _ = _setup(name, T, **shape)
    k, E = wl.topk, wl.experts
    assert ops.gemm_tiling(T, wl.hidden, E, k, wl.inter, T, fp8=True) == kind
    d = {n: p.to(gpu) for n, p in params.items()}
    _, _, ridx, rw = orc.router(x, params["gate.weight"], k)
    gate_logit = orc.bf16(orc._f(x) @ orc._f(params["shared_expert_gate.weight"]).reshape(-1))
    wq_ref = orc.quant_weights_fp8(params)
    ref_out, ref = orc.experts_fp8(x, ridx, rw, wq_ref, k, gate_logit)
    # Weights and tokens quantised on the GPU: bit-exact to the oracle's.
    wq = ops.quantize_weights_fp8(d)
    xq, sx = ops.quantize_rows(x.to(gpu))
    torch.cuda.synchronize()
    for n, (q, s) in wq.items():
        assert torch.equal(q.cpu(), wq_ref[n][0]) and torch.equal(s.cpu(), wq_ref[n][1]), n
    assert torch.equal(xq.cpu(), ref["xq"]) and torch.equal(sx.cpu(), ref["sx"])
    didx = ridx.to(gpu)
    hist = ops.histogram(didx, E)
    counts, starts, perm, inv, tiles, tcount = ops.permute(didx, hist, E, shared_rows=T)
    row_scale = torch.cat([sx[perm.long() // k], sx])
    H = ops.gate_up_fp8(xq, row_scale, wq, perm, tiles, tcount, k, shared_rows=T)
    torch.cuda.synchronize()
    # Intermediates: the bf16 bar scaled to their magnitude (H and Y reach |x| > 1 at h = 2048).
    assert_bf16_close(H.cpu(), ref["H"], max_abs=2e-2 * max(1.0, float(ref["H"].float().abs().max())),
                      what=f"{name} H (e4m3 gate/up + SwiGLU)")
    _assert_ulps(H, ref["H"], f"{name} H")
    # Down on the oracle's own e4m3 SwiGLU rows isolates the down GEMM.
    Y = ops.down_fp8(ref["Hq"].to(gpu), ref["sH"].to(gpu), wq, tiles, tcount, T, k, shared_rows=T)
    torch.cuda.synchronize()
    assert_bf16_close(Y.cpu(), ref["Y"], max_abs=2e-2 * max(1.0, float(ref["Y"].float().abs().max())),
                      what=f"{name} Y (e4m3 down)")
    _assert_ulps(Y, ref["Y"], f"{name} Y")
    # The GPU's H, quantised on the GPU: bit-exact to the oracle quantiser of that H.
    Hq, sH = ops.quantize_rows(H)
    torch.cuda.synchronize()
    rHq, rsH = orc.quant_e4m3_rows(H.cpu())
    assert torch.equal(Hq.cpu(), rHq) and torch.equal(sH.cpu(), rsH)


@pytest.mark.parametrize("T", [2048, 20000])
def test_block_fp8_equals_staged_pipeline(gpu, T):
    """The fp8 block equals bit for bit the same pipeline staged through the separate entry points
    (route, quantize_rows of x, permute, gate_up_fp8, quantize_rows of H, down_fp8, combine): the
    block adds no arithmetic of its own. T = 20000 runs the router's 128-token blocks (the last one
    ragged)."""
    ops = _ops()
    wl, x, params, _ = _setup("c4", T)
    k, E = wl.topk, wl.experts
    d = {n: p.to(gpu) for n, p in params.items()}
    wq = ops.quantize_weights_fp8(d)
    dx = x.to(gpu)
    out, _, idx, w = ops.block_forward_fp8(dx, d["gate.weight"], wq, d["shared_expert_gate.weight"], k,
                                           return_router=True)
    _, idx2, w2, gate, hist = ops.route(dx, d["gate.weight"], k, w_shared_gate=d["shared_expert_gate.weight"],
                                        want_hist=True)
    xq, sx = ops.quantize_rows(dx)
    counts, starts, perm, inv, tiles, tc = ops.permute(idx2, hist, E, shared_rows=T)
    H = ops.gate_up_fp8(xq, torch.cat([sx[perm.long() // k], sx]), wq, perm, tiles, tc, k, shared_rows=T)
    Hq, sH = ops.quantize_rows(H)
    Y = ops.down_fp8(Hq, sH, wq, tiles, tc, T, k, shared_rows=T)
    out2 = ops.combine(Y[:T * k], inv, w2, E, idx=idx2, shared_out=Y[T * k:], shared_gate_logit=gate)
    torch.cuda.synchronize()
    assert torch.equal(idx.cpu(), idx2.cpu()) and torch.equal(w.cpu(), w2.cpu())
    assert torch.equal(out.cpu(), out2.cpu())


@pytest.mark.parametrize("name,T", [("c1", 2048), ("c4", 2048), ("c4", 999), ("c4", 1), ("c4", 100)])
def test_block_forward_fp8(gpu, name, T):
    """Whole fp8 block vs the fake-quant oracle on the GPU's own routing (bit-exact routing)."""
    ops = _ops()
    wl, x, params, _ = _setup(name, T)
    d = {n: p.to(gpu) for n, p in params.items()}
    wq = ops.quantize_weights_fp8(d)
    out, logits, idx, w = ops.block_forward_fp8(x.to(gpu), d["gate.weight"], wq, d["shared_expert_gate.weight"],
                                                wl.topk, return_router=True)
    torch.cuda.synchronize()
    _, _, sidx, sw = orc.router(None, None, wl.topk, logits=logits.cpu())
    assert torch.equal(idx.cpu().long(), sidx)
    gate_logit = orc.bf16(orc._f(x) @ orc._f(params["shared_expert_gate.weight"]).reshape(-1))
    ref_out, _ = orc.experts_fp8(x, idx.cpu().long(), w.cpu(), orc.quant_weights_fp8(params), wl.topk, gate_logit)
    mx, r = assert_bf16_close(out.cpu(), ref_out, max_abs=5e-2, what=f"{name} fp8 block vs fake-quant oracle")
    bf_out, _ = orc.block(x, params, wl.topk)
    rel_bf16 = float((out.cpu().float() - bf_out.float()).norm() / bf_out.float().norm())
    print(f"{name} T={T}: vs fake-quant max-abs {mx:.3e} rel {r:.3e}; vs bf16 block rel {rel_bf16:.3e}")
    assert rel_bf16 < 8e-2


@pytest.mark.parametrize("shape", [
    dict(experts=8, topk=2, hidden=128, inter=64, T=100),
    dict(experts=1, topk=1, hidden=64, inter=64, T=37),
    dict(experts=64, topk=8, hidden=256, inter=128, T=300),
    dict(experts=16, topk=4, hidden=512, inter=192, T=1),
], ids=lambda s: "E{experts}k{topk}h{hidden}I{inter}T{T}".format(**s))
def test_block_forward_fp8_edge_shapes(gpu, shape):
    """fp8 block off the benchmark shapes: one or two K slices (down on I = 64 is a single e4m3
    slice), few experts, k = 1 and 8, a single token."""
    from q38 import workloads
    ops = _ops()
    shape = dict(shape)
    T = shape.pop("T")
    wl = workloads.get("c4", shared_inter=shape["inter"], **shape)
    x, params, _ = workloads.make(wl, tokens=T)
    d = {n: p.to(gpu) for n, p in params.items()}
    wq = ops.quantize_weights_fp8(d)
    out, logits, idx, w = ops.block_forward_fp8(x.to(gpu), d["gate.weight"], wq, d["shared_expert_gate.weight"],
                                                wl.topk, return_router=True)
    torch.cuda.synchronize()
    _, _, sidx, _ = orc.router(None, None, wl.topk, logits=logits.cpu())
    assert torch.equal(idx.cpu().long(), sidx)
    gate_logit = orc.bf16(orc._f(x) @ orc._f(params["shared_expert_gate.weight"]).reshape(-1))
    ref_out, _ = orc.experts_fp8(x, idx.cpu().long(), w.cpu(), orc.quant_weights_fp8(params), wl.topk, gate_logit)
    assert_bf16_close(out.cpu(), ref_out, max_abs=5e-2, what=f"fp8 edge block {shape}")


def test_block_forward_fp8_full_c4(gpu):
    """Configuration 4 at its full size (T = 32768, h = 2048, I = 512): routing bit-exact against the
    CPU oracle on the GPU's logits for every token; outputs finite and bit-identical on a second
    forward; and, since tokens are independent through the block (per-token x scales, per-row H
    scales, per-token k-sum), the fake-quant oracle run on a seeded sample of 256 tokens with their
    GPU routing reproduces those tokens' outputs within the bar of the smaller fp8 block tests."""
    ops = _ops()
    wl, x, params, _ = _setup("c4", None)
    T = wl.tokens
    assert T == 32768 and x.shape == (T, 2048)
    d = {n: p.to(gpu) for n, p in params.items()}
    wq = ops.quantize_weights_fp8(d)
    xd = x.to(gpu)
    args = (xd, d["gate.weight"], wq, d["shared_expert_gate.weight"], wl.topk)
    out, logits, idx, w = ops.block_forward_fp8(*args, return_router=True)
    out2 = ops.block_forward_fp8(*args)
    torch.cuda.synchronize()
    assert torch.equal(out, out2), "fp8 block not deterministic at full size"
    assert bool(torch.isfinite(out).all())
    _, _, sidx, sw = orc.router(None, None, wl.topk, logits=logits.cpu())
    assert torch.equal(idx.cpu().long(), sidx)
    assert torch.equal(w.cpu(), sw)
    sel = torch.from_numpy(np.sort(np.random.RandomState(4).choice(T, 256, replace=False)))
    xs = x[sel]
    gate_logit = orc.bf16(orc._f(xs) @ orc._f(params["shared_expert_gate.weight"]).reshape(-1))
    ref, _ = orc.experts_fp8(xs, sidx[sel], sw[sel], orc.quant_weights_fp8(params), wl.topk, gate_logit)
    mx, r = assert_bf16_close(out.cpu()[sel], ref, max_abs=5e-2, what="c4 T=32768 fp8 block, 256 sampled tokens")
    print(f"c4 T={T}: sampled tokens vs fake-quant max-abs {mx:.3e} rel {r:.3e}")
