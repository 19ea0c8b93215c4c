"""GPU parity of the whole bf16 MoE block (modeling:816-835) over a seeded sweep of shapes across
the C ABI's domain: E in [1, 64], k in [1, min(8, E)], h, I and Is any multiples of 64 (so
hidden sizes and intermediate sizes that are not multiples of the GEMM tiles' 128 or 256
columns, separate and fused shared experts), token counts on both sides of the GEMM tiling rule,
with and without a routing-skew bias.

Bars (as tests/test_gpu_block.py): routing indices and weights bit-exact against the oracle's
router on the GPU's logits; the block output within the bf16 tolerance of tests/_util.py of the
oracle's block (the reference op sequence, fp32 products with the reference's bf16 rounding
points) on that routing. The same sweep, on fewer shapes, runs the fp32 block (bars of
tests/test_gpu_fp32.py), the fp8 block (bars of tests/test_gpu_fp8.py) and the differentiable
experts' backward (bars of tests/test_gpu_backward.py).
"""
import numpy as np
import pytest
import torch

from _util import assert_bf16_close
from oracle import moe_oracle as orc

pytestmark = pytest.mark.gpu

_EXPERTS = (1, 2, 3, 7, 16, 33, 63, 64)


def _shapes(n=32, seed=2026):
    """Every fourth pair of shapes takes h and I from the sizes the small-tile kernels serve
    (128 .. 2048), so that the small side of the tiling rule runs too."""
    rs = np.random.RandomState(seed)
    out = []
    for i in range(n):
        E = int(rs.choice(_EXPERTS))
        k = int(rs.randint(1, min(8, E) + 1))
        if i % 4 < 2:
            h = 64 * int(rs.randint(1, 25))
            I = 64 * int(rs.randint(1, 13))
        else:
            h = int(rs.choice((128, 256, 512, 1024, 2048)))
            I = int(rs.choice((128, 256, 512)))
        Is = I if rs.rand() < 0.5 else 64 * int(rs.randint(1, 13))
        # Small-tile rule: T*k + shared rows <= 32 per group; draw T on either side of it.
        lim = max(1, 32 * (E + 1) // (k + 1))
        T = int(rs.randint(1, lim + 1)) if i % 2 == 0 else int(rs.randint(lim + 1, lim + 1500))
        skew = bool(rs.rand() < 0.3)
        out.append((E, k, h, I, Is, T, skew))
    return out


@pytest.mark.parametrize("E,k,h,I,Is,T,skew", _shapes())
def test_block_shape_sweep(gpu, E, k, h, I, Is, T, skew):
    from q38 import workloads
    from q38.hip import ops
    base = "c3" if skew else "c2"
    wl = workloads.get(base, experts=E, topk=k, hidden=h, inter=I, shared_inter=Is)
    x, p, bias = workloads.make(wl, tokens=T)
    assert (bias is not None) == skew
    kind = ops.gemm_tiling(T, h, E, k, I, T if Is == I else 0)
    d = {n: t.to(gpu) for n, t in p.items()}
    tag = f"E={E} k={k} h={h} I={I} Is={Is} T={T} skew={skew} tiling={kind}"
    print(tag, flush=True)
    out, logits, idx, w = ops.block_forward(
        x.to(gpu), d["gate.weight"], d["experts.gate_up_proj"], d["experts.down_proj"],
        d["shared_expert.gate_proj.weight"], d["shared_expert.up_proj.weight"],
        d["shared_expert.down_proj.weight"], d["shared_expert_gate.weight"], k,
        return_router=True, logit_bias=None if bias is None else bias.to(gpu))
    torch.cuda.synchronize()
    _, _, sidx, srw = orc.router(None, None, k, logit_bias=bias, logits=logits.cpu())
    assert torch.equal(idx.cpu().long(), sidx), tag
    assert torch.equal(w.cpu(), srw), tag
    ref = orc.reference_block_forward(x, p, k, routing=(sidx, srw))
    assert_bf16_close(out.cpu(), ref, what=tag)


def _small_shapes(n, seed, hmax=24, imax=12, tmax=1500):
    rs = np.random.RandomState(seed)
    out = []
    for _ in range(n):
        E = int(rs.choice(_EXPERTS))
        k = int(rs.randint(1, min(8, E) + 1))
        h = 64 * int(rs.randint(1, hmax + 1))
        I = 64 * int(rs.randint(1, imax + 1))
        Is = I if rs.rand() < 0.5 else 64 * int(rs.randint(1, imax + 1))
        T = int(rs.randint(1, tmax + 1))
        out.append((E, k, h, I, Is, T, bool(rs.rand() < 0.3)))
    return out


_BLOCK_NAMES = ("gate.weight", "experts.gate_up_proj", "experts.down_proj", "shared_expert.gate_proj.weight",
                "shared_expert.up_proj.weight", "shared_expert.down_proj.weight", "shared_expert_gate.weight")


@pytest.mark.parametrize("E,k,h,I,Is,T,skew", _small_shapes(10, 77, hmax=12, imax=6, tmax=1200))
def test_block_shape_sweep_fp32(gpu, E, k, h, I, Is, T, skew):
    """fp32 block: logits within fp32 accumulation of the float64 product, routing bit-exact on the
    GPU's logits. Output against the reference op sequence in float64 on that routing: at these
    sizes (K up to 768) the CPU's own fp32 op sequence leaves the reference's elementwise bar
    (rtol 1e-4, atol 2e-8) on near-zero outputs, so the bar is that one widened by three times the
    CPU fp32 sequence's largest deviation from float64, and the relative L2 error at most twice the
    CPU fp32 sequence's."""
    from q38 import workloads
    from q38.hip import ops
    wl = workloads.get("c3" if skew else "c2", experts=E, topk=k, hidden=h, inter=I, shared_inter=Is)
    x, p, bias = workloads.make(wl, tokens=T, dtype=torch.float32)
    tag = f"fp32 E={E} k={k} h={h} I={I} Is={Is} T={T} skew={skew}"
    print(tag, flush=True)
    out, logits, idx, w = ops.block_forward(x.to(gpu), *[p[n].to(gpu) for n in _BLOCK_NAMES], k,
                                            return_router=True,
                                            logit_bias=None if bias is None else bias.to(gpu))
    torch.cuda.synchronize()
    assert out.dtype == torch.float32 and w.dtype == torch.float32, tag
    ref_logits = x.double() @ p["gate.weight"].double().T
    mag = x.double().abs() @ p["gate.weight"].double().abs().T
    assert bool(((logits.cpu().double() - ref_logits).abs() <= mag * 2.0 ** -20).all()), tag
    _, _, ridx, rw = orc.router(None, None, k, logit_bias=bias, logits=logits.cpu())
    assert torch.equal(idx.cpu().long(), ridx) and torch.equal(w.cpu(), rw), tag
    ref32 = orc.reference_block_forward(x, p, k, routing=(ridx, rw)).double()
    ref64 = orc.reference_block_forward(x.double(), {n: t.double() for n, t in p.items()}, k,
                                        routing=(ridx, rw.double()))
    got = out.cpu().double()
    cpu_dev = float((ref32 - ref64).abs().max())
    err = (got - ref64).abs()
    bound = 2e-8 + 1e-4 * ref64.abs() + 3 * cpu_dev
    rel_gpu = float((got - ref64).norm() / ref64.norm())
    rel_cpu = float((ref32 - ref64).norm() / ref64.norm())
    print(f"{tag}: max-abs {float(err.max()):.3e} (cpu fp32 {cpu_dev:.3e}), rel {rel_gpu:.3e} (cpu fp32 {rel_cpu:.3e})")
    assert not bool((err > bound).any()), f"{tag}: {int((err > bound).sum())} elements outside the bar"
    assert rel_gpu <= 2 * rel_cpu + 1e-12, f"{tag}: rel {rel_gpu:.3e} vs cpu fp32 {rel_cpu:.3e}"


@pytest.mark.parametrize("E,k,h,I,Is,T,skew", [s[:4] + (s[3],) + s[5:]
                                                for s in _small_shapes(8, 88, hmax=16, imax=8, tmax=1000)])
def test_block_shape_sweep_fp8(gpu, E, k, h, I, Is, T, skew):
    """fp8 block (e4m3 expert weights and expert inputs; its shared expert has the experts' width,
    Is == I): routing bit-exact on the GPU's logits, output within 5e-2 max-abs / 1e-2 relative L2
    of the fake-quant oracle on that routing."""
    from q38 import workloads
    from q38.hip import ops
    wl = workloads.get("c4", experts=E, topk=k, hidden=h, inter=I, shared_inter=Is)
    x, params, _ = workloads.make(wl, tokens=T)
    tag = f"fp8 E={E} k={k} h={h} I={I} Is={Is} T={T}"
    print(tag, flush=True)
    d = {n: t.to(gpu) for n, t in params.items()}
    wq = ops.quantize_weights_fp8(d)
    out, logits, idx, w = ops.block_forward_fp8(x.to(gpu), d["gate.weight"], wq, d["shared_expert_gate.weight"],
                                                k, return_router=True)
    torch.cuda.synchronize()
    _, _, sidx, _ = orc.router(None, None, k, logits=logits.cpu())
    assert torch.equal(idx.cpu().long(), sidx), tag
    gate_logit = orc.bf16(orc._f(x) @ orc._f(params["shared_expert_gate.weight"]).reshape(-1))
    ref_out, _ = orc.experts_fp8(x, idx.cpu().long(), w.cpu(), orc.quant_weights_fp8(params), k, gate_logit)
    assert_bf16_close(out.cpu(), ref_out, max_abs=5e-2, what=tag)


@pytest.mark.parametrize("E,k,h,I,Is,T,skew", _small_shapes(8, 99, hmax=16, imax=8, tmax=1200))
def test_experts_backward_shape_sweep(gpu, E, k, h, I, Is, T, skew):
    """Differentiable routed experts: forward within the bf16 tolerance, every gradient within
    relative L2 2.5e-2 of fp32 CPU autograd of the eager experts and within twice the eager bf16
    autograd's error + 2e-3; a few pairs routed outside [0, E) get zero weight gradient."""
    from q38 import workloads
    from q38.hip import autograd
    wl = workloads.get("c3" if skew else "c2", experts=E, topk=k, hidden=h, inter=I, shared_inter=Is)
    x, p, bias = workloads.make(wl, tokens=T)
    _, _, idx, w = orc.router(x, p["gate.weight"], k, logit_bias=bias)
    drop = T * k // 20
    if drop:
        sel = torch.randperm(idx.numel(), generator=torch.Generator().manual_seed(T))[:drop]
        idx.view(-1)[sel] = E
    dout = (torch.randn(T, h, generator=torch.Generator().manual_seed(h + T)) * 0.05).to(torch.bfloat16)
    wgu, wdn = p["experts.gate_up_proj"], p["experts.down_proj"]
    tag = f"backward E={E} k={k} h={h} I={I} T={T} skew={skew} dropped={drop}"
    print(tag, flush=True)

    def cpu_grads(dtype):
        leaves = [t.detach().to(dtype).requires_grad_(True) for t in (x, w, wgu, wdn)]
        o = orc.experts_eager(leaves[0], idx, *leaves[1:])
        o.backward(dout.to(dtype))
        return o.detach().float(), [t.grad.float() for t in leaves]

    def rel(a, b):
        a, b = a.detach().float().cpu(), b.detach().float().cpu()
        return float((a - b).norm() / b.norm().clamp_min(1e-30))

    ref_out, ref_g = cpu_grads(torch.float32)
    _, eager_g = cpu_grads(torch.bfloat16)
    leaves = [t.to(gpu).requires_grad_(True) for t in (x, w, wgu, wdn)]
    out = autograd.experts(leaves[0], idx.to(gpu), *leaves[1:])
    out.backward(dout.to(gpu))
    torch.cuda.synchronize()
    assert_bf16_close(out, ref_out, what=tag + " forward")
    for nm, leaf, r, e in zip(("x", "top_k_weights", "gate_up_proj", "down_proj"), leaves, ref_g, eager_g):
        g = leaf.grad
        assert g is not None and g.dtype == torch.bfloat16 and g.shape == leaf.shape, nm
        err, eager_err = rel(g, r), rel(e, r)
        assert err <= 2.5e-2, f"{tag} d{nm}: rel {err:.3e} vs fp32 autograd"
        assert err <= 2 * eager_err + 2e-3, f"{tag} d{nm}: rel {err:.3e}, eager bf16 {eager_err:.3e}"
    if drop:
        assert bool((leaves[1].grad[idx.to(gpu) == E] == 0).all()), tag
