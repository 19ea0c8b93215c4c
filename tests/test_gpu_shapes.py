"""GPU parity of the whole bf16 MoE block (modeling:816-835) over a seeded sweep of shapes across
the C ABI's domain: E in [1, 64], k in [1, min(8, E)], h, I and Is any multiples of 64 (so
hidden sizes and intermediate sizes that are not multiples of the GEMM tiles' 128 or 256
columns, separate and fused shared experts), token counts on both sides of the GEMM tiling rule,
with and without a routing-skew bias.

Bars (as tests/test_gpu_block.py): routing indices and weights bit-exact against the oracle's
router on the GPU's logits; the block output within the bf16 tolerance of tests/_util.py of the
oracle's block (the reference op sequence, fp32 products with the reference's bf16 rounding
points) on that routing.
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
