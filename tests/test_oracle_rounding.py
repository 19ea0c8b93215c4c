"""The bf16 checker's rounding points, pinned against a library routine.

Every bf16 GPU test holds the HIP experts to ``oracle.experts_grouped`` at the ulp level, so that
function's rounding points (bf16 gate, bf16 up, bf16 silu(gate), bf16 product, bf16 down product,
bf16 weighted row, one rounding of the fp32 k-sum; inference.py:90-96, 122-130, 199) must be the
reference's. ``oracle.experts_grouped_mm`` is transformers' ``grouped_mm_experts_forward`` bit for
bit (test_oracle.py::test_experts_grouped_mm_is_transformers); run in bf16, torch's bf16 kernels
round at exactly the points listed above, with the fp32 accumulation order of its GEMMs the only
difference. So the two must agree within one bf16 ulp except where an accumulation-order
difference flips an intermediate rounding, and dropping any one rounding from ``experts_grouped``
(the planted mistakes, ``_skip_rounding``) must break that agreement.

Measured on these inputs: 0.06 % (c2) / 0.01 % (c1) of outputs more than 1 ulp apart and 0.2 % /
0.05 % differing at all; with one rounding dropped, 17-30 % more than 1 ulp apart.
"""
import pytest
import torch

from _util import bf16_ulp_diff
from oracle import moe_oracle as orc

# Accumulation-order flips allowed between the two rounding-identical bf16 computations.
FLIP_FRAC_OVER_1ULP = 1e-3
FLIP_FRAC_ANY = 5e-3
# A dropped rounding point moves far more outputs than that.
PLANTED_MIN_FRAC_OVER_1ULP = 5e-2


def _case(name, T):
    from q38 import workloads
    wl = workloads.get(name)
    x, p, _ = workloads.make(wl, tokens=T)
    _, _, idx, w = orc.router(x, p["gate.weight"], wl.topk)
    return x, idx, w, p["experts.gate_up_proj"], p["experts.down_proj"]


_CASES = {"c2": 512, "c1": 1024}


@pytest.fixture(scope="module", params=sorted(_CASES))
def case(request):
    x, idx, w, wgu, wdn = _case(request.param, _CASES[request.param])
    ref = orc.experts_grouped_mm(x, idx, w, wgu, wdn)
    assert ref.dtype == torch.bfloat16
    return x, idx, w, wgu, wdn, ref


def test_grouped_matches_grouped_mm_to_one_ulp(case):
    x, idx, w, wgu, wdn, ref = case
    out, _, _ = orc.experts_grouped(x, idx, w, wgu, wdn)
    d = bf16_ulp_diff(out, ref)
    over1 = float((d > 1).float().mean())
    anyd = float((d > 0).float().mean())
    print(f"> 1 ulp: {over1:.2e}, differing: {anyd:.2e}")
    assert over1 <= FLIP_FRAC_OVER_1ULP and anyd <= FLIP_FRAC_ANY


@pytest.mark.parametrize("dropped", ["g", "u", "silu", "down"])
def test_dropped_rounding_is_detected(case, dropped):
    x, idx, w, wgu, wdn, ref = case
    out, _, _ = orc.experts_grouped(x, idx, w, wgu, wdn, _skip_rounding=(dropped,))
    over1 = float((bf16_ulp_diff(out, ref) > 1).float().mean())
    print(f"rounding of {dropped} dropped: {over1:.3f} of outputs > 1 ulp")
    assert over1 > PLANTED_MIN_FRAC_OVER_1ULP
