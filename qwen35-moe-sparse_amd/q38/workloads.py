"""Seeded synthetic workloads of the Q38 MoE-layer benchmark configurations.

No checkpoints or datasets are used: weights follow the reference's initialisation
(modeling_qwen3_8_moe.py:956-960 and the HF default normal(0, initializer_range=0.02) for the
nn.Linear layers), activations are N(0, 1).

Generator: ``numpy.random.RandomState`` (the legacy stream, frozen by NumPy's compatibility
policy) draws float64 normals; they are scaled, rounded to float32 by NumPy, and rounded to bf16
by torch (round-to-nearest-even). Weights come from one stream (seed ``seed_w``) in the fixed
name order of ``PARAM_ORDER``; activations from a second stream (seed ``seed_x``).
"""
from dataclasses import dataclass, field, replace

import numpy as np
import torch

# State-dict names of one Qwen3_8MoeSparseMoeBlock (modeling:816-822), in generation order.
PARAM_ORDER = (
    "gate.weight",
    "experts.gate_up_proj",
    "experts.down_proj",
    "shared_expert.gate_proj.weight",
    "shared_expert.up_proj.weight",
    "shared_expert.down_proj.weight",
    "shared_expert_gate.weight",
)

INIT_STD = 0.02


@dataclass(frozen=True)
class Workload:
    name: str
    hidden: int
    experts: int
    topk: int
    inter: int
    shared_inter: int
    batch: int
    seq: int
    dtype: str = "bf16"
    zipf_s: float = 0.0      # > 0: add the routing-skew logit bias (configuration 3)
    zipf_alpha: float = 0.0  # bias scale, calibrated for a ~20x max/min expert load
    zipf_seed: int = 7
    notes: str = field(default="", compare=False)

    @property
    def tokens(self):
        return self.batch * self.seq

    def shapes(self):
        E, h, I, Is = self.experts, self.hidden, self.inter, self.shared_inter
        return {
            "gate.weight": (E, h),
            "experts.gate_up_proj": (E, 2 * I, h),
            "experts.down_proj": (E, h, I),
            "shared_expert.gate_proj.weight": (Is, h),
            "shared_expert.up_proj.weight": (Is, h),
            "shared_expert.down_proj.weight": (h, Is),
            "shared_expert_gate.weight": (1, h),
        }

    def flops(self):
        """Algorithmic FLOPs of one block forward (real pair rows only; q38/flops.py:25,38-40)."""
        T, h, E, k, I, Is = self.tokens, self.hidden, self.experts, self.topk, self.inter, self.shared_inter
        P = T * k
        gate_up = 2 * P * h * 2 * I
        down = 2 * P * I * h
        shared = 6 * T * h * Is
        router = 2 * T * h * E
        sgate = 2 * T * h
        return dict(gate_up=gate_up, down=down, experts=gate_up + down, shared=shared, router=router,
                    shared_gate=sgate, block=gate_up + down + shared + router + sgate)


WORKLOADS = {
    # Reference CPU-runnable case (fp32 on CPU). The GPU path computes it in bf16.
    "c1": Workload("c1", hidden=256, experts=64, topk=5, inter=64, shared_inter=64, batch=1, seq=2048,
                   dtype="fp32"),
    # Headline configuration: 4 x 4096 packed tokens, bf16.
    "c2": Workload("c2", hidden=1024, experts=64, topk=5, inter=256, shared_inter=256, batch=4, seq=4096),
    # Routing skew: C2 plus a per-expert Zipf(1.2) logit bias. alpha = 0.24 is calibrated on these
    # seeded inputs for a ~20x span of expert loads: max 7620 / min 369 pairs (20.7x).
    "c3": Workload("c3", hidden=1024, experts=64, topk=5, inter=256, shared_inter=256, batch=4, seq=4096,
                   zipf_s=1.2, zipf_alpha=0.24),
    # FP8 expert path: bf16 router and activations, e4m3 expert weights (per-output-channel
    # scales) and per-token e4m3 expert inputs (q38moe_block_forward_fp8).
    "c4": Workload("c4", hidden=2048, experts=64, topk=5, inter=512, shared_inter=512, batch=8, seq=4096,
                   dtype="fp8"),
}


def get(name, **overrides):
    wl = WORKLOADS[name]
    return replace(wl, **overrides) if overrides else wl


def weights_np(wl, seed_w=0):
    """float32 numpy weights by state-dict name, drawn in PARAM_ORDER from one RandomState."""
    rs = np.random.RandomState(seed_w)
    out = {}
    for name in PARAM_ORDER:
        shape = wl.shapes()[name]
        out[name] = (rs.standard_normal(size=shape) * INIT_STD).astype(np.float32)
    return out


def input_np(wl, seed_x=1234, tokens=None):
    rs = np.random.RandomState(seed_x)
    T = wl.tokens if tokens is None else tokens
    return rs.standard_normal(size=(T, wl.hidden)).astype(np.float32)


def zipf_bias_np(wl):
    """Routing-skew logit bias: seeded rank permutation r_e in 1..E, bias_e = -alpha * s * ln(r_e).

    Zipf(s) assigns weight r^-s to rank r; adding its log (scaled by alpha) to every token's
    logits skews the softmax top-k toward low ranks. No reference function exists for this.
    """
    if wl.zipf_s <= 0:
        return None
    ranks = np.random.RandomState(wl.zipf_seed).permutation(wl.experts) + 1
    return (-wl.zipf_alpha * wl.zipf_s * np.log(ranks.astype(np.float64))).astype(np.float32)


def to_torch(arrs, device="cpu", dtype=torch.bfloat16):
    """float32 numpy -> torch (RNE to dtype)."""
    if isinstance(arrs, dict):
        return {k: torch.from_numpy(v).to(device=device, dtype=dtype) for k, v in arrs.items()}
    return torch.from_numpy(arrs).to(device=device, dtype=dtype)


def make(wl, device="cpu", dtype=torch.bfloat16, seed_w=0, seed_x=1234, tokens=None):
    """(x [T,h], params by name, logit_bias fp32 [E] or None) as torch tensors."""
    params = to_torch(weights_np(wl, seed_w), device, dtype)
    x = to_torch(input_np(wl, seed_x, tokens), device, dtype)
    bias = zipf_bias_np(wl)
    if bias is not None:
        bias = torch.from_numpy(bias).to(device)
    return x, params, bias
