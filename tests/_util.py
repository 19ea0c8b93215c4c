"""Shared helpers for the parity tests."""
import torch

# Block/experts output tolerance of the bf16 path: max |a-b| <= 2e-2 and
# ||a-b||_2 / ||b||_2 <= 1e-2 (relative, over the whole tensor).
BF16_MAX_ABS = 2e-2
BF16_REL = 1e-2


def assert_bf16_close(actual, expected, max_abs=BF16_MAX_ABS, rel=BF16_REL, what="output"):
    a = actual.detach().float().cpu()
    b = expected.detach().float().cpu()
    assert a.shape == b.shape, f"{what}: shape {tuple(a.shape)} vs {tuple(b.shape)}"
    assert torch.isfinite(a).all(), f"{what}: non-finite values"
    diff = (a - b).abs()
    mx = float(diff.max()) if diff.numel() else 0.0
    r = float(diff.norm() / b.norm().clamp_min(1e-30)) if diff.numel() else 0.0
    assert mx <= max_abs and r <= rel, f"{what}: max-abs {mx:.3e} (<= {max_abs}), rel {r:.3e} (<= {rel})"
    return mx, r


# fp32 path: the reference's fp32 experts bar (scripts/check_q38_kernels.py:26).
FP32_RTOL, FP32_ATOL = 1e-4, 2e-8


def assert_fp32_close(actual, expected, what, allowance=None):
    """torch.allclose(actual, expected, rtol=1e-4, atol=2e-8) elementwise, optionally widened by an
    fp32 accumulation allowance (for intermediates whose sums cancel)."""
    a = actual.detach().cpu()
    b = expected.detach().cpu()
    assert a.dtype == torch.float32 and a.shape == b.shape, what
    err = (a - b).abs()
    bound = FP32_ATOL + FP32_RTOL * b.abs()
    if allowance is not None:
        bound = bound + allowance
    bad = err > bound
    worst = float((err / bound).max()) if err.numel() else 0.0
    print(f"{what}: max-abs {float(err.max()):.3e}, worst err/bound {worst:.3f}")
    assert not bool(bad.any()), \
        f"{what}: {int(bad.sum())} of {bad.numel()} outside rtol {FP32_RTOL}, atol {FP32_ATOL}"


def bf16_ulp_diff(a, b):
    """|ordinal(a) - ordinal(b)| of bf16 values, elementwise (0 = identical bits)."""
    def ordinal(t):
        u = t.detach().cpu().contiguous().view(torch.int16).to(torch.int32) & 0xFFFF
        return torch.where(u >= 0x8000, 0x8000 - u, u)
    return (ordinal(a) - ordinal(b)).abs()


def assert_gemm_bf16_rounding(actual, x, w, what="logits"):
    """A bf16 GEMM output with fp32 accumulation: |actual - exact| <= 1 bf16 ulp of the exact value
    plus an fp32 accumulation allowance of 2^-20 * sum_i |x_i w_i| (needed where the exact value is
    near zero, where a bf16 ulp is smaller than fp32 rounding of the partial sums)."""
    a = actual.detach().float().cpu().double()
    xd, wd = x.double(), w.double().reshape(-1, x.shape[1])
    exact = xd @ wd.T
    mag = xd.abs() @ wd.abs().T
    e = exact.abs().clamp_min(1e-38)
    ulp = torch.pow(2.0, torch.floor(torch.log2(e)) - 7)
    bound = ulp + mag * 2.0 ** -20
    err = (a.reshape(exact.shape) - exact).abs()
    bad = err > bound
    assert not bool(bad.any()), f"{what}: {int(bad.sum())} values off; worst excess {float((err - bound).max()):.3e}"


def collision_logits(rows, E=64, k=5, seed=0):
    """bf16 router logits whose distinct values collide in the fp32 softmax: a few logits at 1.0
    (fewer than k, so the k-th pick falls among the rest), several distinct tiny logits in
    [2^-34, 2^-25] with random signs (x - max rounds them to one fp32 value, so their
    probabilities tie although their logits differ), and -3 elsewhere; random positions."""
    import numpy as np
    rng = np.random.RandomState(seed)
    z = np.full((rows, E), -3.0)
    for r in range(rows):
        pos = rng.permutation(E)
        n_big = rng.randint(1, k)
        n_tiny = rng.randint(2, min(9, E - n_big + 1))
        z[r, pos[:n_big]] = 1.0
        tiny = 2.0 ** rng.uniform(-34, -25, n_tiny) * rng.choice([-1.0, 1.0], n_tiny)
        z[r, pos[n_big:n_big + n_tiny]] = tiny
    return torch.from_numpy(z).to(torch.bfloat16)


def collision_bias(E=64, seed=0):
    """fp32 logit bias whose neighbouring entries differ by one or two fp32 ulps around -0.3, and
    bf16 logits drawn from {0, 0.5}: the biased values then differ by a few ulps, so exp() and the
    1/sum scaling merge neighbours into equal fp32 probabilities."""
    import numpy as np
    rng = np.random.RandomState(seed)
    steps = np.cumsum(rng.randint(1, 3, E)).astype(np.uint32)
    # -0.3 moved towards zero by `steps` ulps (the bit pattern of a negative float falls)
    bias = (np.float32(-0.3).view(np.uint32) - steps).view(np.float32)
    return torch.from_numpy(rng.permutation(bias).astype(np.float32))


def collision_bias_logits(rows, E=64, seed=0):
    """The bf16 logits that go with collision_bias: 0 or 0.5 (one in ten)."""
    import numpy as np
    rng = np.random.RandomState(seed + 1)
    return torch.from_numpy(rng.choice([0.0, 0.5], size=(rows, E), p=[0.9, 0.1])).to(torch.bfloat16)
