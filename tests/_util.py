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
