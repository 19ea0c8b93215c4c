"""Host-side contracts of the differentiable HIP experts (q38.hip.autograd), no GPU needed: bf16
only outside bf16 autocast, and no CPU fallback (CPU tensors are refused before any kernel launch)."""
import pytest
import torch


def _args(dtype=torch.bfloat16):
    T, h, E, k, I = 8, 64, 4, 2, 64
    x = torch.randn(T, h).to(dtype).requires_grad_(True)
    idx = torch.randint(0, E, (T, k))
    w = torch.rand(T, k).to(dtype).requires_grad_(True)
    wgu = (torch.randn(E, 2 * I, h) * 0.02).to(dtype).requires_grad_(True)
    wdn = (torch.randn(E, h, I) * 0.02).to(dtype).requires_grad_(True)
    return x, idx, w, wgu, wdn


def test_experts_requires_bf16():
    from q38.hip import autograd
    with pytest.raises(TypeError, match="bf16"):
        autograd.experts(*_args(torch.float32))
    with pytest.raises(TypeError, match="bf16"):
        autograd.experts(*_args(torch.float16))


def test_experts_refuses_cpu_tensors():
    from q38.hip import autograd
    with pytest.raises(RuntimeError, match="CUDA/HIP tensor"):
        autograd.experts(*_args())


def test_registered_experts_route_to_autograd_under_grad():
    """Under autograd the ExpertsInterface entry takes the differentiable path (which, on CPU
    tensors, refuses them) instead of raising the forward-only error."""
    from q38.inference import hip_experts_forward
    x, idx, w, wgu, wdn = _args()

    class Experts(torch.nn.Module):
        def __init__(self):
            super().__init__()
            self.gate_up_proj = torch.nn.Parameter(wgu.detach())
            self.down_proj = torch.nn.Parameter(wdn.detach())

    with pytest.raises(RuntimeError, match="CUDA/HIP tensor"):
        hip_experts_forward(Experts(), x, idx, w)
