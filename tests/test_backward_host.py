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


@pytest.mark.parametrize("bias", [False, True])
def test_router_backward_matches_autograd(bias):
    """q38.hip.autograd.router_backward (the differentiable router's backward, run after the HIP
    route kernel) against torch autograd of the reference router's op sequence (modeling:805-812:
    linear, softmax in fp32, top-k, renormalisation), in float64 on the same logits and indices,
    with gradients on both outputs (the routing weights and the logits, as the load-balancing loss
    reads them)."""
    from q38.hip import autograd
    g = torch.Generator().manual_seed(5)
    T, h, E, k = 37, 48, 16, 4
    x = torch.randn(T, h, generator=g, dtype=torch.float64, requires_grad=True)
    wr = (torch.randn(E, h, generator=g, dtype=torch.float64) * 0.2).requires_grad_(True)
    b = torch.randn(E, generator=g, dtype=torch.float64) * 0.3 if bias else None
    logits = torch.nn.functional.linear(x, wr)
    z = logits if b is None else logits + b
    probs = torch.softmax(z, dim=-1)
    top, idx = torch.topk(probs, k, dim=-1)
    w = top / top.sum(dim=-1, keepdim=True)
    d_w = torch.randn(T, k, generator=g, dtype=torch.float64)
    d_logits = torch.randn(T, E, generator=g, dtype=torch.float64) * 0.1
    (w * d_w).sum().add_((logits * d_logits).sum()).backward()
    dx, dwr = autograd.router_backward(x.detach(), wr.detach(), logits.detach(), idx, b, d_logits, d_w)
    # router_backward works in float32 internally: compare at float32 accuracy
    assert torch.allclose(dx, x.grad, rtol=1e-5, atol=1e-6)
    assert torch.allclose(dwr, wr.grad, rtol=1e-5, atol=1e-6)
    # each output's gradient alone
    for dl, dww in ((None, d_w), (d_logits, None)):
        x.grad = wr.grad = None
        lo = torch.nn.functional.linear(x, wr)
        zz = lo if b is None else lo + b
        t2, _ = torch.topk(torch.softmax(zz, -1), k, -1)
        terms = []
        if dww is not None:
            terms.append((t2 / t2.sum(-1, keepdim=True) * dww).sum())
        if dl is not None:
            terms.append((lo * dl).sum())
        sum(terms).backward()
        dx1, dwr1 = autograd.router_backward(x.detach(), wr.detach(), lo.detach(), idx, b, dl, dww)
        assert torch.allclose(dx1, x.grad, rtol=1e-5, atol=1e-6) and torch.allclose(dwr1, wr.grad, rtol=1e-5, atol=1e-6)
