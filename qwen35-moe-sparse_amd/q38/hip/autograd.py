"""Differentiable HIP MoE pieces: the routed experts (the training counterpart of
``ops.experts_forward``), the router and the shared expert.

The reference's differentiable experts path is ``padded_batched_experts_forward``
(q38/inference.py:358-384: gather, bmm gate/up, SiLU * up, bmm down, * top_k_weights, scatter-sum);
its gradients of x, top_k_weights, gate_up_proj and down_proj are what
scripts/check_q38_kernels.py:19-27 compares. Here the forward is the inference pipeline (histogram,
permutation, grouped gate/up + SwiGLU, grouped down, combine) keeping the sorted H and Y rows and
the rounded gate/up pre-activations [g | u] (q38moe_gate_up_save writes them next to H; 2I bf16
per row), and the backward runs, with Y' = dout[t] * w[p] (the routed raw rows' gradient) in sorted
order:

  dw[p]   = <dout[t], Y[p]>                       q38moe_pair_dots (which also writes Y')
  dH      = Y' . down_proj[e]                     q38moe_down_kn on down_proj [E, h, I] as stored
  dGU     = SwiGLU backward (dH, g, u)            q38moe_swiglu_backward
  dx_p    = dGU . gate_up_proj[e]                 q38moe_down_kn on gate_up_proj [E, 2I, h] as stored
  dx[t]   = sum_j dx_p[inv[t*k+j]]                q38moe_combine with unit weights
  d down_proj[e]    = Y'_e^T . H_e                q38moe_expert_wgrad (sorted rows)
  d gate_up_proj[e] = dGU_e^T . x_e               q38moe_expert_wgrad (x rows gathered through perm)

Expert row ranges stay on the device (starts/counts of the permutation): the backward makes no
host synchronisation.

The kernels take bf16. Under bf16 autocast, parameters and activations of another dtype (the
reference's training setup: fp32 parameters with torch.autocast, scripts/check_q38_kernels.py:19-26,
whose padded path then runs its bmm in bf16) are cast to bf16 by differentiable .to() calls, and
the output comes back in hidden_states' dtype, so their gradients arrive in their own dtype. Indices
are int32/int64 as in the forward.
"""
import torch

from . import ops


class HipExperts(torch.autograd.Function):
    @staticmethod
    def forward(ctx, x, topk_idx, topk_w, w_gate_up, w_down):
        T, h = x.shape
        k = topk_idx.shape[1]
        E = w_gate_up.shape[0]
        hist = ops.histogram(topk_idx, E)
        counts, starts, perm, inv, tiles, tcount = ops.permute(topk_idx, hist, E)
        H, GU = ops.gate_up_save(x, w_gate_up, perm, tiles, tcount, k)
        Y = ops.down(H, w_down, tiles, tcount, T, k)
        out = ops.combine(Y, inv, topk_w, E, idx=topk_idx)
        ctx.save_for_backward(x, topk_idx, topk_w, w_gate_up, w_down, counts, starts, perm, inv, tiles, tcount, H, Y,
                              GU)
        return out

    @staticmethod
    def backward(ctx, dout):
        x, idx, w, w_gate_up, w_down, counts, starts, perm, inv, tiles, tcount, H, Y, GU = ctx.saved_tensors
        T, h = x.shape
        k = idx.shape[1]
        E, twoI, _ = w_gate_up.shape
        dout = dout.to(torch.bfloat16).contiguous()
        need_x, _, need_w, need_gu, need_dn = ctx.needs_input_grad
        need_rows = need_x or need_gu or need_dn
        dw = d_raw = None
        if need_w and need_rows:
            dw, d_raw = ops.pair_dots(dout, Y, inv, idx, E, w=w)  # one pass over dout for both
        elif need_w:
            dw = ops.pair_dots(dout, Y, inv, idx, E)
        elif need_rows:
            d_raw = ops.gather_rows(dout, perm, starts, counts, k, w=w)
        dx = dgu_w = ddn_w = None
        if need_rows:
            if need_dn:
                ddn_w = ops.expert_wgrad(d_raw, H, starts, counts, k)
            if need_x or need_gu:
                dH = ops.down_kn(d_raw, w_down, tiles, tcount, T, k)
                dGU = ops.swiglu_backward(dH, GU)
                if need_gu:
                    dgu_w = ops.expert_wgrad(dGU, x, starts, counts, k, perm=perm)
                if need_x:
                    dxp = ops.down_kn(dGU, w_gate_up, tiles, tcount, T, k)
                    dx = ops.combine(dxp, inv, torch.ones_like(w), E, idx=idx)
        return dx, None, dw, dgu_w, ddn_w


def _bf16_autocast():
    return torch.is_autocast_enabled("cuda") and torch.get_autocast_dtype("cuda") == torch.bfloat16


def experts(x, topk_idx, topk_w, w_gate_up, w_down):
    """Routed experts with autograd (ExpertsInterface contract): [T,h] in x's dtype; gradients flow
    to x, topk_w, w_gate_up and w_down. Tensors must be bf16, or any float dtype under bf16
    autocast (cast to bf16 differentiably, as autocast casts the reference's bmm operands)."""
    named = ((x, "hidden_states"), (topk_w, "top_k_weights"), (w_gate_up, "gate_up_proj"), (w_down, "down_proj"))
    cast = False
    for t, n in named:
        if t.dtype != torch.bfloat16:
            if not (_bf16_autocast() and t.is_floating_point()):
                raise TypeError(f"{n} must be bf16 for the HIP experts (or run under bf16 autocast), got {t.dtype}")
            cast = True
    args = [t.to(torch.bfloat16).contiguous() for t, _ in named]
    out = HipExperts.apply(args[0], topk_idx.contiguous(), args[1], args[2], args[3])
    return out.to(x.dtype) if cast else out


class HipRouter(torch.autograd.Function):
    """Qwen3_8MoeTopKRouter.forward (modeling:805-812) with a backward. Forward: the HIP route kernel
    (logits on MFMA, fp32 softmax, top-k, renormalised weights). Backward, differentiating the same
    steps in fp32 from the saved logits: the renormalisation w = v / sum(v) of the top-k
    probabilities v, torch.topk's scatter of their gradient into the probability row, the softmax,
    plus the logits' own gradient (the load-balancing loss reads them through the gate's forward
    hook, q38/train.py:228-233); then the linear layer's two products in the logits' dtype."""

    @staticmethod
    def forward(ctx, x, w_router, k, logit_bias):
        logits, idx, w, _, _ = ops.route(x, w_router, k, logit_bias=logit_bias, want_logits=True)
        ctx.save_for_backward(x, w_router, logits, idx, logit_bias)
        ctx.mark_non_differentiable(idx)
        return logits, w, idx

    @staticmethod
    def backward(ctx, d_logits, d_w, _):
        x, w_router, logits, idx, bias = ctx.saved_tensors
        need_x, need_w = ctx.needs_input_grad[:2]
        return (*router_backward(x, w_router, logits, idx, bias, d_logits, d_w, need_x, need_w), None, None)


def router_backward(x, w_router, logits, idx, bias, d_logits, d_w, need_x=True, need_w=True):
    """Gradients (dx, d w_router) of the router's outputs (logits, renormalised top-k weights) given
    their gradients (either may be None), from the forward's logits and indices."""
    z = logits.float() if bias is None else logits.float() + bias
    p = torch.softmax(z, dim=-1)
    dz = None
    if d_w is not None:
        il = idx.long()
        v = p.gather(1, il)
        s = v.sum(1, keepdim=True)
        gw = d_w.float()
        dv = (gw - (gw * (v / s)).sum(1, keepdim=True)) / s  # through w = v / sum(v)
        dp = torch.zeros_like(p).scatter_(1, il, dv)           # torch.topk's backward
        dz = p * (dp - (dp * p).sum(1, keepdim=True))           # softmax's backward
    if d_logits is not None:
        dz = d_logits.float() if dz is None else dz + d_logits.float()
    if dz is None:
        return None, None
    dz = dz.to(logits.dtype)
    dx = dz @ w_router if need_x else None
    dwr = dz.t().contiguous() @ x if need_w else None
    return dx, dwr


def router(x, w_router, k, logit_bias=None):
    """Router with autograd: (logits [T,E], weights [T,k], indices int32 [T,k]) as the gate module
    returns them (modeling:805-813); gradients flow to x and w_router through the weights and the
    logits. bf16 or fp32 tensors; under bf16 autocast other float dtypes are cast to bf16
    differentiably (autocast's F.linear), and the logits and weights come out in bf16."""
    if _bf16_autocast() and (x.dtype != torch.bfloat16 or w_router.dtype != torch.bfloat16):
        x, w_router = x.to(torch.bfloat16), w_router.to(torch.bfloat16)
    if logit_bias is not None:
        logit_bias = logit_bias.float().contiguous()
    return HipRouter.apply(x.contiguous(), w_router.contiguous(), k, logit_bias)


def shared_expert(x, w_gate, w_up, w_down):
    """The shared SwiGLU MLP (modeling:751-753) with autograd, as the routed experts' path with one
    expert and every token routed to it at weight 1: gate/up, bf16 SiLU * up and down round at the
    MLP's own points, and the k-sum of one exact term changes nothing. Gradients flow to x and the
    three weights (through the concatenation [gate; up] = gate_up_proj[0])."""
    T = x.shape[0]
    idx = torch.zeros(T, 1, dtype=torch.int32, device=x.device)
    ones = torch.ones(T, 1, dtype=torch.bfloat16, device=x.device)
    w_gate_up = torch.cat([w_gate, w_up], 0).unsqueeze(0)
    out = experts(x, idx, ones, w_gate_up, w_down.unsqueeze(0))
    # Under autocast the MLP's last nn.Linear returns the autocast dtype, whatever x's dtype.
    return out.to(torch.bfloat16) if _bf16_autocast() else out
