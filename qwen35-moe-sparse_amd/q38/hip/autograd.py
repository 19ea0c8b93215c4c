"""Differentiable routed experts on HIP: the training counterpart of ``ops.experts_forward``.

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
