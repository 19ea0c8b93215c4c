"""Inference fast path for the MoE feed-forward: the HIP experts implementation and installer.

Mirrors the MoE part of the reference's q38/inference.py: ``hip_experts_forward`` has the
ExpertsInterface signature of ``triton_experts_forward`` (inference.py:158-199) and is registered
under ``EXPERTS_IMPLEMENTATION`` like inference.py:337-338; ``hip_moe_block_forward`` replaces a
whole ``Qwen3_8MoeSparseMoeBlock.forward`` (modeling_qwen3_8_moe.py:824-835) with one fused call.
Under autograd ``hip_experts_forward`` runs the differentiable HIP experts (``q38.hip.autograd``,
the counterpart of the reference's padded path, inference.py:358-384); the fused block stays
forward-only and raises under autograd, as the reference's Triton path does (inference.py:160-161).
They work on the reference's own modules and on the drop-in modules of ``q38.models.qwen3_8_moe``.
"""
import types

import torch

from .hip import ops

EXPERTS_IMPLEMENTATION = "q38_hip"


def _needs_grad(*tensors):
    return torch.is_grad_enabled() and any(t is not None and t.requires_grad for t in tensors)


def _forward_only(*tensors):
    if _needs_grad(*tensors):
        raise RuntimeError("The fused HIP MoE block has no backward; run it under torch.inference_mode() "
                           "or call the block module, which runs its differentiable submodules")


def _check_act(act_name):
    if act_name not in (None, "silu", "swish"):
        raise ValueError(f"the HIP MoE kernels implement SiLU gating only, got hidden_act={act_name!r}")


def hip_experts_forward(self, hidden_states, top_k_index, top_k_weights):
    """Routed experts on HIP: fn(self, hidden_states[T,h], top_k_index[T,k], top_k_weights[T,k]) -> [T,h].

    self provides ``gate_up_proj`` [E,2I,h] and ``down_proj`` [E,h,I] (modeling:756-767).
    Same math and rounding order as inference.py:158-199; indices outside [0,E) contribute nothing.
    When autograd needs gradients of any input or weight, the differentiable HIP experts run
    (gradients of x, top_k_weights, gate_up_proj, down_proj, as the reference's padded path).
    """
    cfg = getattr(self, "config", None)
    _check_act(getattr(cfg, "hidden_act", None))
    weights = top_k_weights
    if weights.dtype != hidden_states.dtype:
        weights = weights.to(hidden_states.dtype)
    if torch.is_grad_enabled() and any(t.requires_grad for t in (hidden_states, weights, self.gate_up_proj,
                                                                    self.down_proj)):
        from .hip import autograd
        return autograd.experts(hidden_states, top_k_index, weights, self.gate_up_proj, self.down_proj)
    return ops.experts_forward(hidden_states.contiguous(), top_k_index.contiguous(), weights.contiguous(),
                               self.gate_up_proj.contiguous(), self.down_proj.contiguous())


def _block_weights(block):
    sh = block.shared_expert
    return (block.gate.weight, block.experts.gate_up_proj, block.experts.down_proj, sh.gate_proj.weight,
            sh.up_proj.weight, sh.down_proj.weight, block.shared_expert_gate.weight)


def hip_moe_block_forward(self, hidden_states):
    """Qwen3_8MoeSparseMoeBlock.forward (modeling:824-835) as one fused HIP call: [B,S,h] -> [B,S,h].

    An optional ``routing_bias`` attribute (fp32 [E]) is added to the router logits before the
    softmax (routing-skew workload; None = reference behaviour).
    """
    return _fused_block(self, hidden_states, False)


def hip_moe_block_forward_with_router(self, hidden_states):
    """``hip_moe_block_forward`` that also returns the router logits [B*S, E] (the gate's output[0],
    modeling:805-807, what the reference's router-logits recorder keeps), from the same fused call."""
    return _fused_block(self, hidden_states, True)


def _fused_block(self, hidden_states, want_logits):
    weights = _block_weights(self)
    _forward_only(hidden_states, *weights)
    _check_act(getattr(getattr(self.experts, "config", None), "hidden_act", None))
    shape = hidden_states.shape
    x = hidden_states.reshape(-1, shape[-1]).contiguous()
    k = self.gate.top_k
    res = ops.block_forward(x, *(w.contiguous() for w in weights), k,
                            logit_bias=getattr(self, "routing_bias", None), return_router=want_logits,
                            workspace=_workspace(self, x.device, ops.block_workspace_bytes(
                                x.shape[0], x.shape[1], weights[0].shape[0], k, weights[1].shape[1] // 2,
                                weights[3].shape[0], x.dtype)))
    if want_logits:
        return res[0].view(shape), res[1]
    return res.view(shape)


def _workspace(module, device, nbytes):
    ws = getattr(module, "_q38_workspace", None)
    if ws is None or ws.device != device or ws.numel() < nbytes:
        ws = torch.empty(nbytes, dtype=torch.uint8, device=device)
        module._q38_workspace = ws
    return ws


def register_experts_implementation():
    """Register ``hip_experts_forward`` with transformers' ExpertsInterface (inference.py:337)."""
    from transformers.integrations.moe import ALL_EXPERTS_FUNCTIONS

    ALL_EXPERTS_FUNCTIONS.register(EXPERTS_IMPLEMENTATION, hip_experts_forward)
    return EXPERTS_IMPLEMENTATION


def optimize_for_inference(model, fuse_blocks=True):
    """Install the HIP MoE path on a loaded model in place (the MoE part of inference.py:333-355).

    Registers and selects the HIP experts implementation; with ``fuse_blocks`` every MoE block's
    forward becomes one fused HIP call. Returns counts for logging.
    """
    register_experts_implementation()
    if hasattr(model, "set_experts_implementation"):
        model.set_experts_implementation(EXPERTS_IMPLEMENTATION)
    blocks = 0
    if fuse_blocks:
        for module in model.modules():
            if all(hasattr(module, a) for a in ("gate", "experts", "shared_expert", "shared_expert_gate")):
                module._reference_forward = module.forward
                module.forward = types.MethodType(hip_moe_block_forward, module)
                blocks += 1
    return dict(experts=EXPERTS_IMPLEMENTATION, moe_blocks=blocks)
