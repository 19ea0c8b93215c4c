"""Drop-in MoE modules of the Q38 model, running on the gfx950 HIP kernels.

Same class names, constructor signatures, submodule names, parameter names/shapes and forward
signatures as the reference (q38/models/qwen3_8_moe/modeling_qwen3_8_moe.py:740-835), so a
reference state dict loads unchanged and callers (the packed prefill's ``layer.mlp(...)`` at
modeling:1271, the decoder layer at :909) use them as they are. Forward-only: every forward raises
under autograd. Inputs and weights must be bf16 CUDA tensors; there is no CPU path.
"""
import torch
from torch import nn

from ...hip import ops
from ...inference import (EXPERTS_IMPLEMENTATION, _check_act, _forward_only, hip_experts_forward,
                          hip_moe_block_forward)

try:  # the reference decorates its experts class with transformers' dispatcher (modeling:756)
    from transformers.integrations.moe import use_experts_implementation
except ImportError:  # pragma: no cover - transformers is part of the image
    use_experts_implementation = None


class Qwen3_8MoeMLP(nn.Module):
    """SwiGLU MLP used as the shared expert (modeling:740-753)."""

    def __init__(self, config, intermediate_size: int):
        super().__init__()
        self.config = config
        self.hidden_size = config.hidden_size
        self.intermediate_size = intermediate_size
        self.gate_proj = nn.Linear(self.hidden_size, self.intermediate_size, bias=False)
        self.up_proj = nn.Linear(self.hidden_size, self.intermediate_size, bias=False)
        self.down_proj = nn.Linear(self.intermediate_size, self.hidden_size, bias=False)
        _check_act(config.hidden_act)
        self.act_fn = nn.SiLU()

    def forward(self, x):
        _forward_only(x, self.gate_proj.weight, self.up_proj.weight, self.down_proj.weight)
        shape = x.shape
        out = ops.shared_expert(x.reshape(-1, shape[-1]).contiguous(), self.gate_proj.weight,
                                self.up_proj.weight, self.down_proj.weight)
        return out.view(shape)


class Qwen3_8MoeExperts(nn.Module):
    """Collection of expert weights stored as 3D tensors (modeling:756-793)."""

    def __init__(self, config):
        super().__init__()
        self.num_experts = config.num_experts
        self.hidden_dim = config.hidden_size
        self.intermediate_dim = config.moe_intermediate_size
        self.gate_up_proj = nn.Parameter(torch.empty(self.num_experts, 2 * self.intermediate_dim, self.hidden_dim))
        self.down_proj = nn.Parameter(torch.empty(self.num_experts, self.hidden_dim, self.intermediate_dim))
        _check_act(config.hidden_act)
        self.act_fn = nn.SiLU()

    def forward(self, hidden_states: torch.Tensor, top_k_index: torch.Tensor,
                top_k_weights: torch.Tensor) -> torch.Tensor:
        return hip_experts_forward(self, hidden_states, top_k_index, top_k_weights)


if use_experts_implementation is not None:
    Qwen3_8MoeExperts = use_experts_implementation(Qwen3_8MoeExperts)


class Qwen3_8MoeTopKRouter(nn.Module):
    """Softmax top-k router (modeling:796-813): returns (router_logits, router_scores, router_indices)."""

    def __init__(self, config):
        super().__init__()
        self.top_k = config.num_experts_per_tok
        self.num_experts = config.num_experts
        self.hidden_dim = config.hidden_size
        self.weight = nn.Parameter(torch.zeros(self.num_experts, self.hidden_dim))
        self.routing_bias = None  # optional fp32 [E] logit bias (routing-skew workload only)

    def forward(self, hidden_states):
        _forward_only(hidden_states, self.weight)
        hidden_states = hidden_states.reshape(-1, self.hidden_dim).contiguous()
        logits, idx, scores, _, _ = ops.route(hidden_states, self.weight, self.top_k, logit_bias=self.routing_bias,
                                              want_logits=True)
        return logits, scores, idx.long()


class Qwen3_8MoeSparseMoeBlock(nn.Module):
    """Router + routed experts + sigmoid-gated shared expert (modeling:816-835)."""

    def __init__(self, config):
        super().__init__()
        self.gate = Qwen3_8MoeTopKRouter(config)
        self.experts = Qwen3_8MoeExperts(config)
        self.shared_expert = Qwen3_8MoeMLP(config, intermediate_size=config.shared_expert_intermediate_size)
        self.shared_expert_gate = torch.nn.Linear(config.hidden_size, 1, bias=False)

    @property
    def routing_bias(self):
        return self.gate.routing_bias

    def forward(self, hidden_states: torch.Tensor) -> torch.Tensor:
        if self.gate._forward_hooks or self.gate._forward_pre_hooks:
            # Observers of the router output (modeling:928; q38/train.py:228) see the gate
            # module's tuple: run the block as its submodules, each on the HIP kernels.
            return self._forward_by_submodules(hidden_states)
        return hip_moe_block_forward(self, hidden_states)

    def _forward_by_submodules(self, hidden_states):
        batch_size, sequence_length, hidden_dim = hidden_states.shape
        x = hidden_states.view(-1, hidden_dim)
        shared_expert_output = self.shared_expert(x)
        _, routing_weights, selected_experts = self.gate(x)
        expert_output = self.experts(x, selected_experts, routing_weights)
        gate_logit = ops.route(x.contiguous(), self.gate.weight, self.gate.top_k,
                               w_shared_gate=self.shared_expert_gate.weight)[3]
        # sigmoid(shared_expert_gate(x)) * shared + routed, in bf16 (modeling:831-833): the combine
        # with one pair per token, weight 1 (exact in bf16) and the identity row map.
        T = x.shape[0]
        ident = torch.arange(T, dtype=torch.int32, device=x.device)
        ones = torch.ones(T, 1, dtype=torch.bfloat16, device=x.device)
        y = ops.combine(expert_output.contiguous(), ident, ones, self.gate.num_experts,
                        shared_out=shared_expert_output.contiguous(), shared_gate_logit=gate_logit)
        return y.reshape(batch_size, sequence_length, hidden_dim)


def new_config(**kwargs):
    from .configuration_qwen3_8_moe import Qwen3_8MoeTextConfig

    kwargs.setdefault("experts_implementation", EXPERTS_IMPLEMENTATION)
    return Qwen3_8MoeTextConfig(**kwargs)


__all__ = ["Qwen3_8MoeMLP", "Qwen3_8MoeExperts", "Qwen3_8MoeTopKRouter", "Qwen3_8MoeSparseMoeBlock"]
