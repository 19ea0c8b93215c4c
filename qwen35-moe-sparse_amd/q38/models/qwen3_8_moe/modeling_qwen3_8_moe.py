"""Drop-in MoE modules of the Q38 model, running on the gfx950 HIP kernels, and the causal-LM
model class for packed prefill and HF export.

Same class names, constructor signatures, submodule names, parameter names/shapes and forward
signatures as the reference (q38/models/qwen3_8_moe/modeling_qwen3_8_moe.py:740-835), so a
reference state dict loads unchanged and callers (the packed prefill's ``layer.mlp(...)`` at
modeling:1271, the decoder layer at :909) use them as they are. ``Qwen3_8MoeForCausalLM`` is the
reference's causal-LM class for uncached packed prefill (modeling:1358-1433) over the restated trunk
of ``q38.prefill``; it is registered for the Auto classes like the reference (__init__.py:8-12), so
``save_pretrained`` exports this file and ``from_pretrained(..., trust_remote_code=True)`` runs the
kernels again. The imports of the library are absolute because an export runs this file outside
the package: the ``q38`` package must be importable where an export is loaded.
Under autograd the block is differentiable: the routed experts and the shared MLP through the HIP
experts backward (bf16 tensors, or fp32 parameters under bf16 autocast), the router through its
HIP forward and a backward of the softmax / top-k / renormalisation steps, and the shared gate
through torch; the block then runs as its submodules, so a forward hook on ``gate`` (the reference
trainer's router recorder, q38/train.py:228-233) sees the router output and its gradient reaches
the router. Without autograd and hooks the block is one fused HIP call. The causal LM is
forward-only. Inputs and weights are CUDA tensors; there is no CPU path.
"""
import torch
from torch import nn
from transformers.modeling_outputs import MoeCausalLMOutputWithPast
from transformers.modeling_utils import PreTrainedModel

from q38 import prefill as _prefill
from q38.hip import ops
from q38.inference import (EXPERTS_IMPLEMENTATION, _check_act, _needs_grad, hip_experts_forward,
                           hip_moe_block_forward, hip_moe_block_forward_with_router,
                           register_experts_implementation)

from .configuration_qwen3_8_moe import Qwen3_8MoeTextConfig

# "q38_hip" must be a registered experts implementation before a model whose config selects it is
# built (transformers checks the name in PreTrainedModel.__init__).
register_experts_implementation()

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
        shape = x.shape
        if _needs_grad(x, self.gate_proj.weight, self.up_proj.weight, self.down_proj.weight):
            from q38.hip import autograd
            out = autograd.shared_expert(x.reshape(-1, shape[-1]), self.gate_proj.weight, self.up_proj.weight,
                                         self.down_proj.weight)
            return out.view(*shape[:-1], out.shape[-1])
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
        hidden_states = hidden_states.reshape(-1, self.hidden_dim)
        if _needs_grad(hidden_states, self.weight):
            from q38.hip import autograd
            logits, scores, idx = autograd.router(hidden_states, self.weight, self.top_k, logit_bias=self.routing_bias)
            return logits, scores, idx.long()
        hidden_states = hidden_states.contiguous()
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
        if (self.gate._forward_hooks or self.gate._forward_pre_hooks
                or _needs_grad(hidden_states, *(p for p in self.parameters()))):
            # Observers of the router output (modeling:928; q38/train.py:228) see the gate
            # module's tuple, and autograd needs the pieces: run the block as its submodules.
            return self._forward_by_submodules(hidden_states)
        return hip_moe_block_forward(self, hidden_states)

    def _forward_by_submodules(self, hidden_states):
        """modeling:824-835 as its submodules, each on the HIP kernels."""
        batch_size, sequence_length, hidden_dim = hidden_states.shape
        x = hidden_states.view(-1, hidden_dim)
        shared_expert_output = self.shared_expert(x)
        _, routing_weights, selected_experts = self.gate(x)
        expert_output = self.experts(x, selected_experts, routing_weights)
        gate_logit = self.shared_expert_gate(x)
        if torch.is_grad_enabled() and (gate_logit.requires_grad or expert_output.requires_grad
                                        or shared_expert_output.requires_grad):
            # The reference's own ops (modeling:831-833), differentiable.
            out = expert_output + torch.sigmoid(gate_logit) * shared_expert_output
            return out.reshape(batch_size, sequence_length, hidden_dim)
        # sigmoid(shared_expert_gate(x)) * shared + routed, in x's dtype (modeling:831-833): the
        # combine with one pair per token, weight 1 (exact) and the identity row map.
        gate_logit = gate_logit.reshape(-1).to(x.dtype)
        T = x.shape[0]
        ident = torch.arange(T, dtype=torch.int32, device=x.device)
        ones = torch.ones(T, 1, dtype=x.dtype, device=x.device)
        y = ops.combine(expert_output.contiguous(), ident, ones, self.gate.num_experts,
                        shared_out=shared_expert_output.contiguous(), shared_gate_logit=gate_logit)
        return y.reshape(batch_size, sequence_length, hidden_dim)


def new_config(**kwargs):
    kwargs.setdefault("experts_implementation", EXPERTS_IMPLEMENTATION)
    return Qwen3_8MoeTextConfig(**kwargs)


def prefill_config(config):
    """The ``q38.prefill.PrefillConfig`` of a Qwen3_8MoeTextConfig (reference field names)."""
    if config.linear_key_head_dim != config.linear_value_head_dim:
        raise ValueError("the prefill needs equal DeltaNet key and value head widths")
    rope = config.rope_parameters or {}
    eos = config.eos_token_id[0] if isinstance(config.eos_token_id, (list, tuple)) else config.eos_token_id
    return _prefill.PrefillConfig(
        vocab=config.vocab_size, hidden=config.hidden_size, layers=config.num_hidden_layers,
        heads=config.num_attention_heads, kv_heads=config.num_key_value_heads, head_dim=config.head_dim,
        lin_k_heads=config.linear_num_key_heads, lin_v_heads=config.linear_num_value_heads,
        lin_head_dim=config.linear_key_head_dim, conv_kernel=config.linear_conv_kernel_dim,
        experts=config.num_experts, topk=config.num_experts_per_tok, moe_ffn=config.moe_intermediate_size,
        shared_ffn=config.shared_expert_intermediate_size, rope_theta=rope.get("rope_theta", 1e7),
        partial_rotary=rope.get("partial_rotary_factor", 0.25), n_branch=config.n_branch,
        mhc_iters=config.mhc_iters, qsa_blocks=config.qsa_blocks, indexer_heads=config.indexer_heads,
        indexer_head_dim=config.indexer_head_dim, ngram_rows=config.ngram_rows, eos_id=eos,
        pad_id=config.pad_token_id if config.pad_token_id is not None else eos, rms_eps=config.rms_norm_eps,
        layer_types=tuple(config.layer_types))


class Qwen3_8MoePreTrainedModel(PreTrainedModel):
    """Weight initialisation of a fresh model after the reference's (modeling:935-960, 1036-1043,
    1169-1177); loading a checkpoint replaces all of it."""

    config_class = Qwen3_8MoeTextConfig
    base_model_prefix = "model"
    _keys_to_ignore_on_load_unexpected = [r"^mtp\."]

    @torch.no_grad()
    def _init_weights(self, module):
        std = self.config.initializer_range
        if isinstance(module, (nn.Linear, nn.Conv1d, nn.Embedding)):
            module.weight.normal_(0.0, std)
            if getattr(module, "bias", None) is not None:
                module.bias.zero_()
        elif isinstance(module, _prefill._Norm):
            module.weight.fill_(module.init_value)
        elif isinstance(module, nn.RMSNorm):  # the N-gram embedding's norm
            module.weight.fill_(0.02)
        elif isinstance(module, Qwen3_8MoeExperts):
            module.gate_up_proj.normal_(0.0, std)
            module.down_proj.normal_(0.0, std)
        elif isinstance(module, Qwen3_8MoeTopKRouter):
            module.weight.normal_(0.0, std)
        elif isinstance(module, _prefill._DeltaNet):
            module.dt_bias.fill_(1.0)
            module.A_log.copy_(torch.empty_like(module.A_log).uniform_(0.01, 16).log_())
        elif isinstance(module, _prefill._MHC):
            n = module.b_pre.numel()
            pre = torch.full((n,), 0.1)
            pre[module.slot % n] = 0.7
            module.b_pre.copy_(torch.log(pre / (1 - pre)))
            module.b_post.zero_()
            module.b_res.copy_(torch.full((n, n), -8.0) + 8.0 * torch.eye(n))
            module.alphas.fill_(0.1)
            module.B.weight.zero_()
        elif isinstance(module, _prefill._NGram):
            module.gate.bias.fill_(-1.0)


class Qwen3_8MoeForCausalLM(Qwen3_8MoePreTrainedModel):
    """Causal LM head over the Q38 trunk for uncached packed prefill (modeling:1358-1433): the same
    module tree and parameter names as the reference (``model.*``, tied ``lm_head``), the MoE blocks
    on the fused HIP block. ``forward(input_ids, output_router_logits=None, logits_to_keep=0)``
    returns logits (and with router logits, the load-balancing loss) in a MoeCausalLMOutputWithPast."""

    _tied_weights_keys = {"lm_head.weight": "model.embed_tokens.weight"}

    def __init__(self, config):
        super().__init__(config)
        self.prefill_config = prefill_config(config)
        self.model = _prefill._Trunk(self.prefill_config)
        self.lm_head = nn.Linear(config.hidden_size, config.vocab_size, bias=False)
        self.post_init()

    def get_input_embeddings(self):
        return self.model.embed_tokens

    def get_output_embeddings(self):
        return self.lm_head

    def _moe(self, block, x, with_router):
        return hip_moe_block_forward_with_router(block, x) if with_router else block(x)

    def forward(self, input_ids=None, output_router_logits=None, logits_to_keep=0, **kwargs):
        if input_ids is None or kwargs.get("past_key_values") is not None or kwargs.get("attention_mask") is not None:
            raise ValueError("Q38 supports uncached packed prefill from input_ids without attention_mask")
        want = self.config.output_router_logits if output_router_logits is None else output_router_logits
        router = [] if want else None
        cfg = self.prefill_config
        with torch.no_grad():
            hs = _prefill.trunk_forward(self.model, cfg, input_ids, self._moe, router)
            keep = slice(-logits_to_keep, None) if isinstance(logits_to_keep, int) else logits_to_keep
            logits = self.lm_head(hs[:, keep, :])
            aux = _prefill.load_balancing_loss(router, cfg.experts, cfg.topk) if want else None
        return MoeCausalLMOutputWithPast(logits=logits, aux_loss=aux, router_logits=tuple(router) if want else None)


__all__ = ["Qwen3_8MoeMLP", "Qwen3_8MoeExperts", "Qwen3_8MoeTopKRouter", "Qwen3_8MoeSparseMoeBlock",
           "Qwen3_8MoePreTrainedModel", "Qwen3_8MoeForCausalLM"]
