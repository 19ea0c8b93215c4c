"""Q38 text config (the reference's configuration_qwen3_8_moe.py:7-111), as a transformers config.

Same ``model_type`` and field names as the reference, so its config.json files load here and the
drop-in modules read the fields they know. Defaults describe benchmark config 5 (12 layers at
hidden 1024, 64 experts top-5 with h/4 widths, vocab 10112, EOS 53; q38/presets.py:21-83 and
scripts/make_q38_configs.py:81-89), not the reference class defaults. The MoE blocks dispatch to
this library's kernels: ``experts_implementation`` defaults to "q38_hip".
"""
from transformers.configuration_utils import PreTrainedConfig


class Qwen3_8MoeTextConfig(PreTrainedConfig):
    model_type = "qwen38_moe_sparse"
    keys_to_ignore_at_inference = ["past_key_values"]

    vocab_size: int = 10112
    hidden_size: int = 1024
    num_hidden_layers: int = 12
    num_attention_heads: int = 38
    num_key_value_heads: int = 2
    head_dim: int = 64
    hidden_act: str = "silu"
    max_position_embeddings: int = 4096
    initializer_range: float = 0.02
    rms_norm_eps: float = 1e-6
    use_cache: bool = False
    tie_word_embeddings: bool = True
    rope_parameters: dict | None = None
    attention_bias: bool = False
    linear_conv_kernel_dim: int = 4
    linear_key_head_dim: int = 64
    linear_value_head_dim: int = 64
    linear_num_key_heads: int = 13
    linear_num_value_heads: int = 39
    moe_intermediate_size: int = 256
    shared_expert_intermediate_size: int = 256
    num_experts_per_tok: int = 5
    num_experts: int = 64
    n_branch: int = 4
    mhc_iters: int = 20
    qsa_blocks: int = 8
    indexer_heads: int = 4
    indexer_head_dim: int = 64
    ngram_rows: int = 131072
    mtp: bool = False
    output_router_logits: bool = False
    router_aux_loss_coef: float = 0.001
    layer_types: list[str] | None = None
    pad_token_id: int | None = 53
    bos_token_id: int | None = 53
    eos_token_id: int | list[int] | None = 53

    def __post_init__(self, **kwargs):
        partial = kwargs.pop("partial_rotary_factor", 0.25)
        theta = kwargs.pop("rope_theta", 1e7)
        experts_impl = kwargs.pop("experts_implementation", "q38_hip")
        if self.rope_parameters is None:
            self.rope_parameters = {"rope_type": "default", "rope_theta": theta, "partial_rotary_factor": partial}
        self.rope_parameters.setdefault("partial_rotary_factor", partial)
        if self.layer_types is None:  # every 4th layer full attention (presets.py:55-56)
            self.layer_types = ["full_attention" if i % 4 == 3 else "linear_attention"
                                for i in range(self.num_hidden_layers)]
        super().__post_init__(**kwargs)
        # Read by transformers' use_experts_implementation dispatch (integrations/moe.py:567-570).
        self._experts_implementation = experts_impl


__all__ = ["Qwen3_8MoeTextConfig"]
