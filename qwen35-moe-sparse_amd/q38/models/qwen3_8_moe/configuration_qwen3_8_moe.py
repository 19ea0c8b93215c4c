"""MoE fields of the Q38 text config (configuration_qwen3_8_moe.py:63-99 in the reference).

The drop-in MoE modules read only these attributes, so the reference's own
``Qwen3_8MoeTextConfig`` works with them unchanged; this class is a light stand-in for code that
builds MoE blocks without the full model config. Defaults are the Q38 preset values (64 experts,
top-5, h/4 expert widths; q38/presets.py:21-83), not the reference class defaults.
"""


class Qwen3_8MoeTextConfig:
    model_type = "qwen38_moe_sparse"

    def __init__(self, hidden_size=1024, num_experts=64, num_experts_per_tok=5, moe_intermediate_size=256,
                 shared_expert_intermediate_size=256, hidden_act="silu", initializer_range=0.02,
                 experts_implementation="q38_hip", **kwargs):
        self.hidden_size = hidden_size
        self.num_experts = num_experts
        self.num_experts_per_tok = num_experts_per_tok
        self.moe_intermediate_size = moe_intermediate_size
        self.shared_expert_intermediate_size = shared_expert_intermediate_size
        self.hidden_act = hidden_act
        self.initializer_range = initializer_range
        # Read by transformers' use_experts_implementation dispatch (integrations/moe.py:567-570).
        self._experts_implementation = experts_implementation
        for key, value in kwargs.items():
            setattr(self, key, value)


__all__ = ["Qwen3_8MoeTextConfig"]
