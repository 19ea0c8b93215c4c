from .configuration_qwen3_8_moe import Qwen3_8MoeTextConfig
from .modeling_qwen3_8_moe import (Qwen3_8MoeExperts, Qwen3_8MoeMLP, Qwen3_8MoeSparseMoeBlock,
                                   Qwen3_8MoeTopKRouter, new_config)

__all__ = ["Qwen3_8MoeTextConfig", "Qwen3_8MoeExperts", "Qwen3_8MoeMLP", "Qwen3_8MoeSparseMoeBlock",
           "Qwen3_8MoeTopKRouter", "new_config"]
