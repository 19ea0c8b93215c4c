from .configuration_qwen3_8_moe import Qwen3_8MoeTextConfig
from .modeling_qwen3_8_moe import (Qwen3_8MoeExperts, Qwen3_8MoeForCausalLM, Qwen3_8MoeMLP,
                                   Qwen3_8MoePreTrainedModel, Qwen3_8MoeSparseMoeBlock, Qwen3_8MoeTopKRouter,
                                   new_config, prefill_config)

# Exports carry this implementation and its config, as the reference's do (its __init__.py:8-12):
# save_pretrained writes auto_map entries and copies the two files; AutoModelForCausalLM with
# trust_remote_code=True then builds the model from them.
Qwen3_8MoeTextConfig.register_for_auto_class("AutoConfig")
Qwen3_8MoeForCausalLM.register_for_auto_class("AutoModelForCausalLM")

__all__ = ["Qwen3_8MoeTextConfig", "Qwen3_8MoeExperts", "Qwen3_8MoeForCausalLM", "Qwen3_8MoeMLP",
           "Qwen3_8MoePreTrainedModel", "Qwen3_8MoeSparseMoeBlock", "Qwen3_8MoeTopKRouter", "new_config",
           "prefill_config"]
