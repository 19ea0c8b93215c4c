"""HF export of the Q38 causal LM with the drop-in MoE (the reference's tests/test_model.py:39-45
round trip: save_pretrained, then AutoModelForCausalLM.from_pretrained(trust_remote_code=True)).

CPU part: the export carries this repository's model code (auto_map, copied files), the loaded
class comes from the exported module, the weights come back equal and tied, and the parameter
names are the reference's. The forward runs the HIP kernels, so logits are compared on the GPU.
"""
import dataclasses
import json
import os

import pytest
import torch

from q38 import prefill as P
from q38.models.qwen3_8_moe import Qwen3_8MoeForCausalLM, Qwen3_8MoeTextConfig, prefill_config


def tiny_config():
    return Qwen3_8MoeTextConfig(vocab_size=300, hidden_size=128, num_hidden_layers=4, num_attention_heads=4,
                                num_key_value_heads=2, linear_num_key_heads=2, linear_num_value_heads=4,
                                num_experts=8, num_experts_per_tok=2, moe_intermediate_size=64,
                                shared_expert_intermediate_size=64, ngram_rows=512)


def export_and_load(model, tmp):
    from transformers import AutoModelForCausalLM

    model.save_pretrained(tmp)
    return AutoModelForCausalLM.from_pretrained(tmp, trust_remote_code=True, local_files_only=True)


def test_export_round_trip_cpu(tmp_path):
    torch.manual_seed(0)
    model = Qwen3_8MoeForCausalLM(tiny_config()).eval()
    loaded = export_and_load(model, str(tmp_path))
    files = sorted(os.listdir(tmp_path))
    assert {"config.json", "configuration_qwen3_8_moe.py", "modeling_qwen3_8_moe.py"} <= set(files)
    cfg = json.loads((tmp_path / "config.json").read_text())
    assert cfg["model_type"] == "qwen38_moe_sparse"
    assert cfg["auto_map"]["AutoModelForCausalLM"] == "modeling_qwen3_8_moe.Qwen3_8MoeForCausalLM"
    assert type(loaded).__name__ == "Qwen3_8MoeForCausalLM"
    assert type(loaded).__module__.startswith("transformers_modules.")  # the exported code, not ours
    a, b = model.state_dict(), loaded.state_dict()
    assert a.keys() == b.keys() and all(torch.equal(a[k], b[k]) for k in a)
    assert loaded.lm_head.weight.data_ptr() == loaded.model.embed_tokens.weight.data_ptr()
    mlp = loaded.model.layers[0].mlp
    assert type(mlp).__name__ == "Qwen3_8MoeSparseMoeBlock"


def test_default_config_is_config5_and_names_match_reference():
    cfg = Qwen3_8MoeTextConfig()
    assert prefill_config(cfg) == dataclasses.replace(P.c5_config(), layer_types=tuple(cfg.layer_types))
    with torch.device("meta"):
        model = Qwen3_8MoeForCausalLM(cfg)
    names = set(model.state_dict().keys())
    assert names == set(P.param_specs(P.c5_config()).keys()) | {"lm_head.weight"}


def test_forward_refuses_unsupported_inputs():
    model = Qwen3_8MoeForCausalLM(tiny_config())
    with pytest.raises(ValueError):
        model(input_ids=None)
    with pytest.raises(ValueError):
        model(input_ids=torch.zeros(1, 8, dtype=torch.long), attention_mask=torch.ones(1, 8))


@pytest.mark.gpu
def test_export_round_trip_logits_gpu(gpu, tmp_path):
    torch.manual_seed(0)
    model = Qwen3_8MoeForCausalLM(tiny_config()).eval()
    loaded = export_and_load(model, str(tmp_path))
    model = model.to(device=gpu, dtype=torch.bfloat16)
    loaded = loaded.to(device=gpu, dtype=torch.bfloat16)
    ids = P.make_ids(2, 256, P.PrefillConfig(vocab=300), seed=9, eos_every=100).to(gpu)
    with torch.inference_mode():
        a = model(input_ids=ids, output_router_logits=True)
        b = loaded(input_ids=ids, output_router_logits=True)
    assert torch.isfinite(a.logits).all()
    assert torch.equal(a.logits, b.logits)  # atol 0, as the reference's own export test
    assert torch.equal(a.aux_loss, b.aux_loss) and len(a.router_logits) == 4


@pytest.mark.gpu
def test_causal_lm_equals_prefill_on_config5(gpu):
    """The HF class and Q38Prefill run the same trunk: equal logits on the config-5 model."""
    cfg = Qwen3_8MoeTextConfig()
    params = P.init_params(P.c5_config(), 0)
    with torch.device("meta"):
        model = Qwen3_8MoeForCausalLM(cfg)
    model.load_state_dict(params, strict=True, assign=True)
    model.tie_weights()
    model = model.to(device=gpu, dtype=torch.bfloat16).eval()
    ref = P.Q38Prefill(P.c5_config()).load_params(params).to(device=gpu, dtype=torch.bfloat16)
    ids = P.make_ids(1, 512, P.c5_config(), seed=4, eos_every=200).to(gpu)
    with torch.inference_mode():
        assert torch.equal(model(input_ids=ids).logits, ref(ids))
