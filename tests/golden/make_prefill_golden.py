"""Golden vectors for the Q38 packed prefill (benchmark config 5 shape).

Runs the reference model's own forward (Qwen3_8MoeForCausalLM, q38/models/qwen3_8_moe/
modeling_qwen3_8_moe.py) on the CPU, with the seeded parameters of ``q38.prefill.init_params``
loaded by name, on ``q38.prefill.make_ids`` input, in fp32 and in bf16. Only this script imports
the reference, and only in the build container where the checkout lives at /root/reference; the
tests read the vectors it writes (prefill_c5.npz), never the reference.

Each run asks for ``output_router_logits`` and also stores the load-balancing loss the reference
computes over the layers' router logits (modeling:1410-1427). The bf16 run casts the reference
model with ``.to(torch.bfloat16)`` and then puts the rotary inverse-frequency buffers back in fp32,
as a model loaded with ``from_pretrained(dtype=bf16)`` (q38/evaluate.py:185) keeps them.

Usage: python tests/golden/make_prefill_golden.py [--batch 2 --seq 1024] [--debug /tmp/dump.pt]
       python tests/golden/make_prefill_golden.py --batch 4 --seq 4096 --eos-every 1000 --full-rows \
           --out tests/golden/prefill_c5_full.npz      (the configuration-5 input itself)
"""
import argparse
import importlib.util
import sys
import time
from pathlib import Path

import numpy as np
import torch

REF = Path("/root/reference")
REPO = Path(__file__).resolve().parents[2]
sys.path.insert(0, str(REPO / "qwen35-moe-sparse_amd"))
from q38 import prefill as P  # noqa: E402

OUT = Path(__file__).resolve().parent / "prefill_c5.npz"
# (batch row, position) pairs whose full logit rows are stored.
ROWS = ((0, 0), (0, 301), (0, 1023), (1, 64), (1, 640), (1, 1000))
# For the full configuration-5 input (4 x 4096): rows in every sequence, late positions included.
ROWS_FULL = ((0, 0), (0, 1023), (1, 2047), (2, 3000), (3, 4000), (3, 4095))


def reference_package():
    pkg = REF / "q38" / "models" / "qwen3_8_moe"
    spec = importlib.util.spec_from_file_location("ref_qwen3_8_moe", pkg / "__init__.py",
                                                  submodule_search_locations=[str(pkg)])
    mod = importlib.util.module_from_spec(spec)
    sys.modules["ref_qwen3_8_moe"] = mod
    spec.loader.exec_module(mod)
    return mod


def reference_config(mod, c):
    """The reference text config for PrefillConfig c (fields of q38/presets.py:59-83), no MTP head."""
    cfg = mod.Qwen3_8MoeTextConfig(
        vocab_size=c.vocab, hidden_size=c.hidden, num_hidden_layers=c.layers,
        num_attention_heads=c.heads, num_key_value_heads=c.kv_heads, head_dim=c.head_dim,
        linear_num_key_heads=c.lin_k_heads, linear_num_value_heads=c.lin_v_heads,
        linear_key_head_dim=c.lin_head_dim, linear_value_head_dim=c.lin_head_dim,
        linear_conv_kernel_dim=c.conv_kernel, num_experts=c.experts, num_experts_per_tok=c.topk,
        moe_intermediate_size=c.moe_ffn, shared_expert_intermediate_size=c.shared_ffn,
        output_router_logits=False, layer_types=[c.layer_kind(i) for i in range(c.layers)],
        max_position_embeddings=4096, rms_norm_eps=c.rms_eps,
        rope_parameters={"rope_type": "default", "rope_theta": c.rope_theta,
                         "partial_rotary_factor": c.partial_rotary},
        partial_rotary_factor=c.partial_rotary, tie_word_embeddings=True, attention_bias=False,
        initializer_range=0.02, bos_token_id=c.eos_id, eos_token_id=c.eos_id, pad_token_id=c.pad_id)
    cfg.n_branch, cfg.mhc_iters, cfg.qsa_blocks = c.n_branch, c.mhc_iters, c.qsa_blocks
    cfg.indexer_heads, cfg.indexer_head_dim = c.indexer_heads, c.indexer_head_dim
    cfg.mtp = False
    cfg.ngram_rows = c.ngram_rows
    cfg.use_cache = False
    cfg._attn_implementation = "sdpa"
    return cfg


def bf16_bits(t):
    return t.to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)


def run(model, ids, debug):
    layers_out = []
    if debug:
        inner = model.model._layer

        def recording(i, X, *a):
            X, kl = inner(i, X, *a)
            layers_out.append(X.sum(2).float().clone())
            return X, kl
        model.model._layer = recording
    t = time.time()
    with torch.no_grad():
        out = model(input_ids=ids, use_cache=False, output_router_logits=True)
    print(f"  forward {time.time() - t:.1f} s, aux_loss {float(out.aux_loss):.8f}", flush=True)
    if debug:
        model.model._layer = inner
    return out.logits, float(out.aux_loss), layers_out


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--batch", type=int, default=2)
    ap.add_argument("--seq", type=int, default=1024)
    ap.add_argument("--eos-every", type=int, default=300)
    ap.add_argument("--seed", type=int, default=0)
    ap.add_argument("--ids-seed", type=int, default=1234)
    ap.add_argument("--debug", default=None, help="also save per-layer stream sums here (torch.save)")
    ap.add_argument("--out", default=str(OUT))
    ap.add_argument("--full-rows", action="store_true", help="store the ROWS_FULL logit rows (4 x 4096 input)")
    args = ap.parse_args()
    rows = ROWS_FULL if args.full_rows else ROWS
    out_path = Path(args.out)
    torch.manual_seed(0)
    c = P.c5_config()
    params = P.init_params(c, args.seed)
    ids = P.make_ids(args.batch, args.seq, c, seed=args.ids_seed, eos_every=args.eos_every)
    mod = reference_package()
    model = mod.Qwen3_8MoeForCausalLM(reference_config(mod, c)).eval()
    model.load_state_dict(params, strict=True)
    out = dict(batch=args.batch, seq=args.seq, eos_every=args.eos_every, seed=args.seed,
               ids_seed=args.ids_seed, ids=ids.numpy().astype(np.int32), rows=np.array(rows, dtype=np.int32))
    dumps = {}
    print("reference fp32", flush=True)
    logits, aux, layers = run(model, ids, args.debug)
    lf = logits.float()
    out["aux_loss_fp32"] = np.float64(aux)
    out["lse_fp32"] = torch.logsumexp(lf, -1).numpy()
    out["argmax_fp32"] = lf.argmax(-1).numpy().astype(np.int32)
    out["logits_fp32"] = np.stack([lf[b, s].numpy() for b, s in rows])
    dumps["fp32"] = layers
    print("reference bf16", flush=True)
    model = model.to(torch.bfloat16)
    for m in model.modules():  # fp32 rotary tables, as from_pretrained(dtype=bf16) leaves them
        if hasattr(m, "inv_freq") and hasattr(m, "compute_default_rope_parameters"):
            m.inv_freq = m.compute_default_rope_parameters(m.config)[0]
    logits, aux, layers = run(model, ids, args.debug)
    lf = logits.float()
    out["aux_loss_bf16"] = np.float64(aux)
    out["lse_bf16"] = torch.logsumexp(lf, -1).numpy()
    out["argmax_bf16"] = lf.argmax(-1).numpy().astype(np.int32)
    out["logits_bf16"] = np.stack([bf16_bits(logits[b, s]) for b, s in rows])
    dumps["bf16"] = layers
    np.savez_compressed(out_path, **out)
    print("wrote", out_path, out_path.stat().st_size, "bytes")
    if args.debug:
        torch.save(dumps, args.debug)


if __name__ == "__main__":
    main()
