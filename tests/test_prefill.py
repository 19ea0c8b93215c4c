"""Packed prefill (config 5 shape): the restated Q38 trunk on the CPU.

The trunk is pinned three ways: its two reformulated pieces against their mathematical definitions
(the chunked gated delta rule against the token recurrence, block-gathered attention against dense
masked attention), and the whole 12-layer forward in fp32, with the CPU oracle in place of the HIP
MoE blocks, against the reference model's own forward (tests/golden/prefill_c5.npz, written by
tests/golden/make_prefill_golden.py from the reference with the same seeded parameters).
"""
from pathlib import Path

import numpy as np
import pytest
import torch

from oracle import moe_oracle as O
from q38 import prefill as P

GOLDEN = Path(__file__).resolve().parent / "golden" / "prefill_c5.npz"


def _recurrent_delta(q, k, v, g, beta):
    """The token-by-token gated delta rule (modeling_qwen3_8_moe.py:352-413), plain loops."""
    def l2(x):
        return x * torch.rsqrt((x * x).sum(-1, keepdim=True) + 1e-6)
    B, S, H, dk = q.shape
    qn, kn = l2(q) * dk ** -0.5, l2(k)
    st = torch.zeros(B, H, dk, v.shape[-1], dtype=torch.float64)
    out = torch.zeros(B, S, H, v.shape[-1], dtype=torch.float64)
    for t in range(S):
        st = st * g[:, t].exp()[..., None, None]
        d = (v[:, t] - (st * kn[:, t][..., None]).sum(-2)) * beta[:, t][..., None]
        st = st + kn[:, t][..., None] * d[..., None, :]
        out[:, t] = (st * qn[:, t][..., None]).sum(-2)
    return out


@pytest.mark.parametrize("n", [1, 2, 17, 64])
def test_prefix_sum_is_cpu_cumsum(n):
    """The fixed-order prefix sum in the delta rule equals torch's CPU cumsum (float64 accumulation,
    left to right) bit for bit on gate values of the DeltaNet's range and on magnitudes spread over
    2^-40 .. 2^20; a first-order (float32) doubling scan is not."""
    torch.manual_seed(n)
    g = -torch.rand(64, 7, n).exp() * torch.nn.functional.softplus(torch.randn(64, 7, n) * 4)
    wide = -torch.exp2(torch.randint(-40, 21, (64, 7, n)).float()) * torch.rand(64, 7, n)
    for t in (g, wide):
        assert torch.equal(P.prefix_sum(t), t.cumsum(-1))
    if n == 64:
        c = g.clone()
        s = 1
        while s < n:  # the same doubling in float32: a different rounding sequence
            c = torch.cat([c[..., :s], c[..., s:] + c[..., :-s]], dim=-1)
            s *= 2
        assert not torch.equal(c, g.cumsum(-1))


@pytest.mark.parametrize("S", [1, 64, 150])
def test_delta_rule_matches_recurrence(S):
    torch.manual_seed(S)
    B, H, dk, dv = 2, 3, 16, 8
    q, k = torch.randn(B, S, H, dk), torch.randn(B, S, H, dk)
    v = torch.randn(B, S, H, dv)
    g = -torch.rand(B, S, H) * 0.7
    beta = torch.rand(B, S, H)
    got = P.gated_delta_rule(q, k, v, g, beta)
    ref = _recurrent_delta(*(t.double() for t in (q, k, v, g, beta)))
    assert got.shape == (B, S, H, dv)
    assert (got.double() - ref).abs().max() < 1e-5


def test_select_blocks_invariants():
    torch.manual_seed(0)
    B, nb, budget = 2, 12, 4
    lp = torch.log_softmax(torch.randn(B, nb, nb), -1)
    sel, valid = P.select_blocks(lp, budget)
    for b in range(B):
        for qb in range(nb):
            chosen = sel[b, qb][valid[qb]].tolist()
            assert len(chosen) == min(qb + 1, budget)
            assert qb in chosen and all(0 <= c <= qb for c in chosen)
            assert len(set(chosen)) == len(chosen)
            if qb + 1 > budget:  # the others are the most probable earlier blocks
                rest = sorted(range(qb), key=lambda j: -lp[b, qb, j].item())[:budget - 1]
                assert sorted(chosen) == sorted(rest + [qb])


def test_block_sparse_attention_matches_masked_dense():
    torch.manual_seed(1)
    B, H, KV, nb, d, kk = 2, 6, 2, 10, 16, 4
    S = nb * P.BLK
    q, k, v = torch.randn(B, H, S, d), torch.randn(B, KV, S, d), torch.randn(B, KV, S, d)
    sel, valid = P.select_blocks(torch.log_softmax(torch.randn(B, nb, nb), -1), kk)
    got = P.block_sparse_attention(q, k, v, sel, valid, d ** -0.5)
    chosen = torch.zeros(B, nb, nb, dtype=torch.bool)
    for b in range(B):
        for qb in range(nb):
            chosen[b, qb, sel[b, qb][valid[qb]]] = True
    mask = chosen.repeat_interleave(P.BLK, 1).repeat_interleave(P.BLK, 2) & torch.ones(S, S, dtype=torch.bool).tril()
    kr, vr = k.repeat_interleave(H // KV, 1), v.repeat_interleave(H // KV, 1)
    s = (q.double() @ kr.double().transpose(-1, -2)) * d ** -0.5
    ref = torch.softmax(s.masked_fill(~mask[:, None], float("-inf")), -1) @ vr.double()
    assert (got.double() - ref).abs().max() < 1e-5


def test_ngram_indices_reset_after_eos():
    """An EOS starts a document: it sees no earlier token, and the tokens after it see only it and
    their own document, so their hashed rows equal those of the same tokens at a sequence start."""
    cfg = P.c5_config()
    E = cfg.eos_id
    i2, i3 = P.ngram_indices(torch.tensor([[5, 6, E, 7, 8, 9]]), cfg)
    s2, s3 = P.ngram_indices(torch.tensor([[E, 7, 8, 9]]), cfg)
    assert torch.equal(i2[0, 2:], s2[0]) and torch.equal(i3[0, 2:], s3[0])
    n2, _ = P.ngram_indices(torch.tensor([[4, E, 7, 8, 9]]), cfg)
    assert not torch.equal(i2[0, :2], n2[0, :2])  # before the EOS the history differs
    assert ((i2 >= 0) & (i2 < cfg.ngram_rows)).all() and ((i3 >= 0) & (i3 < cfg.ngram_rows)).all()


def test_golden_inputs_regenerate():
    g = np.load(GOLDEN)
    ids = P.make_ids(int(g["batch"]), int(g["seq"]), P.c5_config(), seed=int(g["ids_seed"]),
                     eos_every=int(g["eos_every"]))
    assert np.array_equal(ids.numpy(), g["ids"].astype(np.int64))


def _oracle_moe(block, x):
    """The MoE block on the CPU oracle (the reference op sequence), in x's dtype."""
    params = {n: p.to(x.device) for n, p in block.named_parameters()}
    B, S, h = x.shape
    return O.reference_block_forward(x.reshape(-1, h), params, block.gate.top_k).view(B, S, h)


def test_prefill_matches_reference_fp32():
    """Whole 12-layer trunk, fp32, CPU oracle MoE, against the reference forward."""
    g = np.load(GOLDEN)
    cfg = P.c5_config()
    model = P.Q38Prefill(cfg, moe_forward=_oracle_moe).load_params(P.init_params(cfg, int(g["seed"])))
    ids = torch.from_numpy(g["ids"].astype(np.int64))
    out = model(ids, output_router_logits=True)
    logits = out.logits
    assert logits.shape == (int(g["batch"]), int(g["seq"]), cfg.vocab) and logits.dtype == torch.float32
    # Router logits of every layer and the load-balancing loss over them (modeling:1289-1355, 1410-1427).
    assert len(out.router_logits) == cfg.layers
    assert all(r.shape == (ids.numel(), cfg.experts) for r in out.router_logits)
    assert abs(float(out.aux_loss) - float(g["aux_loss_fp32"])) < 1e-5
    lse = torch.logsumexp(logits, -1).numpy()
    assert np.abs(lse - g["lse_fp32"]).max() < 1e-5
    assert (logits.argmax(-1).numpy() == g["argmax_fp32"]).mean() > 0.999
    rows = np.stack([logits[b, s].numpy() for b, s in g["rows"]])
    ref = g["logits_fp32"]
    assert np.linalg.norm(rows - ref) / np.linalg.norm(ref) < 1e-4
    assert np.abs(rows - ref).max() < 1e-3


def test_load_balancing_loss_closed_forms():
    """k = E selects every expert in every row, so the loss is E whatever the logits; with one
    layer of identical rows the loss is E * p[top] summed over the top-k experts."""
    torch.manual_seed(3)
    E = 8
    lg = (torch.randn(50, E) * 3, torch.randn(20, E))
    assert abs(float(P.load_balancing_loss(lg, E, E)) - E) < 1e-5
    row = torch.tensor([[2.0, 1.0, 0.5, 0.0, -1.0, -2.0, -3.0, -4.0]])
    p = torch.softmax(row, -1)[0]
    got = float(P.load_balancing_loss((row.repeat(7, 1),), E, 2))
    assert abs(got - E * float(p[0] + p[1])) < 1e-5


def test_prefill_pads_to_whole_blocks():
    """A length that is not a multiple of 64 is right-padded and cut back (modeling:1236-1257)."""
    cfg = P.PrefillConfig(layers=4, hidden=128, heads=4, kv_heads=2, lin_k_heads=2, lin_v_heads=4,
                          moe_ffn=32, shared_ffn=32, experts=8, topk=2, ngram_rows=512, vocab=300)
    model = P.Q38Prefill(cfg, moe_forward=_oracle_moe).load_params(P.init_params(cfg, 3))
    ids = P.make_ids(1, 100, cfg, seed=5, eos_every=40)
    padded = torch.cat([ids, torch.full((1, 28), cfg.pad_id)], 1)
    a, b = model(ids), model(padded)
    assert a.shape == (1, 100, cfg.vocab)
    assert torch.equal(a, b[:, :100])
    with pytest.raises(ValueError):
        model(ids[:, :0])
    # Full attention layer 3 selects blocks: tokens past the budget still see their own block.
    assert torch.isfinite(a).all()


def test_param_names_match_reference_layout():
    cfg = P.c5_config()
    specs = P.param_specs(cfg)
    assert "model.layers.0.linear_attn.in_proj_qkv.weight" in specs
    assert "model.layers.3.self_attn.q_proj.weight" in specs and "model.indexers.3.wq.weight" in specs
    assert specs["model.layers.3.mlp.experts.gate_up_proj"][0] == (64, 512, 1024)
    assert specs["model.mhc.23.B.weight"][0] == (24, 128)
    model = P.Q38Prefill(cfg)
    assert set(dict(model.named_parameters()).keys()) == set(specs.keys())
    with pytest.raises(ValueError):  # the head is tied to the embedding
        P.Q38Prefill(cfg).load_params({"model.embed_tokens.weight": torch.ones(2),
                                       "lm_head.weight": torch.zeros(2)})
