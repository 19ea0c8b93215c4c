"""Packed prefill (benchmark config 5) on the GPU: the restated Q38 trunk with the fused HIP MoE block
in every layer, against the reference model's forward (tests/golden/prefill_c5.npz on 2 x 1024
tokens, tests/golden/prefill_c5_full.npz on the config-5 input itself, 4 x 4096).

Tolerances. The fp32 check runs the trunk on the GPU with the CPU oracle in place of the MoE
kernels, so it pins the GPU execution of every trunk op: logsumexp within 1e-4, stored logit rows
within 1e-3 relative L2. The bf16 check is the product path. This random-init 12-layer model
amplifies rounding noise by about 1.3x per layer: the reference's own bf16 forward is 0.26 relative
L2 away from its fp32 forward at the logits (argmax agreement ~49 %), so bf16 results are judged
against that spread: ours must be no further from the fp32 reference than 1.25x the reference's bf16
run is (logsumexp within 1.5x), and closer to the reference's bf16 run than that run is to fp32.
That spread cannot see a MoE-block error well under 10 %, so the bf16 checks also hold every one of
the twelve HIP blocks, on the inputs the trunk gave it in this very forward, to the block bar of the
bf16 path (2e-2 max-abs, 1e-2 relative L2 against the CPU oracle's block on sampled tokens).
"""
from pathlib import Path

import numpy as np
import pytest
import torch

from _util import assert_bf16_close
from oracle import moe_oracle as O
from q38 import prefill as P

pytestmark = pytest.mark.gpu
GOLDEN = Path(__file__).resolve().parent / "golden" / "prefill_c5.npz"


@pytest.fixture(scope="module")
def golden():
    return np.load(GOLDEN)


@pytest.fixture(scope="module")
def params(golden):
    return P.init_params(P.c5_config(), int(golden["seed"]))


def _rows(logits, g):
    return np.stack([logits[b, s].float().cpu().numpy() for b, s in g["rows"]])


def _bf16_rows(bits):
    return (bits.astype(np.uint32) << 16).view(np.float32)


def _record_blocks(model):
    """Keep every MoE call's input and output: the list gets one (x, y, block) per layer and forward."""
    calls = []
    inner = model._moe

    def moe(block, x, with_router):
        res = inner(block, x, with_router)
        calls.append((x.clone(), (res[0] if with_router else res).clone(), block))
        return res

    model._moe = moe
    return calls


def _assert_deterministic(logits, again, first, second):
    """Two forwards on the same ids (the first with the router-logits output, the second without)
    must agree bit for bit. On failure, say how many positions differ and the first one in each
    sequence, and name where the forwards parted: the first layer whose MoE block received different
    inputs (a trunk op diverged before it), or whose block gave different outputs for identical
    inputs (the block diverged)."""
    if torch.equal(logits, again):
        return
    diff = (logits != again).any(-1)  # [B, S]
    first_pos = [int(torch.nonzero(r)[0]) if r.any() else -1 for r in diff]
    where = "every block's input and output identical: after the last block (final norm, head)"
    for i, ((x1, y1, _), (x2, y2, _)) in enumerate(zip(first, second)):
        if not torch.equal(x1, x2):
            n = int((x1 != x2).any(-1).sum())
            where = f"layer {i}: the MoE block's input differs at {n} tokens (the trunk diverged before it)"
            break
        if not torch.equal(y1, y2):
            n = int((y1 != y2).any(-1).sum())
            where = f"layer {i}: identical block input, block output differs at {n} tokens (the block diverged)"
            break
    raise AssertionError(f"the HIP prefill must be deterministic: {int(diff.sum())} of {diff.numel()} "
                         f"positions differ; first differing position per sequence {first_pos}; {where}")


def _rel(a, b):
    return float(np.linalg.norm(a - b) / np.linalg.norm(b))


def _assert_blocks_within_bar(calls, k, samples):
    """Every recorded HIP MoE block against the CPU oracle's block (oracle.block: the reference's
    roundings, its own router) on the same bf16 inputs, at `samples` tokens spread over the packed
    sequence: the bf16 block bar (max-abs 2e-2, relative L2 1e-2), as for the standalone block."""
    assert len(calls) == 12
    for i, (x, y, block) in enumerate(calls):
        h = x.shape[-1]
        xs, ys = x.reshape(-1, h), y.reshape(-1, h)
        sel = torch.linspace(0, xs.shape[0] - 1, samples).long().to(xs.device)
        params = {n: p.detach().cpu() for n, p in block.named_parameters()}
        ref, _ = O.block(xs[sel].cpu(), params, k)
        mx, r = assert_bf16_close(ys[sel].cpu(), ref, what=f"layer {i} MoE block in the prefill")
        print(f"layer {i:2d}: block max-abs {mx:.2e} rel {r:.2e}")


def test_prefill_fp32_trunk_on_gpu(gpu, golden, params):
    def oracle_moe(block, x):
        w = {n: p.cpu() for n, p in block.named_parameters()}
        B, S, h = x.shape
        return O.reference_block_forward(x.reshape(-1, h).cpu(), w, block.gate.top_k).view(B, S, h).to(x.device)

    model = P.Q38Prefill(P.c5_config(), moe_forward=oracle_moe).load_params(params).to(gpu)
    logits = model(torch.from_numpy(golden["ids"].astype(np.int64)).to(gpu))
    assert logits.dtype == torch.float32
    lse = torch.logsumexp(logits, -1).cpu().numpy()
    assert np.abs(lse - golden["lse_fp32"]).max() < 1e-4
    assert (logits.argmax(-1).cpu().numpy() == golden["argmax_fp32"]).mean() > 0.99
    assert _rel(_rows(logits, golden), golden["logits_fp32"]) < 1e-3


def test_prefill_bf16_hip_within_reference_bf16_spread(gpu, golden, params):
    model = P.Q38Prefill(P.c5_config()).load_params(params).to(device=gpu, dtype=torch.bfloat16)
    ids = torch.from_numpy(golden["ids"].astype(np.int64)).to(gpu)
    calls = _record_blocks(model)
    with torch.inference_mode():
        out = model(ids, output_router_logits=True)
        first = list(calls)
        calls.clear()
        again = model(ids)
    logits = out.logits
    assert logits.dtype == torch.bfloat16 and torch.isfinite(logits).all()
    # The load-balancing loss over the fused blocks' router logits: within the spread the bf16 trunk
    # gives the router inputs, measured on the loss's distance from its uniform-load value k.
    k = P.c5_config().topk
    spread_aux = abs(float(golden["aux_loss_bf16"]) - float(golden["aux_loss_fp32"]))
    assert len(out.router_logits) == 12 and out.router_logits[0].dtype == torch.bfloat16
    aux_ref = float(golden["aux_loss_fp32"])
    print(f"aux loss {float(out.aux_loss):.7f} vs reference fp32 {aux_ref:.7f} (bf16 {float(golden['aux_loss_bf16']):.7f})")
    assert abs(float(out.aux_loss) - aux_ref) <= max(2 * spread_aux, 0.1 * abs(aux_ref - k))
    _assert_deterministic(logits, again, first, calls)
    _assert_blocks_within_bar(first, k, 256)
    ref32, ref16 = golden["logits_fp32"], _bf16_rows(golden["logits_bf16"])
    spread = _rel(ref16, ref32)
    spread_lse = np.abs(golden["lse_bf16"] - golden["lse_fp32"]).max()
    spread_am = (golden["argmax_bf16"] == golden["argmax_fp32"]).mean()
    ours = _rows(logits, golden)
    lse = torch.logsumexp(logits.float(), -1).cpu().numpy()
    am = logits.float().argmax(-1).cpu().numpy()
    assert _rel(ours, ref32) <= 1.25 * spread
    assert np.abs(lse - golden["lse_fp32"]).max() <= 1.5 * spread_lse
    assert (am == golden["argmax_fp32"]).mean() >= spread_am - 0.1
    assert _rel(ours, ref16) <= spread


GOLDEN_FULL = Path(__file__).resolve().parent / "golden" / "prefill_c5_full.npz"


@pytest.fixture(scope="module")
def golden_full():
    return np.load(GOLDEN_FULL)


def test_prefill_full_config5_fp32_trunk(gpu, golden_full, params):
    """The config-5 input itself (4 x 4096 packed tokens, EOS about every 1000) against the
    reference's fp32 forward on it, with the trunk on the GPU and the CPU oracle for the MoE blocks.

    Bar. On this input a few tokens sit on a near-tie between their 5th and 6th expert, and two fp32
    evaluation orders of the same forward choose differently there; the changed expert output then
    moves the rest of that packed segment a little. The restated trunk run on the CPU already does
    this against the reference's CPU forward (0.24 % of tokens beyond 1e-4 in logsumexp, in bursts
    inside segments; everything else within 1e-5), so the bar is on the bulk: the 99th percentile of
    the logsumexp difference below 1e-4, under 1 % of tokens beyond 1e-4, none beyond 1e-2, argmax
    agreement above 99 %, and the stored logit rows within 1e-3 relative L2."""
    g = golden_full
    assert g["ids"].shape == (4, 4096)
    ids = P.make_ids(4, 4096, P.c5_config())
    assert np.array_equal(ids.numpy(), g["ids"].astype(np.int64)), "golden made from another input"

    def oracle_moe(block, x):
        w = {n: p.cpu() for n, p in block.named_parameters()}
        B, S, h = x.shape
        return O.reference_block_forward(x.reshape(-1, h).cpu(), w, block.gate.top_k).view(B, S, h).to(x.device)

    model = P.Q38Prefill(P.c5_config(), moe_forward=oracle_moe).load_params(params).to(gpu)
    with torch.inference_mode():
        logits = model(ids.to(gpu))
    lse = torch.logsumexp(logits, -1).cpu().numpy()
    d = np.abs(lse - g["lse_fp32"])
    print(f"full fp32 trunk: lse diff p50 {np.percentile(d, 50):.1e} p99 {np.percentile(d, 99):.1e} max "
          f"{d.max():.1e}, beyond 1e-4: {(d > 1e-4).mean():.4f}")
    assert np.percentile(d, 99) < 1e-4
    assert (d > 1e-4).mean() < 0.01
    assert d.max() < 1e-2
    assert (logits.argmax(-1).cpu().numpy() == g["argmax_fp32"]).mean() > 0.99
    assert _rel(_rows(logits, g), g["logits_fp32"]) < 1e-3


def test_prefill_full_config5_bf16_hip(gpu, golden_full, params):
    """The product path on the config-5 input itself (4 x 4096 packed tokens, the fused HIP MoE block
    in all 12 layers): finite, deterministic, and within the reference's own bf16 spread of its fp32
    forward on this input (the bars of the 2 x 1024 check)."""
    g = golden_full
    cfg = P.c5_config()
    model = P.Q38Prefill(cfg).load_params(params).to(device=gpu, dtype=torch.bfloat16)
    ids = torch.from_numpy(g["ids"].astype(np.int64)).to(gpu)
    calls = _record_blocks(model)
    with torch.inference_mode():
        out = model(ids, output_router_logits=True)
        first = list(calls)
        calls.clear()
        again = model(ids)
    logits = out.logits
    assert logits.shape == (4, 4096, cfg.vocab)
    assert torch.isfinite(logits).all()
    _assert_deterministic(logits, again, first, calls)
    k = cfg.topk
    _assert_blocks_within_bar(first, k, 512)
    spread_aux = abs(float(g["aux_loss_bf16"]) - float(g["aux_loss_fp32"]))
    aux_ref = float(g["aux_loss_fp32"])
    assert abs(float(out.aux_loss) - aux_ref) <= max(2 * spread_aux, 0.1 * abs(aux_ref - k))
    ref32, ref16 = g["logits_fp32"], _bf16_rows(g["logits_bf16"])
    spread = _rel(ref16, ref32)
    spread_lse = np.abs(g["lse_bf16"] - g["lse_fp32"]).max()
    spread_am = (g["argmax_bf16"] == g["argmax_fp32"]).mean()
    ours = _rows(logits, g)
    lse = torch.logsumexp(logits.float(), -1).cpu().numpy()
    am = logits.float().argmax(-1).cpu().numpy()
    print(f"full bf16: rows rel {_rel(ours, ref32):.3f} (reference bf16 {spread:.3f}), lse max diff "
          f"{np.abs(lse - g['lse_fp32']).max():.3f} (reference bf16 {spread_lse:.3f}), argmax agreement "
          f"{(am == g['argmax_fp32']).mean():.3f} (reference bf16 {spread_am:.3f})")
    assert _rel(ours, ref32) <= 1.25 * spread
    assert np.abs(lse - g["lse_fp32"]).max() <= 1.5 * spread_lse
    assert (am == g["argmax_fp32"]).mean() >= spread_am - 0.1
    assert _rel(ours, ref16) <= spread
