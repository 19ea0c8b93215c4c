"""GPU parity of the router (R1-R2): routing indices and renormalised weights bit-exact against
the CPU oracle.

The oracle is torch's CPU top-k restated in oracle/q38_oracle.cpp (libstdc++ nth_element/sort,
ATen/native/TopKImpl.h:45-76) applied to torch's CPU fp32 softmax of the same bf16 logits (plus
the optional fp32 bias), renormalised by torch's sum and division. The kernel computes the same
fp32 probabilities bit for bit, so rows whose distinct logits collapse to equal probabilities
(collision rows below) tie exactly where the CPU's do.
"""
import numpy as np
import pytest
import torch

from _util import (assert_gemm_bf16_rounding, bf16_ulp_diff, collision_bias, collision_bias_logits,
                   collision_logits)
from oracle import moe_oracle as orc

pytestmark = pytest.mark.gpu


def _ops():
    from q38.hip import ops
    return ops


def _check_selection(logits, k, gpu, bias=None):
    ops = _ops()
    idx, w, hist = ops.route_from_logits(logits.to(gpu), k,
                                         logit_bias=None if bias is None else bias.to(gpu), want_hist=True)
    torch.cuda.synchronize()
    _, _, ridx, rw = orc.router(None, None, k, logit_bias=bias, logits=logits)
    idx = idx.cpu().long()
    bad = (idx != ridx).any(dim=1)
    assert int(bad.sum()) == 0, f"{int(bad.sum())} rows differ; first: {torch.nonzero(bad)[:5].flatten().tolist()}"
    # Renormalised weights: the same fp32 probabilities, sum and division, so identical bits.
    assert int(bf16_ulp_diff(w.cpu(), rw).max()) == 0
    T, E = logits.shape
    # Histogram of 64-token blocks.
    ref_hist = torch.zeros((T + 63) // 64, E, dtype=torch.int64)
    blk = torch.arange(T).repeat_interleave(k) // 64
    ref_hist.index_put_((blk, ridx.reshape(-1)), torch.ones(T * k, dtype=torch.int64), accumulate=True)
    assert torch.equal(hist.cpu().long(), ref_hist)


@pytest.mark.parametrize("T,E,k,scale,seed", [
    (16384, 64, 5, 0.64, 0),   # config-2 logit scale (x ~ N(0,1), h=1024, W ~ N(0,0.02))
    (2048, 64, 5, 0.32, 1),    # config-1 logit scale
    (1000, 8, 3, 1.0, 2),      # the reference's parity-script routing shape (E=8, k=3)
    (777, 64, 8, 0.5, 3),      # k = 8, ragged T
    (129, 17, 4, 0.5, 4),      # E not a multiple of 16
    (40001, 64, 5, 0.64, 5),   # more 64-token blocks than CUs: 128-token blocks, ragged last block
    (33000, 17, 4, 0.5, 6),    # the same with E not a multiple of 16
    (20001, 64, 8, 0.5, 7),    # and k = 8
])
def test_route_from_logits_random(gpu, T, E, k, scale, seed):
    g = torch.Generator().manual_seed(seed)
    logits = (torch.randn(T, E, generator=g) * scale).to(torch.bfloat16)
    _check_selection(logits, k, gpu)


@pytest.mark.parametrize("levels,seed", [(6, 10), (3, 11), (2, 12), (1, 13)])
def test_route_from_logits_ties(gpu, levels, seed):
    """Tie-heavy rows: integer-valued logits in [0, levels); exercises the libstdc++ replay."""
    g = torch.Generator().manual_seed(seed)
    logits = torch.randint(0, levels, (8192, 64), generator=g).to(torch.bfloat16)
    _check_selection(logits, 5, gpu)


def test_route_known_answer(gpu):
    """[.1,.5,.5,.2,.5,.5,.5,0] top-5 -> [1,6,5,4,2] on torch CPU (not index order)."""
    vals = torch.tensor([[0.1, 0.5, 0.5, 0.2, 0.5, 0.5, 0.5, 0.0]]).log().to(torch.bfloat16)
    ops = _ops()
    idx, _, _ = ops.route_from_logits(vals.to(gpu), 5)
    assert idx.cpu().tolist() == [[1, 6, 5, 4, 2]]


def test_route_partial_sort_path(gpu):
    """k*64 <= E (k=1, E=64): torch takes std::partial_sort -> lowest-index maximum."""
    g = torch.Generator().manual_seed(5)
    logits = torch.randint(0, 3, (4096, 64), generator=g).to(torch.bfloat16)
    _check_selection(logits, 1, gpu)


def test_route_special_rows(gpu):
    T, E = 64, 64
    logits = torch.zeros(T, E)
    logits[1, 7] = float("nan")               # softmax row all NaN -> all tied
    logits[2, :] = float("-inf")              # all -inf -> NaN row
    logits[3, 5] = float("inf")
    logits[4, :] = -0.0                       # signed zeros tie with +0
    logits[4, ::2] = 0.0
    logits[5, :] = torch.arange(E, dtype=torch.float32)  # strictly increasing
    logits[6, :] = -torch.arange(E, dtype=torch.float32)
    logits = logits.to(torch.bfloat16)
    ops = _ops()
    idx, w, _ = ops.route_from_logits(logits.to(gpu), 5)
    _, probs, ridx, rw = orc.router(None, None, 5, logits=logits)
    assert torch.equal(idx.cpu().long(), ridx)
    # Rows with finite softmax: weights match within 1 ulp; NaN rows are NaN in both.
    wn, rn = w.cpu().float(), rw.float()
    assert torch.equal(torch.isnan(wn), torch.isnan(rn))
    fin = ~torch.isnan(rn)
    assert int(bf16_ulp_diff(w.cpu()[fin], rw[fin]).max()) == 0


def test_route_with_bias(gpu):
    """Routing-skew bias added to the logits before the softmax (configuration 3)."""
    g = torch.Generator().manual_seed(21)
    logits = (torch.randn(4096, 64, generator=g) * 0.64).to(torch.bfloat16)
    ranks = torch.from_numpy(np.random.RandomState(7).permutation(64) + 1).double()
    bias = (-1.2 * ranks.log()).float()
    _check_selection(logits, 5, gpu, bias=bias)


@pytest.mark.parametrize("E,k", [(64, 5), (64, 8), (17, 4), (8, 3)])
def test_route_collision_logits(gpu, E, k):
    """Distinct tiny logits next to logits at 1.0: x - max rounds the tiny ones to one fp32 value,
    so their probabilities tie and torch's top-k picks among them by introselect position (a
    selection on the logits would take the largest)."""
    _check_selection(collision_logits(4096, E=E, k=k, seed=E + k), k, gpu)


@pytest.mark.parametrize("E,k", [(64, 5), (64, 7), (17, 5)])
def test_route_collision_bias(gpu, E, k):
    """Biased logits a few fp32 ulps apart: exp() and the 1/sum scaling merge neighbours into
    equal probabilities, which only an exact restatement of the CPU softmax reproduces."""
    bias = collision_bias(E=E, seed=k)
    _check_selection(collision_bias_logits(4096, E=E, seed=k), k, gpu, bias=bias)


@pytest.mark.parametrize("T", [16384, 40001])
def test_route_logits_output_on_tied_rows(gpu, T):
    """The logits output with most rows tied: 0/1 activations and router weights make every logit
    an exact small integer (the MFMA sums are exact and bf16 holds them), so nearly every row ties
    within its top k + 1 and takes the replay, whose probabilities replace the row's logits in LDS.
    The logits written out must still be the exact integers, and the selection exact on them, on
    each of several launches (T = 40001 runs 128-token blocks)."""
    ops = _ops()
    g = torch.Generator().manual_seed(T)
    h, E, k = 256, 64, 5
    x = (torch.rand(T, h, generator=g) < 0.5).to(torch.bfloat16)
    wr = (torch.rand(E, h, generator=g) < 0.1).to(torch.bfloat16)
    ws = (torch.rand(1, h, generator=g) < 0.1).to(torch.bfloat16)
    exact = (x.double() @ wr.double().T).to(torch.bfloat16)
    gate_exact = (x.double() @ ws.double().reshape(-1)).to(torch.bfloat16)
    top = exact.float().topk(k + 1, dim=1).values
    tied = (top[:, 1:] == top[:, :-1]).any(dim=1)
    assert float(tied.float().mean()) > 0.9
    _, _, ridx, rw = orc.router(None, None, k, logits=exact)
    xg, wg, wsg = x.to(gpu), wr.to(gpu), ws.to(gpu)
    for rep in range(4):
        logits, idx, w, gate, _ = ops.route(xg, wg, k, w_shared_gate=wsg, want_logits=True, want_hist=True)
        torch.cuda.synchronize()
        assert torch.equal(logits.cpu(), exact), f"launch {rep}: router logits output differs"
        assert torch.equal(gate.cpu().reshape(-1), gate_exact), f"launch {rep}: shared gate logit differs"
        assert torch.equal(idx.cpu().long(), ridx), f"launch {rep}: indices differ"
        assert torch.equal(w.cpu(), rw), f"launch {rep}: weights differ"


@pytest.mark.parametrize("wl_name,T", [("c1", 2048), ("c2", 16384), ("c2", 20000), ("c2", 33333)])
def test_route_full(gpu, wl_name, T):
    """Logits GEMM on MFMA: within 1 bf16 ulp of the fp32 reference; selection exact on them.
    T = 20000 and 33333 (more 64-token blocks than CUs) run 128-token blocks, the last one ragged
    (33333: its second 64-token half lies past T and has no histogram row)."""
    from q38 import workloads
    wl = workloads.get(wl_name)
    x, params, _ = workloads.make(wl, tokens=T)
    ops = _ops()
    wr = params["gate.weight"]
    ws = params["shared_expert_gate.weight"]
    logits, idx, w, gate, hist = ops.route(x.to(gpu), wr.to(gpu), wl.topk, w_shared_gate=ws.to(gpu),
                                           want_logits=True, want_hist=True)
    torch.cuda.synchronize()
    ref_logits = orc.bf16(x.float() @ wr.float().T)
    assert_gemm_bf16_rounding(logits, x, wr, "router logits")
    assert_gemm_bf16_rounding(gate, x, ws, "shared gate logit")
    # Without the logits output the kernel gives the same indices, weights and histogram; the
    # histogram holds each 64-token block's expert counts.
    _, idx2, w2, _, hist2 = ops.route(x.to(gpu), wr.to(gpu), wl.topk, w_shared_gate=ws.to(gpu),
                                      want_logits=False, want_hist=True)
    assert torch.equal(idx2, idx) and torch.equal(w2, w) and torch.equal(hist2, hist)
    blk = torch.arange(T).repeat_interleave(wl.topk) // 64
    ref_hist = torch.zeros_like(hist.cpu()).index_put_((blk, idx.cpu().long().flatten()), torch.tensor(1, dtype=torch.int32), accumulate=True)
    assert torch.equal(hist.cpu(), ref_hist)
    # Selection is a function of the logits: exact against the oracle on the GPU logits.
    _, _, ridx, rw = orc.router(None, None, wl.topk, logits=logits.cpu())
    assert torch.equal(idx.cpu().long(), ridx)
    assert torch.equal(w.cpu(), rw)
    # End to end against CPU-computed logits: every differing row must trace to a 1-ulp logit
    # difference (report, do not hide, the count).
    _, _, eidx, _ = orc.router(x, wr, wl.topk)
    rows = (idx.cpu().long() != eidx).any(dim=1)
    if rows.any():
        assert (logits.cpu()[rows] != ref_logits[rows]).any(dim=1).all()
    print(f"{wl_name}: {int(rows.sum())} of {T} rows route differently from CPU-computed logits")
