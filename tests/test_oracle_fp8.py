"""The fp8 oracle (R14: this repository's e4m3 definition; the reference has no fp8), pinned on
the CPU: the e4m3 rounding against an independent table-driven round-to-nearest-even over all
256 codes, the per-row scale and saturation, and the fake-quant block against the bf16 block."""
import numpy as np
import pytest
import torch

from oracle import moe_oracle as orc


def _e4m3_table():
    """Values of the 256 OCP e4m3 codes (1 sign, 4 exponent bits with bias 7, 3 mantissa bits;
    exponent 0 subnormal; S.1111.111 is NaN, so the largest finite value is 1.75 * 2^8 = 448)."""
    vals = np.empty(256, dtype=np.float64)
    for c in range(256):
        s, e, m = c >> 7, (c >> 3) & 15, c & 7
        if e == 15 and m == 7:
            vals[c] = np.nan
            continue
        mag = (m / 8.0) * 2.0 ** -6 if e == 0 else (1 + m / 8.0) * 2.0 ** (e - 7)
        vals[c] = -mag if s else mag
    return vals


def _rne_e4m3(x):
    """Nearest finite e4m3 code by brute force, ties to the even mantissa (inputs within +-448)."""
    vals = _e4m3_table()
    codes = np.arange(256)
    fin = ~np.isnan(vals)
    out = np.empty(x.shape, dtype=np.uint8)
    for i, v in enumerate(x.ravel()):
        d = np.abs(vals[fin] - v)
        best = np.flatnonzero(d == d.min())
        cand = codes[fin][best]
        if len(cand) > 1:  # a tie: the even mantissa wins
            even = cand[(cand & 1) == 0]
            cand = even if len(even) else cand
        if (cand[0] & 127) == 0:  # a zero result keeps the sign of v
            cand = [0x80 if np.signbit(v) else 0x00]
        out.ravel()[i] = cand[0]
    return out


def test_e4m3_rounding_matches_table():
    vals = _e4m3_table()
    fin = vals[~np.isnan(vals)]
    pos = np.unique(np.abs(fin))
    mids = (pos[1:] + pos[:-1]) / 2           # exact ties between neighbours
    rng = np.random.RandomState(3)
    x = np.concatenate([fin, mids, -mids, rng.uniform(-448, 448, 3000), rng.uniform(-0.02, 0.02, 2000),
                        [448.0, -448.0, 2.0 ** -9, 2.0 ** -10, 3 * 2.0 ** -11]]).astype(np.float32)
    got = torch.from_numpy(x).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    want = _rne_e4m3(x.astype(np.float64))
    assert (got == want).all(), x[got != want][:10]


def test_quant_rows_scale_and_saturation():
    g = torch.Generator().manual_seed(5)
    x = (torch.randn(64, 256, generator=g) * torch.logspace(-3, 3, 64)[:, None]).to(torch.bfloat16)
    x[3] = 0
    q, s = orc.quant_e4m3_rows(x)
    xf = x.float()
    amax = xf.abs().amax(dim=1)
    assert torch.equal(s, amax / 448.0)
    v = orc.e4m3_value(q)
    assert v.abs().max() <= 448
    # each row's largest element lands on +-448 (the clamp absorbs x*inv rounding above 448)
    big = xf.abs().argmax(dim=1)
    rows = torch.arange(64)
    nz = amax > 0
    assert torch.equal(v[rows[nz], big[nz]].abs(), torch.full((int(nz.sum()),), 448.0))
    assert torch.equal(q[3], torch.zeros(256, dtype=torch.uint8))
    # relative error of e4m3 with 3 mantissa bits: at most half an ulp (2^-4) of the value
    deq = v * s[:, None]
    err = (deq - xf).abs()
    tol = xf.abs() * 2.0 ** -4 + s[:, None] * 2.0 ** -10  # half an ulp; subnormals: half of 2^-9
    assert (err <= tol).all()


def test_block_fp8_close_to_bf16_block():
    """Fake-quant fp8 block vs the bf16 block on a small seeded layer: e4m3 operands keep the
    output within a few percent (relative L2) of bf16."""
    from q38 import workloads
    wl = workloads.get("c1")
    x, params, _ = workloads.make(wl, tokens=256)
    x = x.to(torch.bfloat16)
    params = {n: p.to(torch.bfloat16) for n, p in params.items()}
    wq = orc.quant_weights_fp8(params)
    out8, inter = orc.block_fp8(x, params, wq, wl.topk)
    out, _ = orc.block(x, params, wl.topk)
    rel = float((out8.float() - out.float()).norm() / out.float().norm())
    assert rel < 0.08, rel
    # routing is bf16 in both
    assert torch.equal(inter["idx"], orc.router(x, params["gate.weight"], wl.topk)[2])
