"""The fp8 oracle (R14: this repository's e4m3 definition; the reference has no fp8), pinned on
the CPU:

* the e4m3 rounding against an independent table-driven round-to-nearest-even over all 256 codes,
  and the per-row scale and saturation;
* experts_fp8 against a per-token float64 brute force from the e4m3 codes and scales (no
  permutation, no shared code with the oracle beyond the pinned quantiser), stage by stage: H
  within one bf16 rounding on significant elements, Y one rounding of the exact product, out one
  rounding of the float64 assembly;
* on operands that quantise exactly (power-of-two scales), the fp8 gate/up stage equals the bf16
  oracle's, which float64 brute force pins separately;
* three scale-algebra mistakes planted in the oracle (gate/up channel scales swapped, token scale
  taken by sorted row, shared down rows with another row's scale) each fail the brute force;
* block_fp8 = the bf16 router and gate logit, then experts_fp8."""
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


def _bf16_ulps(a, b):
    """|ordinal(a) - ordinal(b)| of bf16 values (0 = identical bits)."""
    def ordinal(t):
        u = t.contiguous().view(torch.int16).to(torch.int32) & 0xFFFF
        return torch.where(u >= 0x8000, 0x8000 - u, u)
    return (ordinal(a.to(torch.bfloat16)) - ordinal(b.to(torch.bfloat16))).abs()


def _lossless_rows(rng, rows, cols, exp_lo, exp_hi):
    """bf16 rows that per-row e4m3 quantisation represents exactly: e4m3 code values (finite codes,
    random signs) with one element of each row at +-448, times 2^a per row (a in [exp_lo, exp_hi]).
    Returns (x bf16, codes' values fp64, 2^a fp64)."""
    vals = _e4m3_table()
    fin = np.flatnonzero(~np.isnan(vals) & (np.arange(256) < 128) & (np.arange(256) > 0))
    codes = rng.choice(fin, size=(rows, cols))
    v = vals[codes] * rng.choice([-1.0, 1.0], size=(rows, cols))
    v[np.arange(rows), rng.randint(0, cols, rows)] = 448.0 * rng.choice([-1.0, 1.0], size=rows)
    scale = 2.0 ** rng.randint(exp_lo, exp_hi + 1, size=rows)
    x = torch.from_numpy(v * scale[:, None]).to(torch.bfloat16)
    assert torch.equal(x.double(), torch.from_numpy(v * scale[:, None]))  # exact in bf16
    return x, v, scale


def _fp8_inputs(lossless, seed=0, T=37, h=128, E=8, k=3, I=64):
    """Tiny fp8 layer: x [T,h], weights, routing and shared-gate logits. lossless=True builds every
    quantised operand so that per-row e4m3 quantisation is exact (power-of-two scales); otherwise
    N(0,1) tokens and N(0,0.02) weights."""
    rng = np.random.RandomState(seed)
    if lossless:
        # magnitudes like the N(0,1) / N(0,0.02) layers: |x| <= 448 * 2^-6, |W| <= 448 * 2^-13
        x, _, _ = _lossless_rows(rng, T, h, -9, -6)
        gu, _, _ = _lossless_rows(rng, E * 2 * I, h, -16, -13)
        dn, _, _ = _lossless_rows(rng, E * h, I, -16, -13)
        sg, _, _ = _lossless_rows(rng, I, h, -16, -13)
        su, _, _ = _lossless_rows(rng, I, h, -16, -13)
        sd, _, _ = _lossless_rows(rng, h, I, -16, -13)
        gu, dn = gu.reshape(E, 2 * I, h), dn.reshape(E, h, I)
    else:
        def nrm(*s, std=0.02):
            return torch.from_numpy(rng.randn(*s) * std).to(torch.bfloat16)
        x = nrm(T, h, std=1.0)
        gu, dn, sg, su, sd = nrm(E, 2 * I, h), nrm(E, h, I), nrm(I, h), nrm(I, h), nrm(h, I)
    params = {"experts.gate_up_proj": gu, "experts.down_proj": dn, "shared_expert.gate_proj.weight": sg,
              "shared_expert.up_proj.weight": su, "shared_expert.down_proj.weight": sd}
    # Routing: distinct experts per token, random bf16 weights; token 0 uses the last experts.
    idx = torch.from_numpy(np.stack([rng.permutation(E)[:k] for _ in range(T)])).long()
    idx[0] = torch.arange(E - k, E)
    w = torch.from_numpy(rng.uniform(0.05, 0.6, (T, k))).to(torch.bfloat16)
    gate_logit = torch.from_numpy(rng.randn(T)).to(torch.bfloat16)
    return x, params, idx, w, gate_logit


def _brute_force_fp8(x, wq, idx, w, gate_logit):
    """experts_fp8 restated per token in float64 from the e4m3 codes and their scales: each
    operand dequantised as code * row scale (per token) and code * channel scale (per output
    channel); one bf16 rounding at each point of inference:90-96 (g, u, silu(g), h), h quantised
    per row, down rounded to bf16; no permutation (pair p = t*k + j maps to its sorted row by a
    stable argsort of the expert ids). Returns (H [P+T,I], Y [P+T,h], out [T,h]) and the bounds'
    magnitudes for the two GEMM stages."""
    T, h = x.shape
    k = idx.shape[1]
    qg, sg = wq["experts.gate_up_proj"]
    qd, sd = wq["experts.down_proj"]
    E, twoI, _ = qg.shape
    I = twoI // 2
    P = T * k
    xq, sx = orc.quant_e4m3_rows(x)
    X = orc.e4m3_value(xq).double() * sx.double()[:, None]        # per-token scale
    Wg = orc.e4m3_value(qg).double() * sg.double()[..., None]     # per-channel scales
    Wd = orc.e4m3_value(qd).double() * sd.double()[..., None]
    ids = idx.reshape(-1).numpy()
    sorted_row = np.empty(P, np.int64)
    sorted_row[np.argsort(ids, kind="stable")] = np.arange(P)
    H = torch.zeros(P + T, I, dtype=torch.bfloat16)
    gu_exact = torch.zeros(P + T, 2 * I, dtype=torch.float64)
    gu_mag = torch.zeros(P + T, 2 * I, dtype=torch.float64)

    def swiglu(xrow, Wgate, Wup):
        g64, u64 = Wgate @ xrow, Wup @ xrow
        g = g64.to(torch.bfloat16).double()
        u = u64.to(torch.bfloat16).double()
        act = (g / (1.0 + torch.exp(-g))).to(torch.bfloat16).double()
        mag = torch.cat([Wgate.abs() @ xrow.abs(), Wup.abs() @ xrow.abs()])
        return (act * u).to(torch.bfloat16), torch.cat([g64, u64]), mag

    def deq(name):
        q, s = wq[name]
        return orc.e4m3_value(q).double() * s.double()[:, None]
    Sg, Su, Sd = deq("shared_expert.gate_proj.weight"), deq("shared_expert.up_proj.weight"), deq(
        "shared_expert.down_proj.weight")
    for t in range(T):
        for j in range(k):
            e, r = int(idx[t, j]), int(sorted_row[t * k + j])
            H[r], gu_exact[r], gu_mag[r] = swiglu(X[t], Wg[e, :I], Wg[e, I:])
        H[P + t], gu_exact[P + t], gu_mag[P + t] = swiglu(X[t], Sg, Su)
    Hq, sH = orc.quant_e4m3_rows(H)
    Hd = orc.e4m3_value(Hq).double() * sH.double()[:, None]       # per-row scale of each H row
    Y_exact = torch.zeros(P + T, h, dtype=torch.float64)
    Y_mag = torch.zeros(P + T, h, dtype=torch.float64)
    for t in range(T):
        for j in range(k):
            e, r = int(idx[t, j]), int(sorted_row[t * k + j])
            Y_exact[r], Y_mag[r] = Wd[e] @ Hd[r], Wd[e].abs() @ Hd[r].abs()
        Y_exact[P + t], Y_mag[P + t] = Sd @ Hd[P + t], Sd.abs() @ Hd[P + t].abs()
    return dict(H=H, gu_exact=gu_exact, gu_mag=gu_mag, Y_exact=Y_exact, Y_mag=Y_mag, sorted_row=sorted_row)


def _rounding_ok(actual, exact, mag):
    """actual (bf16) is one rounding of the float64 value `exact`: within one bf16 ulp of it plus
    an fp32-accumulation allowance of 2^-20 * (sum of |terms|)."""
    e = exact.abs().clamp_min(1e-38)
    ulp = torch.pow(2.0, torch.floor(torch.log2(e)) - 7)
    return not bool(((actual.double() - exact).abs() > ulp + mag * 2.0 ** -20).any())


def _fp8_failures(x, params, idx, w, gate_logit, out, inter):
    """Stages of an experts_fp8 result (out, inter) that disagree with the float64 brute force of
    the true quantisation: [] when H, Y and out all agree."""
    T, h = x.shape
    k = idx.shape[1]
    P = T * k
    wq = orc.quant_weights_fp8(params)
    bf = _brute_force_fp8(x, wq, idx, w, gate_logit)
    fails = []
    # H: one bf16 rounding sequence of the exact computation; fp32 summation order may flip a
    # rounding of g or u in a small fraction of elements.
    # Only significant elements count: where the gate and up sums exceed 2^-12 of their terms'
    # magnitude, fp32 accumulation moves them by less than a bf16 ulp.
    I = inter["H"].shape[1]
    signif = bf["gu_exact"].abs() >= bf["gu_mag"] * 2.0 ** -12
    signif = signif[:, :I] & signif[:, I:]
    ulps = _bf16_ulps(inter["H"], bf["H"])[signif]
    if int(ulps.max()) > 1 or float((ulps > 0).float().mean()) >= 0.01:
        fails.append(f"H: max {int(ulps.max())} ulp, {float((ulps > 0).float().mean()):.4f} differ")
    # Y: one bf16 rounding of the exact product of the result's own H rows, quantised by the true
    # quantiser (per-row scale of each H row, per-channel scale of each weight row).
    Hq, sH = orc.quant_e4m3_rows(inter["H"])
    Hd = orc.e4m3_value(Hq).double() * sH.double()[:, None]
    qd, sd = wq["experts.down_proj"]
    Wd = orc.e4m3_value(qd).double() * sd.double()[..., None]
    qs, ss = wq["shared_expert.down_proj.weight"]
    Sd = orc.e4m3_value(qs).double() * ss.double()[:, None]
    rowof = bf["sorted_row"]
    Y_exact = torch.zeros(P + T, h, dtype=torch.float64)
    Y_mag = torch.zeros_like(Y_exact)
    for t in range(T):
        for j in range(k):
            e, r = int(idx[t, j]), int(rowof[t * k + j])
            Y_exact[r], Y_mag[r] = Wd[e] @ Hd[r], Wd[e].abs() @ Hd[r].abs()
        Y_exact[P + t], Y_mag[P + t] = Sd @ Hd[P + t], Sd.abs() @ Hd[P + t].abs()
    if not _rounding_ok(inter["Y"], Y_exact, Y_mag):
        fails.append("Y")
    # out: float64 assembly from the result's Y rows: pair rows weighted (bf16 rounding), k-sum
    # rounded once, then the sigmoid-gated shared row (modeling:831-833).
    Yf = inter["Y"].double()
    routed = torch.zeros(T, h, dtype=torch.float64)
    for t in range(T):
        for j in range(k):
            routed[t] += (Yf[rowof[t * k + j]] * float(w[t, j])).to(torch.bfloat16).double()
    routed = routed.to(torch.bfloat16).double()
    sig = torch.sigmoid(gate_logit.double()).to(torch.bfloat16).double()
    ref_out = routed + (sig[:, None] * Yf[P:]).to(torch.bfloat16).double()
    if int(_bf16_ulps(out, ref_out).max()) > 1:
        fails.append("out")
    return fails


@pytest.mark.parametrize("lossless", [False, True])
def test_experts_fp8_brute_force(lossless):
    """experts_fp8 against a per-token float64 restatement from the e4m3 codes and scales."""
    x, params, idx, w, gate_logit = _fp8_inputs(lossless, seed=1 if lossless else 2)
    out, inter = orc.experts_fp8(x, idx, w, orc.quant_weights_fp8(params), idx.shape[1], gate_logit)
    assert _fp8_failures(x, params, idx, w, gate_logit, out, inter) == []


def test_block_fp8_composes_router_and_experts():
    """block_fp8 = the bf16 router and shared-gate logit of the bf16 block, then experts_fp8."""
    from q38 import workloads
    wl = workloads.get("c1")
    x, params, _ = workloads.make(wl, tokens=96)
    x = x.to(torch.bfloat16)
    params = {n: p.to(torch.bfloat16) for n, p in params.items()}
    wq = orc.quant_weights_fp8(params)
    out, inter = orc.block_fp8(x, params, wq, wl.topk)
    _, _, idx, w = orc.router(x, params["gate.weight"], wl.topk)
    gl = orc.bf16(x.float() @ params["shared_expert_gate.weight"].float().reshape(-1))
    assert torch.equal(inter["idx"], idx) and torch.equal(inter["w"], w) and torch.equal(inter["gate_logit"], gl)
    out2, inter2 = orc.experts_fp8(x, idx, w, wq, wl.topk, gl)
    assert torch.equal(out, out2)
    assert _fp8_failures(x, params, idx, w, gl, out2, inter2) == []


def test_experts_fp8_lossless_equals_bf16_oracle():
    """On operands that per-row e4m3 quantisation represents exactly (power-of-two scales), the fp8
    gate/up stage is the bf16 gate/up stage: H equals experts_grouped's H (up to fp32 summation
    order: at most one bf16 rounding flip in a small fraction of elements), shared rows included."""
    x, params, idx, w, gate_logit = _fp8_inputs(True, seed=3)
    k = idx.shape[1]
    wq = orc.quant_weights_fp8(params)
    xq, sx = orc.quant_e4m3_rows(x)
    assert torch.equal((orc.e4m3_value(xq) * sx[:, None]).to(torch.bfloat16), x)
    for n, (q, s) in wq.items():
        assert torch.equal((orc.e4m3_value(q) * s[..., None]).to(torch.bfloat16), params[n]), n
    _, inter = orc.experts_fp8(x, idx, w, wq, k, gate_logit)
    _, _, H_bf16 = orc.experts_grouped(x, idx, w, params["experts.gate_up_proj"], params["experts.down_proj"])
    P = idx.numel()
    g = orc.bf16(x.float() @ params["shared_expert.gate_proj.weight"].float().T).float()
    u = orc.bf16(x.float() @ params["shared_expert.up_proj.weight"].float().T).float()
    hs = orc.bf16(orc.bf16(torch.nn.functional.silu(g)).float() * u)
    for got, want in ((inter["H"][:P], H_bf16), (inter["H"][P:], hs)):
        ulps = _bf16_ulps(got, want)
        assert int(ulps.max()) <= 1 and float((ulps > 0).float().mean()) < 0.01


def _run_with_planted(mistake, x, params, idx, w, gate_logit):
    """experts_fp8 with one scale-algebra mistake planted in the oracle (on the CPU)."""
    k = idx.shape[1]
    wq = dict(orc.quant_weights_fp8(params))
    real_quant = orc.quant_e4m3_rows
    calls = [0]
    if mistake == "swap_gate_up_scales":
        q, s = wq["experts.gate_up_proj"]
        I = s.shape[1] // 2
        wq["experts.gate_up_proj"] = (q, torch.cat([s[:, I:], s[:, :I]], dim=1))

    def patched(t):
        q, s = real_quant(t)
        calls[0] += 1
        if mistake == "token_scale_by_sorted_row" and calls[0] == 1:
            # token t takes the scale of the token behind sorted row t
            perm = torch.from_numpy(np.argsort(idx.reshape(-1).numpy(), kind="stable"))
            s = s[perm[: s.shape[0]] // k].clone()
        if mistake == "shared_down_other_row_scale" and calls[0] == 2:
            P = idx.numel()
            s = s.clone()
            s[P:] = torch.roll(s[P:], 1)
        return q, s
    orc.quant_e4m3_rows = patched
    try:
        return orc.experts_fp8(x, idx, w, wq, k, gate_logit)
    finally:
        orc.quant_e4m3_rows = real_quant


@pytest.mark.parametrize("mistake", ["swap_gate_up_scales", "token_scale_by_sorted_row",
                                     "shared_down_other_row_scale"])
@pytest.mark.parametrize("lossless", [False, True])
def test_brute_force_catches_planted_scale_mistakes(mistake, lossless):
    """Each scale-algebra mistake planted in the oracle makes the brute-force comparison fail (the
    former 8%-of-bf16 bar let a gate/up scale swap through)."""
    x, params, idx, w, gate_logit = _fp8_inputs(lossless, seed=4)
    out, inter = _run_with_planted(mistake, x, params, idx, w, gate_logit)
    assert _fp8_failures(x, params, idx, w, gate_logit, out, inter) != []


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
