"""Pins of the CPU oracle (oracle/) against independent facts. CPU only.

The reference ships no MoE golden vectors (its only parity artefact, audits/q38_kernel_parity.json,
holds error magnitudes). The oracle is pinned instead by: torch's own CPU top-k on tie-heavy data
(the library whose semantics the router must reproduce), a hand-worked tie case, torch.sort(stable)
for the permutation, float64 brute force on tiny blocks, and closed-form special cases.
"""
import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import moe_oracle as orc


def test_topk_known_answer():
    """Hand-worked libstdc++ introselect on [.1,.5,.5,.2,.5,.5,.5,0], k=5 -> [1,6,5,4,2]."""
    v = np.array([[0.1, 0.5, 0.5, 0.2, 0.5, 0.5, 0.5, 0.0]], np.float32)
    vals, idx = orc.topk_cpu(v, 5)
    assert idx.tolist() == [[1, 6, 5, 4, 2]]
    assert torch.topk(torch.from_numpy(v), 5).indices.tolist() == [[1, 6, 5, 4, 2]]


@pytest.mark.parametrize("kind", ["int", "bf16", "nan"])
def test_topk_matches_torch_cpu(kind):
    g = torch.Generator().manual_seed(0)
    if kind == "int":
        v = torch.randint(0, 6, (20000, 64), generator=g).float()
    elif kind == "bf16":
        v = torch.softmax((torch.randn(20000, 64, generator=g) * 0.64).to(torch.bfloat16).float(), -1)
    else:
        v = torch.randint(0, 4, (5000, 64), generator=g).float()
        v[torch.rand(5000, 64, generator=g) < 0.05] = float("nan")
    for k in (1, 3, 5, 8):
        ov, oi = orc.topk_cpu(v.numpy(), k)
        tv, ti = torch.topk(v, k)
        assert np.array_equal(oi, ti.numpy()), f"k={k}"
        assert np.array_equal(np.isnan(ov), torch.isnan(tv).numpy())


def test_topk_small_n():
    g = torch.Generator().manual_seed(1)
    v = torch.randint(0, 3, (5000, 8), generator=g).float()
    ov, oi = orc.topk_cpu(v.numpy(), 3)
    assert np.array_equal(oi, torch.topk(v, 3).indices.numpy())


@pytest.mark.parametrize("T,E,k", [(1000, 64, 5), (53, 8, 3), (0, 64, 5)])
def test_permute_matches_stable_sort(T, E, k):
    g = torch.Generator().manual_seed(2)
    idx = torch.randint(0, E, (T, k), generator=g)
    counts, starts, perm = orc.permute_cpu(idx.numpy(), E)
    ids = idx.reshape(-1)
    sorted_ids, tperm = torch.sort(ids, stable=True)
    assert np.array_equal(perm, tperm.numpy())
    assert np.array_equal(counts, torch.bincount(ids, minlength=E).numpy())
    bounds = torch.searchsorted(sorted_ids, torch.arange(E + 1))
    assert np.array_equal(starts, bounds[:-1].numpy())
    # Invariants: a permutation, ids non-decreasing along it, ascending within an expert.
    assert np.array_equal(np.sort(perm), np.arange(T * k))
    assert (np.diff(ids.numpy()[perm]) >= 0).all()


def test_permute_drops_sentinels():
    ids = np.array([3, 8, -1, 0, 3, 7, 9], np.int64)
    counts, starts, perm = orc.permute_cpu(ids, 8)
    assert perm.tolist() == [3, 0, 4, 5] and counts.sum() == 4


def _tiny_params(h=64, E=8, I=64, Is=64, seed=0):
    from q38 import workloads
    wl = workloads.Workload("tiny", hidden=h, experts=E, topk=3, inter=I, shared_inter=Is, batch=1, seq=37)
    x, p, _ = workloads.make(wl, seed_w=seed)
    return wl, x, p


def test_block_vs_float64_bruteforce():
    """Per-token float64 loop of the block's math; oracle (bf16 roundings) must be within bf16
    tolerance. A transposed weight, wrong gate/up half or dropped routing weight fails this."""
    wl, x, p = _tiny_params()
    out, inter = orc.block(x, p, wl.topk)
    xd = x.double()
    wr, gu, dn = p["gate.weight"].double(), p["experts.gate_up_proj"].double(), p["experts.down_proj"].double()
    I = wl.inter
    ref = torch.zeros_like(xd)
    for t in range(xd.shape[0]):
        probs = torch.softmax(xd[t] @ wr.T, -1)
        idx = inter["idx"][t]
        wsel = probs[idx] / probs[idx].sum()
        for j, e in enumerate(idx.tolist()):
            hv = gu[e] @ xd[t]
            act = hv[:I] / (1 + torch.exp(-hv[:I])) * hv[I:]
            ref[t] += wsel[j] * (dn[e] @ act)
        g = p["shared_expert.gate_proj.weight"].double() @ xd[t]
        u = p["shared_expert.up_proj.weight"].double() @ xd[t]
        sh = p["shared_expert.down_proj.weight"].double() @ (g / (1 + torch.exp(-g)) * u)
        sg = torch.sigmoid(p["shared_expert_gate.weight"].double().reshape(-1) @ xd[t])
        ref[t] += sg * sh
    diff = (out.double() - ref).abs()
    assert float(diff.max()) < 2e-2
    assert float(diff.norm() / ref.norm()) < 1e-2


def test_grouped_vs_eager_experts():
    """The oracle's grouped rounding (inference.py:60-130,199) vs the eager loop (modeling:769-793)."""
    from q38 import workloads
    wl = workloads.get("c1")
    x, p, _ = workloads.make(wl, tokens=512)
    _, _, idx, w = orc.router(x, p["gate.weight"], wl.topk)
    a, _, _ = orc.experts_grouped(x, idx, w, p["experts.gate_up_proj"], p["experts.down_proj"])
    b = orc.experts_eager(x, idx, w, p["experts.gate_up_proj"], p["experts.down_proj"])
    diff = (a.float() - b.float()).abs()
    assert float(diff.max()) < 2e-2 and float(diff.norm() / b.float().norm()) < 1e-2


def test_reference_block_forward_matches_oracle():
    from q38 import workloads
    wl = workloads.get("c1")
    x, p, _ = workloads.make(wl, tokens=256)
    a, _ = orc.block(x, p, wl.topk)
    b = orc.reference_block_forward(x, p, wl.topk)
    diff = (a.float() - b.float()).abs()
    assert float(diff.max()) < 2e-2 and float(diff.norm() / b.float().norm()) < 1e-2


def test_special_cases():
    """Zero router weight: uniform probabilities, all tied -> torch's tie order, equal weights 1/k.
    k = E: every expert selected. Zero shared-gate weight: sigmoid(0) = 0.5 exactly."""
    wl, x, p = _tiny_params()
    p0 = dict(p)
    p0["gate.weight"] = torch.zeros_like(p["gate.weight"])
    _, probs, idx, w = orc.router(x, p0["gate.weight"], wl.topk)
    ti = torch.topk(torch.full((1, wl.experts), 1.0 / wl.experts), wl.topk).indices
    assert torch.equal(idx, ti.expand_as(idx))
    assert torch.equal(w, torch.full_like(w, 1.0 / wl.topk))
    _, _, idx_all, w_all = orc.router(x, p["gate.weight"], wl.experts)
    assert torch.equal(idx_all.sort(-1).values, torch.arange(wl.experts).expand_as(idx_all))
    p2 = dict(p)
    p2["shared_expert_gate.weight"] = torch.zeros_like(p["shared_expert_gate.weight"])
    _, inter = orc.block(x, p2, wl.topk)
    out2, _ = orc.block(x, p2, wl.topk)
    half = orc.bf16(0.5 * inter["shared"].float())
    assert torch.equal(out2, orc.bf16(inter["routed"].float() + half.float()))


def test_shared_expert_matches_linear_chain():
    wl, x, p = _tiny_params()
    wg, wu, wd = (p[f"shared_expert.{n}_proj.weight"] for n in ("gate", "up", "down"))
    ref = F.linear(F.silu(F.linear(x, wg)) * F.linear(x, wu), wd)
    diff = (orc.shared_expert(x, wg, wu, wd).float() - ref.float()).abs()
    assert float(diff.max()) < 2e-2


def test_skew_workload_load_span():
    """The routing-skew workload's logit bias gives the ~20x span of expert loads it stands for
    (max/min pair count over experts on its seeded inputs), and the bias is a Zipf law in rank."""
    from q38 import workloads
    wl = workloads.get("c3")
    x, p, bias = workloads.make(wl)
    b = bias.double().numpy()
    ranks = np.argsort(np.argsort(-b)) + 1   # rank 1 = largest bias
    assert np.allclose(b, -wl.zipf_alpha * wl.zipf_s * np.log(ranks), atol=1e-6)
    logits = orc.bf16(x.float() @ p["gate.weight"].float().T)
    _, _, idx, _ = orc.router(x, p["gate.weight"], wl.topk, logit_bias=bias, logits=logits)
    c = np.bincount(idx.reshape(-1).numpy(), minlength=wl.experts)
    assert c.sum() == wl.tokens * wl.topk
    assert 15 <= c.max() / c.min() <= 30, (c.max(), c.min())


@pytest.mark.parametrize("seed,bm,shared", [(0, 256, 0), (1, 256, 3000), (2, 64, 17), (3, 128, 256)])
def test_tile_table_blocks(seed, bm, shared):
    """tile_table lists exactly the reference's per-expert blocks (inference.py:39-50: block j of
    expert e covers sorted rows starts[e] + j*BM .. min(+BM, starts[e] + counts[e])), plus the
    shared rows' blocks, with full blocks first and partial blocks by non-increasing size."""
    rs = np.random.RandomState(seed)
    E = 64
    counts = rs.randint(0, 3 * bm, size=E).astype(np.int32)
    counts[rs.rand(E) < 0.1] = 0
    starts = (np.cumsum(counts) - counts).astype(np.int32)
    P = int(counts.sum())
    tl = orc.tile_table(counts, starts, bm, shared, P=P)
    ref = []
    for e in range(E):
        for j in range(-(-int(counts[e]) // bm)):
            r0 = int(starts[e]) + j * bm
            ref.append((e, r0, min(bm, int(starts[e] + counts[e]) - r0)))
    for j in range(-(-shared // bm)):
        ref.append((E, P + j * bm, min(bm, shared - j * bm)))
    assert sorted(tl) == sorted(ref)
    sizes = [t[2] for t in tl]
    nfull = sum(s == bm for s in sizes)
    assert all(s == bm for s in sizes[:nfull])
    assert all(a >= b for a, b in zip(sizes[nfull:], sizes[nfull + 1:]))


def _same_bits(a, b):
    a, b = np.asarray(a, np.float32), np.asarray(b, np.float32)
    return (a.view(np.uint32) == b.view(np.uint32)) | (np.isnan(a) & np.isnan(b))


@pytest.mark.parametrize("n", [64, 8, 17, 33, 16, 15, 48, 1])
def test_softmax_restatement_is_torch_cpu(n):
    """The router's probabilities follow torch's CPU softmax operation by operation (SLEEF expf_u10,
    the 16-lane reduction order, multiply by 1/sum): bit for bit on mixed scales, wide ranges,
    +-inf and NaN rows, and biased rows."""
    rng = np.random.RandomState(n)
    z = (rng.randn(6000, n) * rng.choice([0.05, 0.64, 5.0, 40.0], size=(6000, 1))).astype(np.float32)
    z[:500] = rng.uniform(-120, 0, (500, n))
    z[500:1000] += (-0.24 * np.log(rng.permutation(n) + 1)).astype(np.float32)
    z[1000:1100, 0] = np.nan
    z[1100:1200] = -np.inf
    z[1200:1300, n // 2] = np.inf
    got = orc.softmax_torch_order(z)
    want = torch.softmax(torch.from_numpy(z), dim=-1).numpy()
    assert _same_bits(got, want).all(), f"{int((~_same_bits(got, want)).sum())} values differ"


def test_topk_renorm_sum_order():
    """torch's CPU sum over the last dimension of a [rows, k] fp32 tensor, the top-k
    renormalisation (modeling:810): the 4-way interleaved row sum for k in 5..7, left to right for
    every other k <= 8 (what the router kernel reproduces)."""
    rng = np.random.RandomState(5)
    for k in range(1, 9):
        v = np.sort(rng.rand(20000, k).astype(np.float32) * 0.3, axis=1)[:, ::-1].copy()
        if 5 <= k <= 7:
            s = v[:, 0] + v[:, 4]
            for r in list(range(5, k)) + [1, 2, 3]:
                s = (s + v[:, r]).astype(np.float32)
        else:
            s = v[:, 0].copy()
            for r in range(1, k):
                s = (s + v[:, r]).astype(np.float32)
        t = torch.from_numpy(v)
        assert _same_bits(s, t.sum(dim=-1).numpy()).all(), k
        assert _same_bits(v / s[:, None], (t / t.sum(dim=-1, keepdim=True)).numpy()).all(), k


def test_collision_rows_need_probabilities():
    """The collision row classes of the route tests really separate selection on probabilities
    from selection on logits: distinct logits there give equal fp32 probabilities, and torch's
    top-k then breaks those ties by introselect position, not by the larger logit."""
    from _util import collision_bias, collision_bias_logits, collision_logits
    for z in (collision_logits(2000).float(), collision_bias_logits(2000).float() + collision_bias()):
        p = torch.softmax(z, -1)
        _, on_p = orc.topk_cpu(p.numpy(), 5)
        _, on_z = orc.topk_cpu(z.numpy(), 5)
        assert (on_p != on_z).any(axis=1).mean() > 0.1


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_experts_grouped_mm_is_transformers(dtype):
    """experts_grouped_mm (the presets' configured implementation, restated on F.grouped_mm) equals
    the installed transformers grouped_mm_experts_forward bit for bit on the same module state,
    dropped sentinel pairs included; and it agrees with the eager loop (fp32: to float rounding)."""
    moe = pytest.importorskip("transformers.integrations.moe")
    g = torch.Generator().manual_seed(9)
    T, h, E, k, I = 93, 64, 8, 3, 32
    x = torch.randn(T, h, generator=g).to(dtype)
    idx = torch.stack([torch.randperm(E, generator=g)[:k] for _ in range(T)])
    idx[5, 1] = E  # a sentinel pair (expert-parallel drop), contributes nothing
    w = torch.rand(T, k, generator=g).to(dtype)
    wgu = (torch.randn(E, 2 * I, h, generator=g) * 0.1).to(dtype)
    wdn = (torch.randn(E, h, I, generator=g) * 0.1).to(dtype)

    class Mod(torch.nn.Module):
        num_experts, has_gate, has_bias, is_transposed = E, True, False, False
        gate_up_proj, down_proj = wgu, wdn
        act_fn = staticmethod(F.silu)

        def _apply_gate(self, gu):
            return moe._default_apply_gate(self, gu)

    want = moe.grouped_mm_experts_forward(Mod(), x, idx, w)
    got = orc.experts_grouped_mm(x, idx, w, wgu, wdn)
    assert got.dtype == dtype and torch.equal(got, want)
    if dtype == torch.float32:
        eager = orc.experts_eager(x, idx, w, wgu, wdn)
        assert torch.allclose(got, eager, rtol=1e-5, atol=1e-6)
