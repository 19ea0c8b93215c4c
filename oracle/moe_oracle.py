"""CPU oracle of the Q38 MoE feed-forward prefill. TEST INFRASTRUCTURE ONLY.

Imported by tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg, as the checker and
as the timed CPU baseline; the product path (qwen35-moe-sparse_amd/q38) never imports it.

What each function restates (reference paths; "modeling" = q38/models/qwen3_8_moe/
modeling_qwen3_8_moe.py, "inference" = q38/inference.py):

  topk_cpu        torch CPU top-k tie order, ATen/native/TopKImpl.h:45-76, via the C restatement
                  in q38_oracle.cpp (liboracle.so) that calls libstdc++'s nth_element/sort.
  softmax_torch_order  torch's CPU fp32 softmax restated operation by operation (C); the router
                  kernel computes its probabilities the same way. router() itself calls
                  torch.softmax, the reference's op.
  permute_cpu     stable counting sort = torch.sort(ids, stable=True) + searchsorted,
                  inference:163-171 (C, q38_oracle.cpp).
  tile_table      the per-expert BM-row blocks of inference:39-50,174-183 in the GEMM's order.
  router          Qwen3_8MoeTopKRouter.forward, modeling:805-813 (fp32 matmul rounded once to
                  bf16 stands for the bf16 F.linear; softmax fp32; torch CPU topk; renorm).
  experts_grouped routed experts with the rounding sequence of inference:60-130,199 (also that
                  of transformers' grouped_mm path): per-expert fp32 matmuls on gathered rows,
                  bf16 rounding of gate/up, silu, product, down, weight; fp32 k-sum.
  experts_eager   Qwen3_8MoeExperts.forward, modeling:769-793, op for op (index_add_ in D).
  experts_grouped_mm  transformers' grouped_mm_experts_forward (integrations/moe.py:377-478), the
                  configured implementation of the presets, on torch.nn.functional.grouped_mm.
  shared_expert   Qwen3_8MoeMLP.forward, modeling:751-753.
  block           Qwen3_8MoeSparseMoeBlock.forward, modeling:824-835.
  reference_block_forward  the whole block computed with the reference's own torch op sequence in
                  the module dtype (eager experts): the timed CPU baseline.

Parity pins (tests/test_oracle.py): topk_cpu vs torch.topk on tie-heavy rows and hand-worked
cases; permute_cpu vs torch.sort(stable=True)/bincount and its invariants; the FP functions vs
float64 brute force on tiny shapes, vs each other (grouped vs eager), and on special cases with
closed forms (zero router weight, k = E, zero shared-gate weight).
"""
import ctypes
import os
import subprocess
from pathlib import Path

import numpy as np
import torch
import torch.nn.functional as F

ORACLE_DIR = Path(__file__).resolve().parent
LIB_PATH = ORACLE_DIR / "_build" / "liboracle.so"


def build():
    """Compile q38_oracle.cpp with g++ into oracle/_build/liboracle.so."""
    (ORACLE_DIR / "_build").mkdir(exist_ok=True)
    tmp = LIB_PATH.with_suffix(".so.tmp")
    subprocess.run(["g++", "-O2", "-std=c++17", "-ffp-contract=off", "-shared", "-fPIC",
                    str(ORACLE_DIR / "q38_oracle.cpp"), "-o", str(tmp)], check=True)
    os.replace(tmp, LIB_PATH)
    return LIB_PATH


_lib = None


def _load():
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            build()
        lib = ctypes.CDLL(str(LIB_PATH))
        lib.oracle_topk.argtypes = [ctypes.c_void_p, ctypes.c_int64, ctypes.c_int64, ctypes.c_int64,
                                    ctypes.c_void_p, ctypes.c_void_p]
        lib.oracle_topk.restype = None
        lib.oracle_permute.argtypes = [ctypes.c_void_p, ctypes.c_int64, ctypes.c_int32, ctypes.c_void_p,
                                       ctypes.c_void_p, ctypes.c_void_p]
        lib.oracle_permute.restype = None
        lib.oracle_softmax_rows.argtypes = [ctypes.c_void_p, ctypes.c_int64, ctypes.c_int64, ctypes.c_void_p]
        lib.oracle_softmax_rows.restype = None
        _lib = lib
    return _lib


def topk_cpu(values, k):
    """(values fp32 [R,k], indices int64 [R,k]) of torch CPU topk(values, k, largest, sorted)."""
    v = np.ascontiguousarray(np.asarray(values, dtype=np.float32))
    R, n = v.shape
    ov = np.empty((R, k), np.float32)
    oi = np.empty((R, k), np.int64)
    _load().oracle_topk(v.ctypes.data, R, n, k, ov.ctypes.data, oi.ctypes.data)
    return ov, oi


def softmax_torch_order(z):
    """fp32 softmax over the last dimension restated as torch's CPU kernel computes it
    (q38_oracle.cpp oracle_softmax_rows); pinned bit for bit against torch.softmax."""
    v = np.ascontiguousarray(np.asarray(z, dtype=np.float32))
    R, n = v.shape
    out = np.empty_like(v)
    _load().oracle_softmax_rows(v.ctypes.data, R, n, out.ctypes.data)
    return out


def permute_cpu(ids, E):
    """(counts int32 [E], starts int32 [E], perm int32 [sum counts]) of a stable sort by expert."""
    a = np.ascontiguousarray(np.asarray(ids, dtype=np.int64).reshape(-1))
    counts = np.empty(E, np.int32)
    starts = np.empty(E, np.int32)
    valid = int(((a >= 0) & (a < E)).sum())
    perm = np.empty(valid, np.int32)
    _load().oracle_permute(a.ctypes.data, a.size, E, counts.ctypes.data, starts.ctypes.data, perm.ctypes.data)
    return counts, starts, perm


def tile_table(counts, starts, block_m, shared_rows=0, P=None):
    """Tile list of the grouped GEMMs as (group, row0, rows) tuples, in walking order.

    The reference splits each expert's sorted segment into cdiv(count, BM) row blocks
    (inference:39-50, 174-183); the same blocks are listed here with the full ones first (by
    expert, then the shared-expert rows [P, P + shared_rows) as group E), then the partial ones by
    falling row count (ties: lower group first).
    """
    E = len(counts)
    P = int(np.sum(counts)) if P is None else P
    full, partial = [], []
    segs = [(e, int(starts[e]), int(counts[e])) for e in range(E)] + [(E, P, int(shared_rows))]
    for g, r0, n in segs:
        for i in range(n // block_m):
            full.append((g, r0 + i * block_m, block_m))
        if n % block_m:
            partial.append((g, r0 + (n // block_m) * block_m, n % block_m))
    partial.sort(key=lambda t: (-t[2], t[0]))
    return full + partial


def bf16(t):
    return t.to(torch.bfloat16)


def _f(t):
    return t.to(torch.float32)


def router(x, w_router, k, logit_bias=None, logits=None, dtype=torch.bfloat16):
    """modeling:805-813. Returns (logits [T,E], probs fp32 [T,E], idx int64 [T,k], w [T,k]) with
    logits and w in ``dtype``: bf16 (the logits one rounding of the fp32 product, as the bf16
    F.linear; w rounded to bf16) or fp32 (nothing rounded: the fp32 model's router).

    ``logits`` may be supplied to run only the selection, as q38moe_route_from_logits does; their
    dtype then decides. The optional fp32 ``logit_bias`` [E] is added before the softmax
    (routing-skew workload).
    """
    if logits is None:
        logits = (_f(x) @ _f(w_router).T).to(dtype)
    dtype = logits.dtype
    z = _f(logits)
    if logit_bias is not None:
        z = z + _f(logit_bias)
    probs = torch.softmax(z, dim=-1)
    vals, idx = topk_cpu(probs.numpy(), k)
    vals = torch.from_numpy(vals)
    vals = vals / vals.sum(dim=-1, keepdim=True)
    return logits, probs, torch.from_numpy(idx), vals.to(dtype)


def experts_grouped(x, idx, w, w_gate_up, w_down, return_sorted=False, _skip_rounding=()):
    """Routed experts, rounding of inference:60-130 and the k-sum of inference:199. Also returns
    the weighted per-pair rows y [T*k,h] bf16 (pair order) and H [T*k,I] bf16 (sorted order);
    with return_sorted, also Y_raw = bf16(H . Wd^T) [T*k,h] in sorted order.

    _skip_rounding (tests only: planted mistakes the rounding-point test must reject) names bf16
    roundings to leave out: "g" (gate), "u" (up), "silu", "down" (the down product)."""
    skip = set(_skip_rounding)
    rnd = {key: (_f if key in skip else (lambda t: _f(bf16(t)))) for key in ("g", "u", "silu", "down")}
    T, h = x.shape
    k = idx.shape[1]
    E, twoI, _ = w_gate_up.shape
    I = twoI // 2
    counts, starts, perm = permute_cpu(idx.numpy(), E)
    perm_t = torch.from_numpy(perm.astype(np.int64))
    wflat = _f(w.reshape(-1))
    y = torch.zeros(T * k, h, dtype=torch.bfloat16)
    H = torch.zeros(perm.size, I, dtype=torch.bfloat16)
    Y_raw = torch.zeros(perm.size, h, dtype=torch.bfloat16)
    xf = _f(x)
    for e in range(E):
        c, s = int(counts[e]), int(starts[e])
        if c == 0:
            continue
        rows = perm_t[s:s + c]
        A = xf[rows // k]
        gu = A @ _f(w_gate_up[e]).T
        g = rnd["g"](gu[:, :I])
        u = rnd["u"](gu[:, I:])
        act = rnd["silu"](F.silu(g))
        He = bf16(act * u)
        H[s:s + c] = He
        d = rnd["down"](_f(He) @ _f(w_down[e]).T)
        Y_raw[s:s + c] = d
        y[rows] = bf16(_f(d) * wflat[rows][:, None])
    out = bf16(_f(y).view(T, k, h).sum(dim=1))
    if return_sorted:
        return out, y, H, Y_raw
    return out, y, H


def experts_eager(x, idx, w, w_gate_up, w_down):
    """Qwen3_8MoeExperts.forward (modeling:769-793) op for op, in the dtype of x."""
    final = torch.zeros_like(x)
    E = w_gate_up.shape[0]
    mask = F.one_hot(idx, num_classes=E + 1).permute(2, 1, 0)
    hit = torch.greater(mask.sum(dim=(-1, -2)), 0).nonzero()
    for e in hit:
        e = int(e[0])
        if e == E:
            continue
        pos, tok = torch.where(mask[e])
        cur = x[tok]
        gate, up = F.linear(cur, w_gate_up[e]).chunk(2, dim=-1)
        hcur = F.silu(gate) * up
        hcur = F.linear(hcur, w_down[e])
        hcur = hcur * w[tok, pos, None]
        final.index_add_(0, tok, hcur.to(final.dtype))
    return final


def experts_grouped_mm(x, idx, w, w_gate_up, w_down):
    """The experts implementation the reference's presets configure (configs/q38_c1.json:22):
    transformers' grouped_mm_experts_forward (installed integrations/moe.py:377-478), restated on
    torch.nn.functional.grouped_mm in the dtype of x. Pairs sorted by expert (torch.sort), per-expert
    row offsets (histc + cumsum), one grouped GEMM over the gathered rows against gate_up_proj^T,
    silu(gate) * up (moe.py:509-520), one grouped GEMM against down_proj^T, times the routing
    weight, rows back in pair order, then the k-sum (accumulated in fp32 for bf16 inputs by
    torch's reduction) cast to x's dtype. Pairs with indices outside [0, E) contribute nothing."""
    T, h = x.shape
    k = idx.shape[1]
    E = w_gate_up.shape[0]
    ids = idx.reshape(-1)
    ids_g, perm = torch.sort(ids)
    rows = x[perm // k]
    wg = w.reshape(-1)[perm]
    counts = torch.histc(ids_g.float(), bins=E, min=0, max=E - 1)
    offs = torch.cumsum(counts, dim=0, dtype=torch.int32)
    dropped = (ids_g >= E).unsqueeze(-1)
    rows = rows.masked_fill(dropped, 0.0)
    gu = F.grouped_mm(rows, w_gate_up.transpose(-2, -1), offs=offs)
    gate, up = gu.chunk(2, dim=-1)
    act = F.silu(gate) * up
    y = F.grouped_mm(act, w_down.transpose(-2, -1), offs=offs)
    y = (y * wg.unsqueeze(-1)).masked_fill(dropped, 0.0)
    inv = torch.empty_like(perm)
    inv[perm] = torch.arange(perm.numel())
    return y[inv].view(T, k, h).sum(dim=1).to(x.dtype)


def shared_expert(x, w_gate, w_up, w_down):
    """modeling:751-753 with fp32 matmuls rounded once to bf16 at each linear."""
    g = _f(bf16(_f(x) @ _f(w_gate).T))
    u = _f(bf16(_f(x) @ _f(w_up).T))
    hs = bf16(_f(bf16(F.silu(g))) * u)
    return bf16(_f(hs) @ _f(w_down).T)


def block(x, params, k, logit_bias=None):
    """modeling:824-835 (grouped expert rounding). Returns out bf16 [T,h] and the intermediates."""
    logits, probs, idx, w = router(x, params["gate.weight"], k, logit_bias)
    routed, y, H = experts_grouped(x, idx, w, params["experts.gate_up_proj"], params["experts.down_proj"])
    sh = shared_expert(x, params["shared_expert.gate_proj.weight"], params["shared_expert.up_proj.weight"],
                       params["shared_expert.down_proj.weight"])
    gate_logit = bf16(_f(x) @ _f(params["shared_expert_gate.weight"]).reshape(-1))
    gated = bf16(_f(bf16(torch.sigmoid(_f(gate_logit))))[:, None] * _f(sh))
    out = bf16(_f(routed) + _f(gated))
    return out, dict(logits=logits, probs=probs, idx=idx, w=w, routed=routed, y=y, H=H, shared=sh,
                     gate_logit=gate_logit)


def reference_block_forward(x, params, k, logit_bias=None, experts="eager", routing=None):
    """The reference block's own op sequence (modeling:805-813, 769-793, 751-753, 824-835) in the
    dtype of the inputs, with the eager experts loop (experts="eager", the module's own forward) or
    the grouped_mm implementation the presets configure (experts="grouped_mm"). This is the CPU
    baseline that bench.py times. The optional fp32 ``logit_bias`` [E] (routing-skew workload) is
    added to the logits before the softmax. ``routing`` = (idx [T,k], w [T,k]) replaces the router
    (to compare a device's block on the device's own routing)."""
    if routing is None:
        logits = F.linear(x, params["gate.weight"])
        z = logits if logit_bias is None else logits.float() + logit_bias.float()
        probs = torch.softmax(z, dtype=torch.float, dim=-1)
        top, idx = torch.topk(probs, k, dim=-1)
        top /= top.sum(dim=-1, keepdim=True)
        w = top.to(logits.dtype)
    else:
        idx, w = routing
    g = F.linear(x, params["shared_expert.gate_proj.weight"])
    u = F.linear(x, params["shared_expert.up_proj.weight"])
    sh = F.linear(F.silu(g) * u, params["shared_expert.down_proj.weight"])
    run = experts_grouped_mm if experts == "grouped_mm" else experts_eager
    routed = run(x, idx, w, params["experts.gate_up_proj"], params["experts.down_proj"])
    sh = torch.sigmoid(F.linear(x, params["shared_expert_gate.weight"])) * sh
    return routed + sh


# ---- fp8 expert path (R14). The reference has no fp8: these restate this repository's definition
# (include/q38moe.h, q38moe_quantize_rows / q38moe_block_forward_fp8) on the CPU. ----

E4M3_MAX = 448.0


def quant_e4m3_rows(t):
    """Per-row e4m3 quantisation: amax = max|x| per row (fp32), inv = 448/amax (0 for a zero row),
    q = e4m3(RNE(clamp(x*inv, +-448))) via torch.float8_e4m3fn, scale = amax/448. Returns
    (q uint8 bit patterns, same shape; scale fp32, shape[:-1])."""
    x = _f(t)
    shape = x.shape
    x2 = x.reshape(-1, shape[-1])
    amax = x2.abs().amax(dim=1)
    inv = torch.where(amax > 0, torch.tensor(E4M3_MAX, dtype=torch.float32) / amax, torch.zeros_like(amax))
    inv = torch.where(torch.isnan(amax), amax, inv)
    q = (x2 * inv[:, None]).clamp(-E4M3_MAX, E4M3_MAX).to(torch.float8_e4m3fn)
    scale = amax / E4M3_MAX
    return q.view(torch.uint8).reshape(shape), scale.reshape(shape[:-1])


def e4m3_value(q):
    """uint8 e4m3 bit patterns -> fp32 values."""
    return q.view(torch.float8_e4m3fn).to(torch.float32)


def quant_weights_fp8(params):
    """The block's expert weights in e4m3 with per-output-channel scales (q38moe_quantize_rows on
    each weight row)."""
    names = ("experts.gate_up_proj", "experts.down_proj", "shared_expert.gate_proj.weight",
             "shared_expert.up_proj.weight", "shared_expert.down_proj.weight")
    return {n: quant_e4m3_rows(params[n]) for n in names}


def _fp8_matmul(qa, sa, qw, sw):
    """(sum_c qa[r,c] qw[n,c]) * sa[r] * sw[n]: exact e4m3 products, fp32 sums, then the scales."""
    return (e4m3_value(qa) @ e4m3_value(qw).T) * sa[:, None] * sw[None, :]


def experts_fp8(x, idx, w, wq, k, gate_logit):
    """The e4m3 experts of q38moe_block_forward_fp8 for given routing (idx [T,k], w bf16 [T,k]) and
    shared-gate logits: tokens quantised per row; routed and shared gate/up on e4m3 with the bf16
    roundings of inference:90-96; SwiGLU rows (sorted routed rows, then the shared rows) quantised
    per row; down on e4m3 rounded to bf16; weight, k-sum and gated shared sum as in ``block``."""
    T, h = x.shape
    qg, sg = wq["experts.gate_up_proj"]
    qd, sd = wq["experts.down_proj"]
    E, twoI, _ = qg.shape
    I = twoI // 2
    xq, sx = quant_e4m3_rows(x)
    counts, starts, perm = permute_cpu(idx.numpy(), E)
    perm_t = torch.from_numpy(perm.astype(np.int64))
    P = T * k
    H = torch.zeros(P + T, I, dtype=torch.bfloat16)  # sorted routed rows [0, P), shared [P, P + T)

    def swiglu(qa, sa, qgate, sgate, qup, sup):
        g = _f(bf16(_fp8_matmul(qa, sa, qgate, sgate)))
        u = _f(bf16(_fp8_matmul(qa, sa, qup, sup)))
        return bf16(_f(bf16(F.silu(g))) * u)

    for e in range(E):
        c, s = int(counts[e]), int(starts[e])
        if c == 0:
            continue
        tok = perm_t[s:s + c] // k
        H[s:s + c] = swiglu(xq[tok], sx[tok], qg[e, :I], sg[e, :I], qg[e, I:], sg[e, I:])
    H[P:] = swiglu(xq, sx, *wq["shared_expert.gate_proj.weight"], *wq["shared_expert.up_proj.weight"])
    Hq, sH = quant_e4m3_rows(H)
    Y = torch.zeros(P + T, h, dtype=torch.bfloat16)
    for e in range(E):
        c, s = int(counts[e]), int(starts[e])
        if c:
            Y[s:s + c] = bf16(_fp8_matmul(Hq[s:s + c], sH[s:s + c], qd[e], sd[e]))
    Y[P:] = bf16(_fp8_matmul(Hq[P:], sH[P:], *wq["shared_expert.down_proj.weight"]))
    wflat = _f(w.reshape(-1))
    y = torch.zeros(P, h, dtype=torch.bfloat16)
    y[perm_t] = bf16(_f(Y[:P]) * wflat[perm_t][:, None])
    routed = bf16(_f(y).view(T, k, h).sum(dim=1))
    sh = Y[P:]
    gated = bf16(_f(bf16(torch.sigmoid(_f(gate_logit))))[:, None] * _f(sh))
    out = bf16(_f(routed) + _f(gated))
    return out, dict(xq=xq, sx=sx, perm=perm_t, H=H, Hq=Hq, sH=sH, Y=Y, routed=routed, shared=sh)


def block_fp8(x, params, wq, k, logit_bias=None):
    """q38moe_block_forward_fp8 on the CPU: the bf16 router and shared-gate logit of ``block``, then
    ``experts_fp8``. Returns out and intermediates."""
    logits, probs, idx, w = router(x, params["gate.weight"], k, logit_bias)
    gate_logit = bf16(_f(x) @ _f(params["shared_expert_gate.weight"]).reshape(-1))
    out, inter = experts_fp8(x, idx, w, wq, k, gate_logit)
    return out, dict(inter, logits=logits, idx=idx, w=w, gate_logit=gate_logit)
