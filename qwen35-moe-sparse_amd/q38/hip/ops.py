"""Torch-tensor front end of the C ABI: shape/dtype checks, output allocation, stream passing.

Every function launches HIP kernels on the current torch stream of the input's device and
returns without synchronising. Inputs must be contiguous CUDA (HIP) tensors in bf16, or, for the
forward path (router, permutation, grouped GEMMs, combine, experts, block), fp32 (the fp32 models
of the reference, computed without intermediate roundings); the activations' dtype decides and the
weights must share it. Weights use the reference parameter layouts (experts.gate_up_proj [E,2I,h],
experts.down_proj [E,h,I], nn.Linear weights [out,in]).
"""
import ctypes

import torch

from ._lib import BF16, FP32, TILING_PERSISTENT, TILING_SMALL, check, lib

_NULL = None


def _ptr(t):
    return None if t is None else ctypes.c_void_p(t.data_ptr())


def _stream(device):
    return ctypes.c_void_p(torch.cuda.current_stream(device).cuda_stream)


def _need(t, name, dtype=torch.bfloat16, ndim=None):
    if not isinstance(t, torch.Tensor):
        raise TypeError(f"{name} must be a tensor")
    if not t.is_cuda:
        raise RuntimeError(f"{name} must be a CUDA/HIP tensor (the Q38 MoE path runs only on the GPU)")
    if dtype is not None and t.dtype != dtype:
        raise TypeError(f"{name} must be {dtype}, got {t.dtype}")
    if ndim is not None and t.dim() != ndim:
        raise ValueError(f"{name} must have {ndim} dims, got shape {tuple(t.shape)}")
    if not t.is_contiguous():
        raise ValueError(f"{name} must be contiguous")
    return t


_DTYPES = {torch.bfloat16: BF16, torch.float32: FP32}


def _fdt(t, name):
    """The float dtype of the forward path given by tensor t (bf16 or fp32)."""
    if not isinstance(t, torch.Tensor) or t.dtype not in _DTYPES:
        raise TypeError(f"{name} must be a bf16 or fp32 tensor, got {getattr(t, 'dtype', type(t))}")
    return t.dtype


def _idx_flag(idx):
    if idx.dtype == torch.int64:
        return 1
    if idx.dtype == torch.int32:
        return 0
    raise TypeError(f"routing indices must be int32 or int64, got {idx.dtype}")


def gemm_block_m():
    return int(lib.q38moe_gemm_block_m())


def max_tiles(T, E, k, shared_rows=0):
    return int(lib.q38moe_max_tiles(T, E, k, shared_rows))


def gemm_tiling(T, h, E, k, I, shared_rows=0, fp8=False):
    """"small" or "persistent": the grouped-GEMM kernels bf16 (or, with fp8, e4m3) calls of this
    shape run."""
    f = lib.q38moe_gemm_tiling_fp8 if fp8 else lib.q38moe_gemm_tiling
    v = int(f(T, h, E, k, I, shared_rows))
    return {TILING_SMALL: "small", TILING_PERSISTENT: "persistent"}[v]


def route(x, w_router, k, w_shared_gate=None, logit_bias=None, want_logits=False, want_hist=False):
    """Router (modeling:805-813). Returns (logits|None, idx int32 [T,k], w [T,k],
    shared_gate_logit [T]|None, hist int32 [ceil(T/64),E]|None); floats in x's dtype (bf16/fp32)."""
    dt = _fdt(x, "x")
    _need(x, "x", dtype=dt, ndim=2)
    _need(w_router, "w_router", dtype=dt, ndim=2)
    T, h = x.shape
    E = w_router.shape[0]
    if w_router.shape[1] != h:
        raise ValueError(f"w_router {tuple(w_router.shape)} does not match hidden {h}")
    dev = x.device
    if w_shared_gate is not None:
        _need(w_shared_gate, "w_shared_gate", dtype=dt)
        if w_shared_gate.numel() != h:
            raise ValueError("w_shared_gate must hold h elements")
    if logit_bias is not None:
        _need(logit_bias, "logit_bias", dtype=torch.float32, ndim=1)
        if logit_bias.numel() != E:
            raise ValueError("logit_bias must hold E elements")
    # fp32: the selection reads the logits back, so they are always materialised.
    logits = torch.empty(T, E, dtype=dt, device=dev) if want_logits or dt == torch.float32 else None
    idx = torch.empty(T, k, dtype=torch.int32, device=dev)
    w = torch.empty(T, k, dtype=dt, device=dev)
    gate = torch.empty(T, dtype=dt, device=dev) if w_shared_gate is not None else None
    hist = torch.empty((T + 63) // 64, E, dtype=torch.int32, device=dev) if want_hist else None
    check(lib.q38moe_route(_ptr(x), _ptr(w_router), _ptr(w_shared_gate), _ptr(logit_bias), _ptr(logits),
                           _ptr(idx), _ptr(w), _ptr(gate), _ptr(hist), T, h, E, k, _DTYPES[dt], _stream(dev)),
          "q38moe_route")
    return (logits if want_logits else None), idx, w, gate, hist


def route_from_logits(logits, k, logit_bias=None, want_hist=False):
    """Router selection (modeling:808-812) on given bf16 or fp32 logits [T,E]: (idx int32, w in the
    logits' dtype, hist)."""
    dt = _fdt(logits, "logits")
    _need(logits, "logits", dtype=dt, ndim=2)
    T, E = logits.shape
    dev = logits.device
    if logit_bias is not None:
        _need(logit_bias, "logit_bias", dtype=torch.float32, ndim=1)
    idx = torch.empty(T, k, dtype=torch.int32, device=dev)
    w = torch.empty(T, k, dtype=dt, device=dev)
    hist = torch.empty((T + 63) // 64, E, dtype=torch.int32, device=dev) if want_hist else None
    check(lib.q38moe_route_from_logits(_ptr(logits), _ptr(logit_bias), _ptr(idx), _ptr(w), _ptr(hist),
                                       T, E, k, _DTYPES[dt], _stream(dev)), "q38moe_route_from_logits")
    return idx, w, hist


def histogram(idx, E):
    """Per-64-token-block expert counts of routing indices idx [T,k] (int32/int64)."""
    _need(idx, "topk_idx", dtype=None, ndim=2)
    T, k = idx.shape
    hist = torch.empty((T + 63) // 64, E, dtype=torch.int32, device=idx.device)
    check(lib.q38moe_histogram(_ptr(idx), _idx_flag(idx), _ptr(hist), T, E, k, _stream(idx.device)),
          "q38moe_histogram")
    return hist


def permute(idx, hist, E, shared_rows=0):
    """Stable counting sort of pairs by expert (inference.py:163-171).

    Returns (counts [E], starts [E], perm [T*k], inv [T*k], tiles [max_tiles, 4], tile_count [1]);
    with shared_rows > 0 the tile table ends with the shared-expert rows T*k .. T*k+shared_rows.
    """
    _need(idx, "topk_idx", dtype=None, ndim=2)
    _need(hist, "hist", dtype=torch.int32, ndim=2)
    T, k = idx.shape
    dev = idx.device
    counts = torch.empty(E, dtype=torch.int32, device=dev)
    starts = torch.empty(E, dtype=torch.int32, device=dev)
    perm = torch.empty(T * k, dtype=torch.int32, device=dev)
    inv = torch.empty(T * k, dtype=torch.int32, device=dev)
    tiles = torch.empty(max_tiles(T, E, k, shared_rows), 4, dtype=torch.int32, device=dev)
    tile_count = torch.empty(1, dtype=torch.int32, device=dev)
    check(lib.q38moe_permute(_ptr(idx), _idx_flag(idx), _ptr(hist), _ptr(counts), _ptr(starts), _ptr(perm),
                             _ptr(inv), _ptr(tiles), _ptr(tile_count), shared_rows, T, E, k, _stream(dev)),
          "q38moe_permute")
    return counts, starts, perm, inv, tiles, tile_count


def gate_up(x, w_gate_up, perm, tiles, tile_count, k, shared_weights=None, shared_rows=0):
    """Grouped gate/up GEMM + SwiGLU (inference.py:60-96): H [T*k + shared_rows, I] bf16, rows in
    expert-sorted order then the shared-expert rows (shared_weights = (gate_proj.weight, up_proj.weight));
    fp32 inputs give fp32 H (no roundings)."""
    dt = _fdt(x, "x")
    _need(x, "x", dtype=dt, ndim=2)
    _need(w_gate_up, "w_gate_up", dtype=dt, ndim=3)
    _need(perm, "perm", dtype=torch.int32)
    _need(tiles, "tiles", dtype=torch.int32, ndim=2)
    T, h = x.shape
    E, twoI, hh = w_gate_up.shape
    if hh != h or twoI % 2:
        raise ValueError(f"w_gate_up {tuple(w_gate_up.shape)} does not match hidden {h}")
    I = twoI // 2
    if tiles.shape[0] != max_tiles(T, E, k, shared_rows):
        raise ValueError("tiles was not built for this shape")
    wg = wu = None
    if shared_rows:
        wg, wu = shared_weights
        _need(wg, "shared gate_proj", dtype=dt, ndim=2)
        _need(wu, "shared up_proj", dtype=dt, ndim=2)
        if wg.shape != (I, h) or wu.shape != (I, h):
            raise ValueError("the shared expert runs inside the grouped GEMM only when its width equals I")
    H = torch.empty(T * k + shared_rows, I, dtype=dt, device=x.device)
    check(lib.q38moe_gate_up(_ptr(x), _ptr(w_gate_up), _ptr(wg), _ptr(wu), _ptr(perm), _ptr(tiles), _ptr(tile_count),
                             shared_rows, _ptr(H), T, h, E, k, I, _DTYPES[dt], _stream(x.device)), "q38moe_gate_up")
    return H


def down(H, w_down, tiles, tile_count, T, k, w_shared_down=None, shared_rows=0):
    """Grouped down GEMM (inference.py:99-127, routing weight left to combine): Y [rows, h] in H's
    dtype (bf16 or fp32)."""
    dt = _fdt(H, "H")
    _need(H, "H", dtype=dt, ndim=2)
    _need(w_down, "w_down", dtype=dt, ndim=3)
    _need(tiles, "tiles", dtype=torch.int32, ndim=2)
    E, h, I = w_down.shape
    if H.shape != (T * k + shared_rows, I):
        raise ValueError(f"H {tuple(H.shape)} does not match ({T * k + shared_rows}, {I})")
    if tiles.shape[0] != max_tiles(T, E, k, shared_rows):
        raise ValueError("tiles was not built for this shape")
    if shared_rows:
        _need(w_shared_down, "shared down_proj", dtype=dt, ndim=2)
    Y = torch.empty(T * k + shared_rows, h, dtype=dt, device=H.device)
    check(lib.q38moe_down(_ptr(H), _ptr(w_down), _ptr(w_shared_down), _ptr(tiles), _ptr(tile_count), shared_rows,
                          _ptr(Y), T, h, E, k, I, _DTYPES[dt], _stream(H.device)), "q38moe_down")
    return Y


def shared_expert(x, w_gate, w_up, w_down):
    """Qwen3_8MoeMLP.forward (modeling:751-753) on x [T,h]: [T,h] in x's dtype (bf16 or fp32)."""
    dt = _fdt(x, "x")
    _need(x, "x", dtype=dt, ndim=2)
    for t, n in ((w_gate, "w_gate"), (w_up, "w_up"), (w_down, "w_down")):
        _need(t, n, dtype=dt, ndim=2)
    T, h = x.shape
    Is = w_gate.shape[0]
    if w_gate.shape != (Is, h) or w_up.shape != (Is, h) or w_down.shape != (h, Is):
        raise ValueError("shared expert weights must be [Is,h], [Is,h], [h,Is]")
    Hs = torch.empty(T, Is, dtype=dt, device=x.device)
    out = torch.empty(T, h, dtype=dt, device=x.device)
    check(lib.q38moe_shared_expert(_ptr(x), _ptr(w_gate), _ptr(w_up), _ptr(w_down), _ptr(Hs), _ptr(out), T, h,
                                   Is, _DTYPES[dt], _stream(x.device)), "q38moe_shared_expert")
    return out


def combine(Y, inv, topk_w, E, idx=None, shared_out=None, shared_gate_logit=None):
    """out[t] = bf16(sum_j bf16(Y[inv[t*k+j]] * w[t,j])) (inference.py:128-130,199), optionally plus
    the sigmoid-gated shared-expert row (modeling:831-833); fp32 Y gives the fp32 sum without
    roundings."""
    dt = _fdt(Y, "Y")
    _need(Y, "Y", dtype=dt, ndim=2)
    _need(inv, "inv", dtype=torch.int32)
    _need(topk_w, "topk_w", dtype=dt, ndim=2)
    T, k = topk_w.shape
    h = Y.shape[1]
    flag = 0
    if idx is not None:
        _need(idx, "topk_idx", dtype=None, ndim=2)
        flag = _idx_flag(idx)
    if shared_out is not None:
        _need(shared_out, "shared_out", dtype=dt, ndim=2)
        _need(shared_gate_logit, "shared_gate_logit", dtype=dt)
    out = torch.empty(T, h, dtype=dt, device=Y.device)
    check(lib.q38moe_combine(_ptr(Y), _ptr(inv), _ptr(idx), flag, _ptr(topk_w), _ptr(shared_out),
                             _ptr(shared_gate_logit), _ptr(out), T, h, E, k, _DTYPES[dt], _stream(Y.device)),
          "q38moe_combine")
    return out


def gather_gemm(x, perm, w, tiles, tile_count, k):
    """C[r] = bf16(x[perm[r] // k] . w[e]^T) over the T*k sorted rows of a tile table built without
    shared-expert rows (the gate/up pre-activations [g | u] when w is gate_up_proj): [T*k, N] bf16."""
    _need(x, "x", ndim=2)
    _need(perm, "perm", dtype=torch.int32)
    _need(w, "w", ndim=3)
    _need(tiles, "tiles", dtype=torch.int32, ndim=2)
    T, K = x.shape
    E, N, KK = w.shape
    if KK != K:
        raise ValueError(f"w {tuple(w.shape)} does not match x {tuple(x.shape)}")
    if perm.numel() != T * k or tiles.shape[0] != max_tiles(T, E, k, 0):
        raise ValueError("perm/tiles were not built for this shape (without shared rows)")
    C = torch.empty(T * k, N, dtype=torch.bfloat16, device=x.device)
    check(lib.q38moe_gather_gemm(_ptr(x), _ptr(perm), _ptr(w), _ptr(tiles), _ptr(tile_count), _ptr(C), T, K, N, E,
                                 k, _stream(x.device)), "q38moe_gather_gemm")
    return C


def pair_dots(dout, Y, inv, idx, E, w=None):
    """Routing-weight gradient dw[t, j] = <dout[t], Y[inv[t*k+j]]> (bf16 products, fp32 sum): [T,k] bf16.
    With w (top_k_weights [T,k]) also returns, from the same pass, the routed raw rows' gradient in
    sorted order, d_raw[inv[p]] = bf16(dout[t] * w[p]) [T*k, h] (rows of dropped pairs unwritten)."""
    _need(dout, "dout", ndim=2)
    _need(Y, "Y", ndim=2)
    _need(inv, "inv", dtype=torch.int32)
    _need(idx, "topk_idx", dtype=None, ndim=2)
    T, h = dout.shape
    k = idx.shape[1]
    dw = torch.empty(T, k, dtype=torch.bfloat16, device=dout.device)
    d_raw = None
    if w is not None:
        _need(w, "topk_w", ndim=2)
        d_raw = torch.empty(T * k, h, dtype=torch.bfloat16, device=dout.device)
    check(lib.q38moe_pair_dots(_ptr(dout), _ptr(Y), _ptr(inv), _ptr(idx), _idx_flag(idx), _ptr(w), _ptr(dw),
                               _ptr(d_raw), T, h, E, k, _stream(dout.device)), "q38moe_pair_dots")
    return dw if w is None else (dw, d_raw)


def gather_rows(src, perm, starts, counts, k, w=None):
    """Sorted rows bf16(src[perm[r] // k] * w[perm[r]]) (w [T,k] or None) in a [T*k, h] bf16 tensor;
    only the rows the permutation filled (starts[E-1] + counts[E-1], read on the device) are
    written, the slots of dropped pairs are left as they were."""
    _need(src, "src", ndim=2)
    _need(perm, "perm", dtype=torch.int32)
    _need(starts, "starts", dtype=torch.int32)
    _need(counts, "counts", dtype=torch.int32)
    if w is not None:
        _need(w, "w")
    T, h = src.shape
    if perm.numel() != T * k:
        raise ValueError("perm must hold T*k entries")
    dst = torch.empty(T * k, h, dtype=torch.bfloat16, device=src.device)
    check(lib.q38moe_gather_rows(_ptr(src), _ptr(perm), _ptr(w), _ptr(starts), _ptr(counts), _ptr(dst), T, h,
                                 counts.numel(), k, _stream(src.device)), "q38moe_gather_rows")
    return dst


def gate_up_save(x, w_gate_up, perm, tiles, tile_count, k):
    """Grouped gate/up + SwiGLU on routed rows that also returns the rounded pre-activations
    (q38moe_gate_up_save): (H [T*k, I], GU [T*k, 2I] = [g | u]) bf16, GU bit-identical to
    ``gather_gemm(x, perm, w_gate_up, ...)``. The tile table must hold no shared-expert rows."""
    _need(x, "x", dtype=torch.bfloat16, ndim=2)
    _need(w_gate_up, "w_gate_up", dtype=torch.bfloat16, ndim=3)
    _need(perm, "perm", dtype=torch.int32)
    _need(tiles, "tiles", dtype=torch.int32, ndim=2)
    T, h = x.shape
    E, twoI, hw = w_gate_up.shape
    if hw != h:
        raise ValueError(f"w_gate_up {tuple(w_gate_up.shape)} does not match x {tuple(x.shape)}")
    if tiles.shape[0] != max_tiles(T, E, k, 0):
        raise ValueError("tiles was not built for this shape (without shared-expert rows)")
    I = twoI // 2
    H = torch.empty(T * k, I, dtype=torch.bfloat16, device=x.device)
    GU = torch.empty(T * k, twoI, dtype=torch.bfloat16, device=x.device)
    check(lib.q38moe_gate_up_save(_ptr(x), _ptr(w_gate_up), _ptr(perm), _ptr(tiles), _ptr(tile_count), _ptr(H),
                                  _ptr(GU), T, h, E, k, I, _stream(x.device)), "q38moe_gate_up_save")
    return H, GU


def down_kn(A, w_kn, tiles, tile_count, T, k):
    """Grouped product with K-major expert weights (q38moe_down_kn): Y[r] = bf16(A[r] . w_kn[e]) for
    the T*k sorted rows, w_kn [E, K, N] as stored (down_proj for dH, gate_up_proj for the input rows'
    gradient). Bit-identical to ``down(A, transpose_experts(w_kn), ...)`` without the transpose.
    A [T*k, K] bf16; returns Y [T*k, N] bf16. The tile table must hold no shared-expert rows."""
    _need(A, "A", dtype=torch.bfloat16, ndim=2)
    _need(w_kn, "w_kn", dtype=torch.bfloat16, ndim=3)
    _need(tiles, "tiles", dtype=torch.int32, ndim=2)
    E, K, N = w_kn.shape
    if A.shape != (T * k, K):
        raise ValueError(f"A {tuple(A.shape)} does not match ({T * k}, {K})")
    if tiles.shape[0] != max_tiles(T, E, k, 0):
        raise ValueError("tiles was not built for this shape (without shared-expert rows)")
    Y = torch.empty(T * k, N, dtype=torch.bfloat16, device=A.device)
    check(lib.q38moe_down_kn(_ptr(A), _ptr(w_kn), _ptr(tiles), _ptr(tile_count), _ptr(Y), T, K, N, E, k,
                             _stream(A.device)), "q38moe_down_kn")
    return Y


def transpose_experts(w):
    """w [E, R, C] bf16 -> contiguous [E, C, R] (each expert's matrix transposed)."""
    _need(w, "w", ndim=3)
    E, R, C = w.shape
    out = torch.empty(E, C, R, dtype=w.dtype, device=w.device)
    check(lib.q38moe_transpose_experts(_ptr(w), _ptr(out), E, R, C, _stream(w.device)), "q38moe_transpose_experts")
    return out


def expert_wgrad(G, X, starts, counts, k, perm=None):
    """Expert weight gradients dW[e] = G_e^T . X_e over each expert's sorted rows: X [T,N] tokens
    gathered through perm (gate_up_proj's gradient, G = [d_g | d_u]) or, with perm None, X [T*k,N]
    in sorted order (down_proj's, X = H). G [T*k, M]. Returns [E, M, N] bf16."""
    _need(G, "G", ndim=2)
    _need(X, "X", ndim=2)
    _need(starts, "starts", dtype=torch.int32)
    _need(counts, "counts", dtype=torch.int32)
    P, M = G.shape
    N = X.shape[1]
    E = counts.numel()
    if perm is not None:
        _need(perm, "perm", dtype=torch.int32)
        if perm.numel() != P or P != X.shape[0] * k:
            raise ValueError("perm must hold T*k entries for X [T, N]")
    elif X.shape[0] != P:
        raise ValueError("without perm, X must hold the G's sorted rows")
    T = P // k
    dW = torch.empty(E, M, N, dtype=torch.bfloat16, device=G.device)
    check(lib.q38moe_expert_wgrad(_ptr(G), _ptr(X), _ptr(perm), _ptr(starts), _ptr(counts), _ptr(dW), T, M, N, E, k,
                                  _stream(G.device)), "q38moe_expert_wgrad")
    return dW


def swiglu_backward(dH, GU):
    """[d_g | d_u] from dH [rows, I] and the pre-activations GU = [g | u] [rows, 2I]: [rows, 2I] bf16."""
    _need(dH, "dH", ndim=2)
    _need(GU, "GU", ndim=2)
    rows, I = dH.shape
    if GU.shape != (rows, 2 * I):
        raise ValueError(f"GU {tuple(GU.shape)} does not match dH {tuple(dH.shape)}")
    dGU = torch.empty(rows, 2 * I, dtype=torch.bfloat16, device=dH.device)
    check(lib.q38moe_swiglu_backward(_ptr(dH), _ptr(GU), _ptr(dGU), rows, I, _stream(dH.device)),
          "q38moe_swiglu_backward")
    return dGU


def experts_workspace_bytes(T, h, E, k, I, dtype=torch.bfloat16):
    n = ctypes.c_size_t()
    check(lib.q38moe_experts_workspace_bytes(T, h, E, k, I, _DTYPES[dtype], ctypes.byref(n)),
          "q38moe_experts_workspace_bytes")
    return n.value


def experts_forward(x, topk_idx, topk_w, w_gate_up, w_down, workspace=None):
    """Routed experts (ExpertsInterface contract, integrations/moe.py:567-570): [T,h] in the
    activations' dtype (bf16, or fp32 without intermediate roundings)."""
    dt = _fdt(x, "hidden_states")
    _need(x, "hidden_states", dtype=dt, ndim=2)
    _need(topk_idx, "top_k_index", dtype=None, ndim=2)
    _need(topk_w, "top_k_weights", dtype=dt, ndim=2)
    _need(w_gate_up, "gate_up_proj", dtype=dt, ndim=3)
    _need(w_down, "down_proj", dtype=dt, ndim=3)
    T, h = x.shape
    k = topk_idx.shape[1]
    E, twoI, _ = w_gate_up.shape
    I = twoI // 2
    if topk_w.shape != topk_idx.shape or topk_idx.shape[0] != T:
        raise ValueError("top_k_index/top_k_weights must both be [T,k]")
    nbytes = experts_workspace_bytes(T, h, E, k, I, dt)
    if workspace is None or workspace.numel() < nbytes:
        workspace = torch.empty(nbytes, dtype=torch.uint8, device=x.device)
    out = torch.empty(T, h, dtype=dt, device=x.device)
    check(lib.q38moe_experts_forward(_ptr(x), _ptr(topk_idx), _idx_flag(topk_idx), _ptr(topk_w), _ptr(w_gate_up),
                                     _ptr(w_down), _ptr(out), T, h, E, k, I, _ptr(workspace), workspace.numel(),
                                     _DTYPES[dt], _stream(x.device)), "q38moe_experts_forward")
    return out


def block_workspace_bytes(T, h, E, k, I, Is, dtype=torch.bfloat16):
    n = ctypes.c_size_t()
    check(lib.q38moe_block_workspace_bytes(T, h, E, k, I, Is, _DTYPES[dtype], ctypes.byref(n)),
          "q38moe_block_workspace_bytes")
    return n.value


def block_forward(x, w_router, w_gate_up, w_down, w_sh_gate, w_sh_up, w_sh_down, w_sh_gate_proj, k,
                  logit_bias=None, return_router=False, workspace=None, out=None):
    """Qwen3_8MoeSparseMoeBlock.forward (modeling:824-835) on x [T,h]. Returns out [T,h], or
    (out, logits [T,E], idx int32 [T,k], w [T,k]) with return_router; floats in x's dtype (bf16, or
    fp32 computed without intermediate roundings)."""
    dt = _fdt(x, "x")
    _need(x, "x", dtype=dt, ndim=2)
    for t, n in ((w_router, "w_router"), (w_sh_gate, "w_sh_gate"), (w_sh_up, "w_sh_up"),
                 (w_sh_down, "w_sh_down")):
        _need(t, n, dtype=dt, ndim=2)
    _need(w_gate_up, "w_gate_up", dtype=dt, ndim=3)
    _need(w_down, "w_down", dtype=dt, ndim=3)
    _need(w_sh_gate_proj, "w_sh_gate_proj", dtype=dt)
    T, h = x.shape
    E = w_router.shape[0]
    I = w_gate_up.shape[1] // 2
    Is = w_sh_gate.shape[0]
    if w_gate_up.shape != (E, 2 * I, h) or w_down.shape != (E, h, I) or w_router.shape != (E, h):
        raise ValueError("expert weights must be [E,2I,h] and [E,h,I], router [E,h]")
    if w_sh_gate.shape != (Is, h) or w_sh_up.shape != (Is, h) or w_sh_down.shape != (h, Is):
        raise ValueError("shared expert weights must be [Is,h], [Is,h], [h,Is]")
    if w_sh_gate_proj.numel() != h:
        raise ValueError("shared_expert_gate weight must hold h elements")
    if logit_bias is not None:
        _need(logit_bias, "logit_bias", dtype=torch.float32, ndim=1)
    dev = x.device
    nbytes = block_workspace_bytes(T, h, E, k, I, Is, dt)
    if workspace is None or workspace.numel() < nbytes:
        workspace = torch.empty(nbytes, dtype=torch.uint8, device=dev)
    if out is None:
        out = torch.empty(T, h, dtype=dt, device=dev)
    logits = idx = w = None
    if return_router:
        logits = torch.empty(T, E, dtype=dt, device=dev)
        idx = torch.empty(T, k, dtype=torch.int32, device=dev)
        w = torch.empty(T, k, dtype=dt, device=dev)
    check(lib.q38moe_block_forward(_ptr(x), _ptr(w_router), _ptr(w_gate_up), _ptr(w_down), _ptr(w_sh_gate),
                                   _ptr(w_sh_up), _ptr(w_sh_down), _ptr(w_sh_gate_proj), _ptr(logit_bias), _ptr(out),
                                   _ptr(logits), _ptr(idx), _ptr(w), T, h, E, k, I, Is, _ptr(workspace),
                                   workspace.numel(), _DTYPES[dt], _stream(dev)), "q38moe_block_forward")
    if return_router:
        return out, logits, idx, w
    return out


def block_forward_noalloc(x, w_router, w_gate_up, w_down, w_sh_gate, w_sh_up, w_sh_down, w_sh_gate_proj, k,
                          logit_bias=None, out=None, logits=None, idx=None, w=None):
    """block_forward through q38moe_block_forward_noalloc: the library's static per-GPU scratch
    instead of a workspace, no allocation inside the call. Outputs are the caller's (allocated
    here only when not given): out [T,h] bf16 and, optionally, logits [T,E] bf16, idx [T,k] int32,
    w [T,k] bf16. Raises RuntimeError when T exceeds what the scratch holds."""
    dt = _fdt(x, "x")
    _need(x, "x", dtype=dt, ndim=2)
    T, h = x.shape
    E = w_router.shape[0]
    I = w_gate_up.shape[1] // 2
    Is = w_sh_gate.shape[0]
    if w_gate_up.shape != (E, 2 * I, h) or w_down.shape != (E, h, I) or w_router.shape != (E, h):
        raise ValueError("expert weights must be [E,2I,h] and [E,h,I], router [E,h]")
    if w_sh_gate.shape != (Is, h) or w_sh_up.shape != (Is, h) or w_sh_down.shape != (h, Is):
        raise ValueError("shared expert weights must be [Is,h], [Is,h], [h,Is]")
    for t, n in ((w_router, "w_router"), (w_gate_up, "w_gate_up"), (w_down, "w_down"), (w_sh_gate, "w_sh_gate"),
                 (w_sh_up, "w_sh_up"), (w_sh_down, "w_sh_down"), (w_sh_gate_proj, "w_sh_gate_proj")):
        _need(t, n, dtype=dt)
    if logit_bias is not None:
        _need(logit_bias, "logit_bias", dtype=torch.float32, ndim=1)
    dev = x.device
    if out is None:
        out = torch.empty(T, h, dtype=dt, device=dev)
    for t, n, shape, tdt in ((out, "out", (T, h), dt), (logits, "logits", (T, E), dt),
                             (idx, "idx", (T, k), torch.int32), (w, "w", (T, k), dt)):
        if t is not None:
            _need(t, n, dtype=tdt)
            if tuple(t.shape) != shape:
                raise ValueError(f"{n} must be {shape}")
    check(lib.q38moe_block_forward_noalloc(_ptr(x), _ptr(w_router), _ptr(w_gate_up), _ptr(w_down), _ptr(w_sh_gate),
                                           _ptr(w_sh_up), _ptr(w_sh_down), _ptr(w_sh_gate_proj), _ptr(logit_bias),
                                           _ptr(out), _ptr(logits), _ptr(idx), _ptr(w), T, h, E, k, I, Is,
                                           _DTYPES[dt], _stream(dev)), "q38moe_block_forward_noalloc")
    return out


# ---- fp8 expert path (R14: e4m3 experts with per-output-channel scales; no reference function) ----

FP8_WEIGHT_NAMES = ("experts.gate_up_proj", "experts.down_proj", "shared_expert.gate_proj.weight",
                    "shared_expert.up_proj.weight", "shared_expert.down_proj.weight")


def quantize_rows(x):
    """Per-row e4m3 quantisation of x [..., C] bf16 (C % 64 == 0, C <= 4096): returns
    (q uint8 [..., C] = torch.float8_e4m3fn bit patterns, scale fp32 [...]) with x ~ q * scale
    (amax/448 per row, round-to-nearest-even, saturating at +-448)."""
    _need(x, "x", dtype=torch.bfloat16)
    C = x.shape[-1]
    R = x.numel() // C if C else 0
    q = torch.empty(x.shape, dtype=torch.uint8, device=x.device)
    scale = torch.empty(x.shape[:-1], dtype=torch.float32, device=x.device)
    check(lib.q38moe_quantize_rows(_ptr(x), _ptr(q), _ptr(scale), R, C, _stream(x.device)), "q38moe_quantize_rows")
    return q, scale


def quantize_weights_fp8(params):
    """e4m3 copies of the expert weights of a MoE block's state dict (per-output-channel scales):
    {name: (q uint8, scale fp32)} for the routed gate_up [E,2I,h] / down [E,h,I] projections and the
    shared expert's gate/up [I,h] and down [h,I] projections. Done once, at load time."""
    return {n: quantize_rows(params[n].contiguous()) for n in FP8_WEIGHT_NAMES}


def gate_up_fp8(xq, row_scale, wq, perm, tiles, tile_count, k, shared_rows=0):
    """Grouped gate/up GEMM on e4m3 (q38moe_gate_up_fp8): xq [T,h] uint8 e4m3 tokens, row_scale
    [T*k + shared_rows] fp32 in sorted row order, wq = quantize_weights_fp8(...). H bf16."""
    _need(xq, "xq", dtype=torch.uint8, ndim=2)
    _need(row_scale, "row_scale", dtype=torch.float32, ndim=1)
    qg, sg = wq["experts.gate_up_proj"]
    T, h = xq.shape
    E, twoI, _ = qg.shape
    I = twoI // 2
    if row_scale.numel() != T * k + shared_rows:
        raise ValueError("row_scale must hold T*k + shared_rows entries")
    (qsg, ssg), (qsu, ssu) = wq["shared_expert.gate_proj.weight"], wq["shared_expert.up_proj.weight"]
    H = torch.empty(T * k + shared_rows, I, dtype=torch.bfloat16, device=xq.device)
    check(lib.q38moe_gate_up_fp8(_ptr(xq), _ptr(row_scale), _ptr(qg), _ptr(sg), _ptr(qsg), _ptr(ssg), _ptr(qsu),
                                 _ptr(ssu), _ptr(perm), _ptr(tiles), _ptr(tile_count), shared_rows, _ptr(H), T, h, E,
                                 k, I, _stream(xq.device)), "q38moe_gate_up_fp8")
    return H


def down_fp8(Hq, row_scale, wq, tiles, tile_count, T, k, shared_rows=0):
    """Grouped down GEMM on e4m3 (q38moe_down_fp8): Hq [T*k + shared_rows, I] uint8, row_scale per
    row; Y bf16 [rows, h]."""
    _need(Hq, "Hq", dtype=torch.uint8, ndim=2)
    _need(row_scale, "row_scale", dtype=torch.float32, ndim=1)
    qd, sd = wq["experts.down_proj"]
    E, h, I = qd.shape
    qsd, ssd = wq["shared_expert.down_proj.weight"]
    Y = torch.empty(T * k + shared_rows, h, dtype=torch.bfloat16, device=Hq.device)
    check(lib.q38moe_down_fp8(_ptr(Hq), _ptr(row_scale), _ptr(qd), _ptr(sd), _ptr(qsd), _ptr(ssd), _ptr(tiles),
                              _ptr(tile_count), shared_rows, _ptr(Y), T, h, E, k, I, _stream(Hq.device)),
          "q38moe_down_fp8")
    return Y


def block_fp8_workspace_bytes(T, h, E, k, I):
    n = ctypes.c_size_t()
    check(lib.q38moe_block_fp8_workspace_bytes(T, h, E, k, I, ctypes.byref(n)), "q38moe_block_fp8_workspace_bytes")
    return n.value


def block_forward_fp8(x, w_router, wq, w_sh_gate_proj, k, logit_bias=None, return_router=False, workspace=None,
                      out=None):
    """The MoE block with e4m3 experts (q38moe_block_forward_fp8): bf16 router and shared gate,
    per-token e4m3 tokens, e4m3 gate/up and down GEMMs with the weights of quantize_weights_fp8."""
    _need(x, "x", ndim=2)
    _need(w_router, "w_router", ndim=2)
    _need(w_sh_gate_proj, "w_sh_gate_proj")
    T, h = x.shape
    E = w_router.shape[0]
    (qg, sg), (qd, sd) = wq["experts.gate_up_proj"], wq["experts.down_proj"]
    (qsg, ssg), (qsu, ssu), (qsd, ssd) = (wq["shared_expert.gate_proj.weight"], wq["shared_expert.up_proj.weight"],
                                          wq["shared_expert.down_proj.weight"])
    I = qg.shape[1] // 2
    if qg.shape != (E, 2 * I, h) or qd.shape != (E, h, I) or qsg.shape != (I, h) or qsd.shape != (h, I):
        raise ValueError("fp8 weights must be gate_up [E,2I,h], down [E,h,I], shared [I,h]/[h,I] (Is == I)")
    if logit_bias is not None:
        _need(logit_bias, "logit_bias", dtype=torch.float32, ndim=1)
    dev = x.device
    nbytes = block_fp8_workspace_bytes(T, h, E, k, I)
    if workspace is None or workspace.numel() < nbytes:
        workspace = torch.empty(nbytes, dtype=torch.uint8, device=dev)
    if out is None:
        out = torch.empty(T, h, dtype=torch.bfloat16, device=dev)
    logits = idx = w = None
    if return_router:
        logits = torch.empty(T, E, dtype=torch.bfloat16, device=dev)
        idx = torch.empty(T, k, dtype=torch.int32, device=dev)
        w = torch.empty(T, k, dtype=torch.bfloat16, device=dev)
    check(lib.q38moe_block_forward_fp8(_ptr(x), _ptr(w_router), _ptr(qg), _ptr(sg), _ptr(qd), _ptr(sd), _ptr(qsg),
                                       _ptr(ssg), _ptr(qsu), _ptr(ssu), _ptr(qsd), _ptr(ssd), _ptr(w_sh_gate_proj),
                                       _ptr(logit_bias), _ptr(out), _ptr(logits), _ptr(idx), _ptr(w), T, h, E, k, I,
                                       _ptr(workspace), workspace.numel(), _stream(dev)), "q38moe_block_forward_fp8")
    if return_router:
        return out, logits, idx, w
    return out
