"""ctypes binding of libq38moe.so (the C ABI declared in include/q38moe.h).

The library is loaded after ``import torch`` so that its libamdhip64.so.7 dependency resolves to
the HIP runtime torch already loaded (same SONAME): device pointers and streams are shared with
torch. There is no fallback: a missing or stale library raises at import.
"""
import ctypes
import os
from pathlib import Path

import torch  # noqa: F401  (loads the HIP runtime first)

LIB_PATH = Path(os.environ.get("Q38MOE_LIB", Path(__file__).resolve().parent / "libq38moe.so"))

ABI_VERSION = 13
BF16 = 1
FP32 = 2
TILING_PERSISTENT = 1
TILING_SMALL = 2

_c_int, _c_i32, _c_i64, _c_size, _vp = ctypes.c_int, ctypes.c_int32, ctypes.c_int64, ctypes.c_size_t, ctypes.c_void_p

# name -> (restype, argtypes); must match include/q38moe.h.
SIGNATURES = {
    "q38moe_abi_version": (_c_int, []),
    "q38moe_last_error": (ctypes.c_char_p, []),
    "q38moe_route": (_c_int, [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp,
                              _c_i64, _c_i32, _c_i32, _c_i32, _c_i32, _vp]),
    "q38moe_route_from_logits": (_c_int, [_vp, _vp, _vp, _vp, _vp, _c_i64, _c_i32, _c_i32, _c_i32, _vp]),
    "q38moe_histogram": (_c_int, [_vp, _c_i32, _vp, _c_i64, _c_i32, _c_i32, _vp]),
    "q38moe_permute": (_c_int, [_vp, _c_i32, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _c_i64, _c_i64, _c_i32, _c_i32,
                                _vp]),
    "q38moe_max_tiles": (_c_i64, [_c_i64, _c_i32, _c_i32, _c_i64]),
    "q38moe_gemm_block_m": (_c_i32, []),
    "q38moe_gemm_tiling": (_c_i32, [_c_i64, _c_i32, _c_i32, _c_i32, _c_i32, _c_i64]),
    "q38moe_gemm_tiling_fp8": (_c_i32, [_c_i64, _c_i32, _c_i32, _c_i32, _c_i32, _c_i64]),
    "q38moe_gate_up": (_c_int, [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _c_i64, _vp, _c_i64, _c_i32, _c_i32, _c_i32,
                                _c_i32, _c_i32, _vp]),
    "q38moe_down": (_c_int, [_vp, _vp, _vp, _vp, _vp, _c_i64, _vp, _c_i64, _c_i32, _c_i32, _c_i32, _c_i32, _c_i32,
                             _vp]),
    "q38moe_shared_expert": (_c_int, [_vp, _vp, _vp, _vp, _vp, _vp, _c_i64, _c_i32, _c_i32, _c_i32, _vp]),
    "q38moe_combine": (_c_int, [_vp, _vp, _vp, _c_i32, _vp, _vp, _vp, _vp, _c_i64, _c_i32, _c_i32, _c_i32, _c_i32,
                                _vp]),
    "q38moe_experts_workspace_bytes": (_c_int, [_c_i64, _c_i32, _c_i32, _c_i32, _c_i32, _c_i32,
                                                ctypes.POINTER(_c_size)]),
    "q38moe_experts_forward": (_c_int, [_vp, _vp, _c_i32, _vp, _vp, _vp, _vp, _c_i64, _c_i32, _c_i32, _c_i32,
                                        _c_i32, _vp, _c_size, _c_i32, _vp]),
    "q38moe_block_workspace_bytes": (_c_int, [_c_i64, _c_i32, _c_i32, _c_i32, _c_i32, _c_i32, _c_i32,
                                              ctypes.POINTER(_c_size)]),
    "q38moe_block_forward": (_c_int, [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp,
                                      _c_i64, _c_i32, _c_i32, _c_i32, _c_i32, _c_i32, _vp, _c_size, _c_i32, _vp]),
    "q38moe_block_noalloc_scratch_bytes": (_c_size, []),
    "q38moe_block_forward_noalloc": (_c_int, [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp,
                                              _c_i64, _c_i32, _c_i32, _c_i32, _c_i32, _c_i32, _c_i32, _vp]),
    "q38moe_quantize_rows": (_c_int, [_vp, _vp, _vp, _c_i64, _c_i32, _vp]),
    "q38moe_gate_up_fp8": (_c_int, [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _c_i64, _vp, _c_i64,
                                    _c_i32, _c_i32, _c_i32, _c_i32, _vp]),
    "q38moe_down_fp8": (_c_int, [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _c_i64, _vp, _c_i64, _c_i32, _c_i32,
                                 _c_i32, _c_i32, _vp]),
    "q38moe_block_fp8_workspace_bytes": (_c_int, [_c_i64, _c_i32, _c_i32, _c_i32, _c_i32, ctypes.POINTER(_c_size)]),
    "q38moe_block_forward_fp8": (_c_int, [_vp] * 18 + [_c_i64, _c_i32, _c_i32, _c_i32, _c_i32, _vp, _c_size, _vp]),
    "q38moe_gather_gemm": (_c_int, [_vp, _vp, _vp, _vp, _vp, _vp, _c_i64, _c_i32, _c_i32, _c_i32, _c_i32, _vp]),
    "q38moe_down_kn": (_c_int, [_vp, _vp, _vp, _vp, _vp, _c_i64, _c_i32, _c_i32, _c_i32, _c_i32, _vp]),
    "q38moe_gate_up_save": (_c_int, [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _c_i64, _c_i32, _c_i32, _c_i32, _c_i32,
                                     _vp]),
    "q38moe_pair_dots": (_c_int, [_vp] * 4 + [_c_i32, _vp, _vp, _vp, _c_i64, _c_i32, _c_i32, _c_i32, _vp]),
    "q38moe_gather_rows": (_c_int, [_vp] * 6 + [_c_i64, _c_i32, _c_i32, _c_i32, _vp]),
    "q38moe_transpose_experts": (_c_int, [_vp, _vp, _c_i32, _c_i32, _c_i32, _vp]),
    "q38moe_expert_wgrad": (_c_int, [_vp] * 6 + [_c_i64, _c_i32, _c_i32, _c_i32, _c_i32, _vp]),
    "q38moe_swiglu_backward": (_c_int, [_vp, _vp, _vp, _c_i64, _c_i32, _vp]),
}


def _load():
    if not LIB_PATH.exists():
        raise RuntimeError(
            f"{LIB_PATH} is not built: run `python qwen35-moe-sparse_amd/csrc/build.py` "
            "(or __graft_entry__.build()); the MoE path has no non-HIP fallback")
    lib = ctypes.CDLL(str(LIB_PATH))
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    ver = lib.q38moe_abi_version()
    if ver != ABI_VERSION:
        raise RuntimeError(f"{LIB_PATH} has ABI version {ver}, expected {ABI_VERSION}: rebuild it")
    return lib


lib = _load()


def check(rc, what):
    """Raise RuntimeError carrying the library's message when a call returned non-zero."""
    if rc != 0:
        msg = lib.q38moe_last_error().decode(errors="replace")
        raise RuntimeError(f"{what} failed ({rc}): {msg}")
