"""The C ABI library: loads, exports every entry point of include/q38moe.h, validates arguments on
the host. CPU only: no call here reaches a kernel launch."""
import ctypes
import os
import subprocess
import sys
import re
from pathlib import Path

import pytest

REPO = Path(__file__).resolve().parents[1]
HEADER = REPO / "include" / "q38moe.h"


def _declared():
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(q38moe_\w+)\s*\(", text)))


def _lib():
    from q38.hip import _lib
    return _lib


def test_header_symbols_exported():
    m = _lib()
    names = _declared()
    assert len(names) >= 15
    for n in names:
        assert hasattr(m.lib, n), f"{n} declared in q38moe.h but not exported"
    assert set(names) == set(m.SIGNATURES), "ctypes signatures and header disagree"


def test_abi_version():
    m = _lib()
    assert m.lib.q38moe_abi_version() == m.ABI_VERSION == 13


def test_max_tiles_and_block_m():
    m = _lib()
    bm = m.lib.q38moe_gemm_block_m()
    assert bm in (64, 128, 256)
    cd = lambda a, b: (a + b - 1) // b  # noqa: E731
    assert m.lib.q38moe_max_tiles(16384, 64, 5, 0) == cd(16384 * 5, bm) + 64
    assert m.lib.q38moe_max_tiles(16384, 64, 5, 16384) == cd(16384 * 5, bm) + 64 + cd(16384, bm)
    assert m.lib.q38moe_max_tiles(-1, 64, 5, 0) == -1


def test_gemm_tiling_rule():
    """Small tiles up to R pair rows per group on average (E experts, plus the shared group when its
    rows are fused), R = 32 at h = 1024, I = 256 and 20.16 at h = 2048, I = 512 (32 (2^18 / (h I))^(1/3)),
    for K in {128, ..., 2048} only; monotone in T; the environment override
    switches the row condition in a fresh process (the variable is read once)."""
    m = _lib()
    tiling = lambda T, sh, h=1024, E=64, k=5, I=256: m.lib.q38moe_gemm_tiling(T, h, E, k, I, sh)  # noqa: E731
    assert tiling(1, 1) == m.TILING_SMALL
    assert tiling(346, 346) == m.TILING_SMALL       # 346 * 6 = 2076 <= 32 * 65
    assert tiling(347, 347) == m.TILING_PERSISTENT
    assert tiling(409, 0) == m.TILING_SMALL         # 409 * 5 = 2045 <= 32 * 64
    assert tiling(410, 0) == m.TILING_PERSISTENT
    assert tiling(16384, 16384) == m.TILING_PERSISTENT
    assert tiling(1, 1, h=4096) == m.TILING_PERSISTENT
    assert tiling(1, 1, I=192) == m.TILING_PERSISTENT
    assert tiling(1, 1, h=2048, I=512) == m.TILING_SMALL
    assert tiling(218, 218, h=2048, I=512) == m.TILING_SMALL        # 218 * 6 = 1308 <= 20.16 * 65
    assert tiling(219, 219, h=2048, I=512) == m.TILING_PERSISTENT
    assert tiling(550, 550, h=512, I=128) == m.TILING_SMALL         # R = 50.8 at h I = 2^16
    assert tiling(551, 551, h=512, I=128) == m.TILING_PERSISTENT
    fp8 = lambda T, sh, h=2048, E=64, k=5, I=512: m.lib.q38moe_gemm_tiling_fp8(T, h, E, k, I, sh)  # noqa: E731
    assert fp8(272, 272) == m.TILING_SMALL       # F = 1.25 R = 25.2: 272 * 6 = 1632 <= 25.2 * 65
    assert fp8(273, 273) == m.TILING_PERSISTENT
    assert fp8(1, 1, h=256, I=64) == m.TILING_PERSISTENT   # e4m3 small tiles need K in {512, 1024, 2048}
    assert tiling(40, 40, E=8, k=2) == m.TILING_SMALL    # 120 <= 32 * 9
    assert tiling(100, 100, E=8, k=2) == m.TILING_PERSISTENT
    kinds = [tiling(T, T) for T in range(1, 5000, 7)]
    first_big = kinds.index(m.TILING_PERSISTENT)
    assert all(v == m.TILING_SMALL for v in kinds[:first_big])
    assert all(v == m.TILING_PERSISTENT for v in kinds[first_big:])
    code = ("import ctypes, sys; lib = ctypes.CDLL(sys.argv[1]); "
            "f = lib.q38moe_gemm_tiling; f.restype = ctypes.c_int32; "
            "f.argtypes = [ctypes.c_int64, ctypes.c_int32, ctypes.c_int32, ctypes.c_int32, ctypes.c_int32, ctypes.c_int64]; "
            "print(f(16384, 1024, 64, 5, 256, 16384), f(1, 1024, 64, 5, 256, 1), f(1, 4096, 64, 5, 256, 1))")
    for value, want in (("small", (m.TILING_SMALL, m.TILING_SMALL, m.TILING_PERSISTENT)),
                        ("persistent", (m.TILING_PERSISTENT,) * 3)):
        env = dict(os.environ, Q38MOE_GEMM_TILING=value)
        r = subprocess.run([sys.executable, "-c", code, str(m.LIB_PATH)], env=env, capture_output=True, text=True,
                           timeout=60)
        assert r.returncode == 0, r.stderr
        assert tuple(int(v) for v in r.stdout.split()) == want


def test_workspace_sizes():
    m = _lib()
    n = ctypes.c_size_t()
    assert m.lib.q38moe_experts_workspace_bytes(16384, 1024, 64, 5, 256, m.BF16, ctypes.byref(n)) == 0
    P = 16384 * 5
    assert n.value >= P * 256 * 2 + P * 1024 * 2 + P * 4
    nb = ctypes.c_size_t()
    assert m.lib.q38moe_block_workspace_bytes(16384, 1024, 64, 5, 256, 256, m.BF16, ctypes.byref(nb)) == 0
    assert nb.value > n.value
    # fp32 intermediates are twice as wide
    n32 = ctypes.c_size_t()
    assert m.lib.q38moe_experts_workspace_bytes(16384, 1024, 64, 5, 256, m.FP32, ctypes.byref(n32)) == 0
    assert n32.value >= P * 256 * 4 + P * 1024 * 4 + P * 4 and n32.value > n.value
    assert m.lib.q38moe_block_workspace_bytes(16384, 1024, 64, 5, 256, 256, 3, ctypes.byref(nb)) == -1


@pytest.mark.parametrize("T,h,E,k,I,msg", [
    (16, 1000, 64, 5, 256, "h must be"),
    (16, 1024, 65, 5, 256, "E must be"),
    (16, 1024, 64, 9, 256, "k must be"),
    (16, 1024, 4, 5, 256, "k must be"),
    (16, 1024, 64, 5, 100, "I must be"),
    (-1, 1024, 64, 5, 256, "T must be"),
    (1 << 29, 1024, 64, 5, 256, "T\\*k"),
])
def test_invalid_shapes_rejected(T, h, E, k, I, msg):
    m = _lib()
    n = ctypes.c_size_t()
    rc = m.lib.q38moe_experts_workspace_bytes(T, h, E, k, I, m.BF16, ctypes.byref(n))
    assert rc == -1
    assert re.search(msg, m.lib.q38moe_last_error().decode())


def test_bad_dtype_and_pointers():
    m = _lib()
    rc = m.lib.q38moe_route(None, None, None, None, None, None, None, None, None, 16, 1024, 64, 5, 7, None)
    assert rc == -1 and "dtype" in m.lib.q38moe_last_error().decode()
    rc = m.lib.q38moe_route(None, None, None, None, None, None, None, None, None, 16, 1024, 64, 5, m.BF16, None)
    assert rc == -1 and "x must not be NULL" in m.lib.q38moe_last_error().decode()
    rc = m.lib.q38moe_route(ctypes.c_void_p(8), ctypes.c_void_p(16), None, None, None, None, None, None, None,
                            16, 1024, 64, 5, m.BF16, None)
    assert rc == -1 and "16-byte aligned" in m.lib.q38moe_last_error().decode()


def test_workspace_too_small():
    m = _lib()
    p = ctypes.c_void_p(1 << 20)
    rc = m.lib.q38moe_experts_forward(p, p, 0, p, p, p, p, 64, 1024, 64, 5, 256, p, 16, m.BF16, None)
    assert rc == -2 and "workspace needs" in m.lib.q38moe_last_error().decode()


def test_empty_problem_is_noop():
    m = _lib()
    assert m.lib.q38moe_route(None, None, None, None, None, None, None, None, None, 0, 1024, 64, 5, m.BF16, None) == 0
    assert m.lib.q38moe_experts_forward(None, None, 0, None, None, None, None, 0, 1024, 64, 5, 256, None, 0,
                                        m.BF16, None) == 0


def test_ops_reject_cpu_tensors():
    """The torch front end fails loudly for non-GPU tensors: there is no CPU fallback."""
    import torch
    from q38.hip import ops
    x = torch.zeros(4, 64, dtype=torch.bfloat16)
    w = torch.zeros(8, 64, dtype=torch.bfloat16)
    with pytest.raises(RuntimeError, match="CUDA/HIP tensor"):
        ops.route(x, w, 2)
