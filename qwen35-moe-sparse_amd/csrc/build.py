"""Build libq38moe.so (gfx950 only) in-tree with hipcc.

Usage: python build.py [--jobs N]. Objects go to csrc/_build/, the library to
q38/hip/libq38moe.so next to the ctypes loader. Every call recompiles.
"""
import argparse
import os
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

CSRC = Path(__file__).resolve().parent
PKG_ROOT = CSRC.parent
REPO = PKG_ROOT.parent
OUT = PKG_ROOT / "q38" / "hip" / "libq38moe.so"
SOURCES = ["q38moe_route.hip", "q38moe_permute.hip", "q38moe_gemm.hip", "q38moe_gemm_small.hip", "q38moe_combine.hip", "q38moe_quant.hip",
           "q38moe_backward.hip", "q38moe_fp32.hip", "q38moe_api.hip"]
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
FLAGS = [
    "-O3", "-std=c++17", "-fPIC", "--offload-arch=gfx950",
    # Packed-fp32 VALU forms are kept out of generated code.
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-I", str(CSRC), "-I", str(REPO / "include"),
    "-Wall", "-Wno-unused-function",
]


def _compile(src):
    obj = CSRC / "_build" / (Path(src).stem + ".o")
    cmd = [HIPCC, *FLAGS, "-c", str(CSRC / src), "-o", str(obj)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    noise = "is not a recognized feature for this target"
    err = "\n".join(l for l in res.stderr.splitlines() if noise not in l)
    return src, res.returncode, err, obj


def build(jobs=None, verbose=False):
    (CSRC / "_build").mkdir(exist_ok=True)
    with ThreadPoolExecutor(max_workers=jobs or min(len(SOURCES), os.cpu_count() or 1)) as ex:
        results = list(ex.map(_compile, SOURCES))
    failed = False
    for src, rc, err, _ in results:
        if err.strip() and (rc != 0 or verbose):
            print(f"--- {src}\n{err}", file=sys.stderr)
        failed |= rc != 0
    if failed:
        raise RuntimeError("hipcc failed; see messages above")
    OUT.parent.mkdir(parents=True, exist_ok=True)
    tmp = OUT.with_suffix(".so.tmp")
    cmd = [HIPCC, "-shared", "-fPIC", "--offload-arch=gfx950", *[str(o) for *_, o in results],
           "-o", str(tmp)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed:\n{res.stderr}")
    os.replace(tmp, OUT)
    return OUT


if __name__ == "__main__":
    ap = argparse.ArgumentParser()
    ap.add_argument("--jobs", type=int, default=None)
    ap.add_argument("--verbose", action="store_true")
    a = ap.parse_args()
    print(build(a.jobs, a.verbose))
