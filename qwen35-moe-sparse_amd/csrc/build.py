"""Build libq38moe.so (gfx950 only) in-tree with hipcc.

Usage: python build.py [--jobs N]. Objects go to csrc/_build/, the library to
q38/hip/libq38moe.so next to the ctypes loader. Every call recompiles.
"""
import argparse
import os
import re
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

CSRC = Path(__file__).resolve().parent
PKG_ROOT = CSRC.parent
REPO = PKG_ROOT.parent
OUT = PKG_ROOT / "q38" / "hip" / "libq38moe.so"
SOURCES = ["q38moe_route.hip", "q38moe_permute.hip", "q38moe_gemm.hip", "q38moe_gemm4w.hip", "q38moe_gemm_small.hip", "q38moe_combine.hip", "q38moe_quant.hip",
           "q38moe_backward.hip", "q38moe_fp32.hip", "q38moe_api.hip"]
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
FLAGS = [
    "-O3", "-std=c++17", "-fPIC", "--offload-arch=gfx950",
    # Packed-fp32 VALU forms are kept out of generated code.
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-I", str(CSRC), "-I", str(REPO / "include"),
    "-Wall", "-Wno-unused-function",
]


# Sources whose kernels issue MFMAs from inline asm: the compiler's hazard recognizer does not see
# them, so their generated code is kept (-save-temps) and checked by mfma_operand_hazards.
ASM_MFMA_SOURCES = ["q38moe_gemm4w.hip"]


def mfma_operand_hazards(asm_text):
    """VALU writes of a VGPR that an MFMA reads as its A or B operand with fewer than two wait states
    in between (gfx950 requires two). Returns the offending (write, mfma) instruction pairs."""
    def regs(tok):
        out = set()
        for m in re.finditer(r"\bv(\d+)\b|\bv\[(\d+):(\d+)\]", tok):
            if m.group(1):
                out.add(int(m.group(1)))
            else:
                out.update(range(int(m.group(2)), int(m.group(3)) + 1))
        return out
    ins = []
    for line in asm_text.splitlines():
        t = line.split(";")[0].strip()
        if t and not t.startswith(".") and not t.endswith(":"):
            ins.append(t)
    bad = []
    for k, t in enumerate(ins):
        op = t.split()[0]
        if not op.startswith("v_") or op.startswith("v_mfma") or len(t.split(None, 1)) < 2:
            continue
        dst = t.split(None, 1)[1].split(",")[0].strip()
        if not dst.startswith("v"):
            continue
        d, waits = regs(dst), 0
        for u in ins[k + 1:k + 4]:
            if u.startswith("s_nop"):
                waits += int(u.split()[1]) + 1
                continue
            if u.startswith("v_mfma") and waits < 2:
                srcs = ",".join(u.split(None, 1)[1].split(",")[1:3])
                if d & regs(srcs):
                    bad.append((t, u))
            waits += 1
    return bad


def barrier_store_coverage(asm_text):
    """Ring stores a barrier may not cover. The four-wave kernels publish each ring slice with
    `s_waitcnt lgkmcnt(n)` + `s_barrier`; LDS operations of a wave complete in order, so the wait
    retires a `ds_write_b128` only if at least n LDS operations follow it before the wait. Returns
    (last store, wait) pairs where fewer follow."""
    bad, seg = [], []
    for line in asm_text.splitlines():
        t = line.split(";")[0].strip()
        if not t or t.startswith("."):
            continue
        if t.endswith(":") or t.startswith("s_endpgm"):
            seg = [] if t.startswith("s_endpgm") else seg
            continue
        if t.startswith("s_barrier"):
            w = [j for j, y in enumerate(seg) if y.startswith("ds_write_b128")]
            waits = [y for y in seg[w[-1] + 1:] if "lgkmcnt(" in y] if w else []
            if waits:
                n = int(re.search(r"lgkmcnt\((\d+)\)", waits[-1]).group(1))
                after = sum(1 for y in seg[w[-1] + 1:] if y.startswith("ds_"))
                if after < n:
                    bad.append((seg[w[-1]], waits[-1]))
            elif w:
                bad.append((seg[w[-1]], "no lgkmcnt wait"))
            seg = []
            continue
        seg.append(t)
    return bad


def _compile(src):
    obj = CSRC / "_build" / (Path(src).stem + ".o")
    cmd = [HIPCC, *FLAGS, "-c", str(CSRC / src), "-o", str(obj)]
    if src in ASM_MFMA_SOURCES:
        cmd.append("-save-temps=obj")
    res = subprocess.run(cmd, capture_output=True, text=True, cwd=str(CSRC / "_build"))
    noise = "is not a recognized feature for this target"
    err = "\n".join(l for l in res.stderr.splitlines() if noise not in l)
    rc = res.returncode
    if rc == 0 and src in ASM_MFMA_SOURCES:
        asm = CSRC / "_build" / (Path(src).stem + "-hip-amdgcn-amd-amdhsa-gfx950.s")
        bad = mfma_operand_hazards(asm.read_text())
        if bad:
            rc = 1
            err += "\n".join(["MFMA operand written by VALU without wait states:"] + [f"  {a}  ->  {b}" for a, b in bad[:8]])
        uncovered = barrier_store_coverage(asm.read_text())
        if uncovered:
            rc = 1
            err += "\n".join(["ring store not covered by the next barrier's wait:"] + [f"  {a}  ->  {b}" for a, b in uncovered[:8]])
    return src, rc, err, obj


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
