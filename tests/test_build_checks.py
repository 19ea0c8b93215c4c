"""The build's static checks of the four-wave kernels' generated code (csrc/build.py), on small
hand-written instruction sequences: each check must flag the planted mistake and pass its fix."""
import sys
from pathlib import Path

sys.path.insert(0, str(Path(__file__).resolve().parents[1] / "qwen35-moe-sparse_amd" / "csrc"))
import build  # noqa: E402


def test_mfma_operand_hazard_flags_unwaited_valu_write():
    bad = """
        v_accvgpr_read_b32 v4, a12
        v_mfma_f32_16x16x32_bf16 a[0:3], v[4:7], v[8:11], a[0:3]
    """
    assert len(build.mfma_operand_hazards(bad)) == 1
    ok = """
        v_accvgpr_read_b32 v4, a12
        s_nop 1
        v_mfma_f32_16x16x32_bf16 a[0:3], v[4:7], v[8:11], a[0:3]
    """
    assert build.mfma_operand_hazards(ok) == []
    other = """
        v_accvgpr_read_b32 v40, a12
        v_mfma_f32_16x16x32_bf16 a[0:3], v[4:7], v[8:11], a[0:3]
    """
    assert build.mfma_operand_hazards(other) == []


def _slice(reads_after_last_store, wait=8):
    body = ["ds_write_b128 v1, v[2:5]", "ds_read_b128 v[6:9], v10"] * 4
    body += ["ds_write_b128 v1, v[2:5] offset:4096"]
    body += ["ds_read_b128 v[6:9], v10 offset:2048"] * reads_after_last_store
    return "\n".join(["s_barrier", *body, f"s_waitcnt lgkmcnt({wait})", "s_barrier", "s_endpgm"])


def test_barrier_store_coverage():
    # A barrier whose lgkmcnt(8) leaves the slice's last ring store possibly outstanding.
    assert len(build.barrier_store_coverage(_slice(7))) == 1
    assert build.barrier_store_coverage(_slice(8)) == []
    assert build.barrier_store_coverage(_slice(0, wait=0)) == []
    # A ring store with no wait before the barrier at all.
    assert len(build.barrier_store_coverage("ds_write_b128 v1, v[2:5]\ns_barrier\ns_endpgm")) == 1
    # Stores of the epilogue's own staging area (8-byte) are not ring stores.
    assert build.barrier_store_coverage("ds_write_b64 v1, v[2:3]\ns_barrier\ns_endpgm") == []
