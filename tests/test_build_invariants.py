"""Build invariants of the HIP library that no GPU run would catch before
they bite: the segment kernel's register budget (its kept probabilities sit
in VGPRs above the compiler's allocation, which the attribute it uses does
not enforce)."""

import os
import shutil
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, os.path.join(ROOT, "draft-kv_amd"))


@pytest.mark.skipif(not os.path.exists(os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")), reason="needs hipcc")
def test_segment_kernel_keeps_its_registers():
    """Outside inline asm the compiled segment kernel names no VGPR at or
    above SEG_VGPRS, uses no scratch and holds 256 VGPRs per wave."""
    import build
    build.check_segment_registers()


def _kernel_text(asm_body: str, after: str = "") -> list:
    k = "_ZN3dkv21draft_attn_seg_kernel" + "ILi1ELi5EEEv"
    return ("{k}: ; @{k}\n"
            "\tv_mov_b32_e32 v3, 0\n"
            "\t;;#ASMSTART\n{asm}\t;;#ASMEND\n"
            "{after}"
            ".Lfunc_end0:\n"
            "\t.amdhsa_kernel {k}\n\t\t.amdhsa_private_segment_fixed_size 0\n\t\t.amdhsa_next_free_vgpr 256\n"
            ).format(k=k, asm=asm_body, after=after).split("\n")


PUT = "\ts_set_gpr_idx_on s1, gpr_idx(DST)\n\tv_mov_b32 v176, v3\n\tv_mov_b32 v177, v4\n\ts_set_gpr_idx_off\n"
GET = "\ts_set_gpr_idx_on s1, gpr_idx(SRC0)\n\tv_mov_b32 v2, v176\n\tv_mul_f32 v5, v191, v6\n\ts_set_gpr_idx_off\n"


def test_register_check_accepts_indexed_operands():
    import build
    build.scan_segment_asm(_kernel_text(PUT + GET), 176)


@pytest.mark.parametrize("asm,after", [
    # compiler code outside asm
    (PUT, "\tv_and_b32_e32 v176, 15, v3\n"),
    (PUT, "\tv_mfma_f32_16x16x32_f16 v[10:13], v[174:177], v[1:4], v[10:13]\n"),
    # a compiler-allocated operand of an asm block (not the indexed one)
    ("\tv_cndmask_b32 v180, v1, v2, s[4:5]\n", ""),
    ("\ts_nop 1\n\tv_add_f32_dpp v181, v181, v181 quad_perm:[1,0,3,2] row_mask:0xf bank_mask:0xf\n", ""),
    # the other operand of an indexed move
    ("\ts_set_gpr_idx_on s1, gpr_idx(DST)\n\tv_mov_b32 v176, v200\n\ts_set_gpr_idx_off\n", ""),
    ("\ts_set_gpr_idx_on s1, gpr_idx(SRC0)\n\tv_mov_b32 v190, v176\n\ts_set_gpr_idx_off\n", ""),
    ("\ts_set_gpr_idx_on s1, gpr_idx(SRC0)\n\tv_mul_f32 v2, v176, v179\n\ts_set_gpr_idx_off\n", ""),
    # a high register in an asm block with no indexing session
    ("\tv_mov_b32 v176, v3\n", ""),
])
def test_register_check_rejects_a_violation(asm, after):
    """A register at or above SEG_VGPRS is an error wherever it is not the
    literal indexed operand of an s_set_gpr_idx session: in the compiler's
    own code, and among the operands the compiler allocates for the asm
    blocks."""
    import build
    with pytest.raises(RuntimeError, match="at or above v176"):
        build.scan_segment_asm(_kernel_text(asm, after), 176)


def test_register_check_reads_the_built_kernel(tmp_path, monkeypatch):
    """check_segment_registers compiles draft_attn.hip to assembly and scans
    it: a clean listing passes, a violation raises."""
    import build
    body = ["\n".join(_kernel_text(PUT + GET))]

    def fake_run(cmd, capture_output, text):
        open(cmd[cmd.index("-o") + 1], "w").write(body[0])

        class R:
            returncode, stdout, stderr = 0, "", ""
        return R()

    monkeypatch.setattr(build, "OBJ_DIR", str(tmp_path))
    monkeypatch.setattr(build.subprocess, "run", fake_run)
    build.check_segment_registers()
    body[0] = "\n".join(_kernel_text(PUT, "\tv_and_b32_e32 v176, 15, v3\n"))
    with pytest.raises(RuntimeError, match="v176"):
        build.check_segment_registers()
