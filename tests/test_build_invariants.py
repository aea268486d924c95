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


def test_register_check_rejects_a_violation(tmp_path, monkeypatch):
    """The checker reads the kernel's instructions, not its asm blocks: a
    compiler register v176 is an error, the same register inside an asm block
    is not."""
    import build
    body = ("{k}: ; @{k}\n"
            "\tv_mov_b32_e32 v3, 0\n"
            "\t;;#ASMSTART\n\tv_mov_b32 v176, v3\n\t;;#ASMEND\n"
            "{bad}"
            ".Lfunc_end0:\n"
            "\t.amdhsa_kernel {k}\n\t\t.amdhsa_private_segment_fixed_size 0\n\t\t.amdhsa_next_free_vgpr 256\n")
    k = build.SEG_KERNEL + "ILi1ELi5EEEv"

    def fake_run(cmd, capture_output, text, _bad=[""]):
        open(cmd[cmd.index("-o") + 1], "w").write(body.format(k=k, bad=_bad[0]))

        class R:
            returncode, stdout, stderr = 0, "", ""
        return R()

    monkeypatch.setattr(build, "OBJ_DIR", str(tmp_path))
    monkeypatch.setattr(build.subprocess, "run", fake_run)
    build.check_segment_registers()
    fake_run.__defaults__[0][0] = "\tv_and_b32_e32 v176, 15, v3\n"
    with pytest.raises(RuntimeError, match="v176"):
        build.check_segment_registers()
    fake_run.__defaults__[0][0] = "\tv_mfma_f32_16x16x32_f16 v[10:13], v[174:177], v[1:4], v[10:13]\n"
    with pytest.raises(RuntimeError, match="v176"):
        build.check_segment_registers()
