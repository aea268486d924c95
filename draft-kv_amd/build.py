"""Builds draft-kv_amd/draftkv/_lib/libdraftkv_hip.so from csrc/*.hip for gfx950.

    python draft-kv_amd/build.py [-j N]

Every source is compiled with hipcc for gfx950 only, with packed-fp32 code
generation disabled (-Xclang -target-feature -Xclang -packed-fp32-ops) and
MFMA accumulators kept in VGPRs (-mllvm -amdgpu-mfma-vgpr-form), then
linked into one shared library exporting the C ABI of include/draftkv_hip.h.
"""

from __future__ import annotations

import argparse
import concurrent.futures as cf
import os
import re
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
OUT_DIR = os.path.join(HERE, "draftkv", "_lib")
LIB = os.path.join(OUT_DIR, "libdraftkv_hip.so")
OBJ_DIR = os.path.join(HERE, "_build")
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")

# -amdgpu-mfma-vgpr-form: MFMA accumulators in VGPRs (gfx950 allows it), so
# a VALU rescale of an accumulator needs no AGPR <-> VGPR copies
FLAGS = ["--offload-arch=gfx950", "-O3", "-fPIC", "-std=c++17",
         "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
         "-mllvm", "-amdgpu-mfma-vgpr-form",
         "-Wno-unused-result"]


def sources() -> list[str]:
    return sorted(os.path.join(CSRC, f) for f in os.listdir(CSRC) if f.endswith(".hip"))


def compile_one(src: str) -> str:
    obj = os.path.join(OBJ_DIR, os.path.basename(src)[:-4] + ".o")
    cmd = [HIPCC, *FLAGS, "-c", src, "-o", obj]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed on {src}:\n{r.stdout}\n{r.stderr}")
    return obj


SEG_KERNEL = "_ZN3dkv21draft_attn_seg_kernel"
_REG = re.compile(r"\bv\[(\d+):(\d+)\]|\bv(\d+)\b")


def _operands(ins: str) -> list[str]:
    """The operand fields of one instruction line (mnemonic dropped, comment
    and trailing modifiers such as ``row_mask:0xf`` kept in the last field)."""
    parts = ins.split(None, 1)
    return [] if len(parts) < 2 else [o.strip() for o in parts[1].split(",")]


def scan_segment_asm(lines: list[str], first: int) -> None:
    """Check the assembly of the segment kernel(s) in ``lines``: no register
    at or above v``first`` anywhere, except as the literal indexed operand of
    an ``s_set_gpr_idx_on`` session inside inline asm (the destination under
    gpr_idx(DST), the first source under gpr_idx(SRC0)) -- the compiler also
    allocates the other operands of the asm blocks, so those are checked
    too. Each kernel must use no scratch and hold 256 VGPRs per wave.
    Raises RuntimeError on the first violation."""
    starts = [i for i, l in enumerate(lines) if re.match(SEG_KERNEL + r"\S*:", l)]
    if not starts:
        raise RuntimeError("segment kernel not found in the device code")
    for st in starts:
        name = lines[st].split(":")[0]
        in_asm, mode = False, None
        for i in range(st + 1, len(lines)):
            t = lines[i].strip()
            if t.startswith(".Lfunc_end"):
                break
            if t.startswith(";;#ASMSTART"):
                in_asm, mode = True, None
                continue
            if t.startswith(";;#ASMEND"):
                if mode is not None:
                    raise RuntimeError(f"{name}: an asm block ends inside an s_set_gpr_idx session "
                                       f"(line {i + 1})")
                in_asm = False
                continue
            if not t or t.startswith((";", ".")):
                continue
            ins = t.split(";")[0].strip()
            op = ins.split(None, 1)[0]
            if op == "s_set_gpr_idx_on":
                if not in_asm:
                    raise RuntimeError(f"{name}: s_set_gpr_idx_on outside inline asm (line {i + 1})")
                m = re.search(r"gpr_idx\((\w+)\)", ins)
                mode = m.group(1) if m else "?"
                if mode not in ("DST", "SRC0"):
                    raise RuntimeError(f"{name}: unexpected gpr_idx mode (line {i + 1}: {t})")
                continue
            if op == "s_set_gpr_idx_off":
                mode = None
                continue
            for k, fld in enumerate(_operands(ins)):
                for g in _REG.finditer(fld):
                    hi = int(g.group(3) if g.group(3) else g.group(2))
                    if hi < first:
                        continue
                    indexed = (in_asm and g.group(3) is not None and fld == f"v{hi}" and op.startswith("v_")
                               and ((mode == "DST" and k == 0) or (mode == "SRC0" and k == 1)))
                    if not indexed:
                        raise RuntimeError(f"{name}: register at or above v{first} outside an indexed operand "
                                           f"(line {i + 1}: {t}); the kept probabilities live there")
        desc = "\n".join(lines[next(i for i, l in enumerate(lines) if l.strip() == f".amdhsa_kernel {name}"):][:60])
        if ".amdhsa_private_segment_fixed_size 0" not in desc or ".amdhsa_next_free_vgpr 256" not in desc:
            raise RuntimeError(f"{name}: expected no scratch and 256 VGPRs per wave")


def check_segment_registers() -> None:
    """The segment kernel (csrc/draft_attn.hip) keeps its probabilities in
    the VGPRs from SEG_VGPRS up, above what it lets the compiler allocate
    (amdgpu_num_vgpr(SEG_VGPRS)). The compiler treats that attribute as a
    target, not a bound -- one build took v176-v177 for code unpacking and
    overwrote a wave's first page -- so the built code is checked by
    ``scan_segment_asm``. Raises RuntimeError on a violation."""
    src = os.path.join(CSRC, "draft_attn.hip")
    m = re.search(r"constexpr int SEG_VGPRS = (\d+);", open(src).read())
    if not m:
        raise RuntimeError("SEG_VGPRS not found in draft_attn.hip")
    first = int(m.group(1))
    asm = os.path.join(OBJ_DIR, "draft_attn.device.s")
    cmd = [HIPCC, *FLAGS, "--cuda-device-only", "-S", src, "-o", asm]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc -S failed on {src}:\n{r.stdout}\n{r.stderr}")
    scan_segment_asm(open(asm).read().split("\n"), first)


def build(jobs: int = 8) -> str:
    os.makedirs(OUT_DIR, exist_ok=True)
    os.makedirs(OBJ_DIR, exist_ok=True)
    srcs = sources()
    with cf.ThreadPoolExecutor(max_workers=max(1, min(jobs, len(srcs) + 1))) as ex:
        seg = ex.submit(check_segment_registers)
        objs = list(ex.map(compile_one, srcs))
        seg.result()
    tmp = LIB + ".tmp"
    cmd = [HIPCC, "--offload-arch=gfx950", "-shared", "-fPIC", *objs, "-o", tmp]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{r.stdout}\n{r.stderr}")
    os.replace(tmp, LIB)
    return LIB


if __name__ == "__main__":
    ap = argparse.ArgumentParser()
    ap.add_argument("-j", type=int, default=8)
    a = ap.parse_args()
    print(build(a.j))
    sys.exit(0)
