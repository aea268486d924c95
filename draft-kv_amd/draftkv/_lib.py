"""ctypes binding of the HIP library (include/draftkv_hip.h).

The product path has no CPU fallback: if ``libdraftkv_hip.so`` is missing or
no GPU is visible, the first call raises. Struct layouts mirror the header
field for field.
"""

from __future__ import annotations

import ctypes as C
import os

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "_lib", "libdraftkv_hip.so")

DKV_F32, DKV_BF16 = 0, 1
DKV_GEMM_SWIGLU, DKV_GEMM_DEFER, DKV_GEMM_WTILED = 1, 2, 4
_ERRORS = {-1: ValueError, -2: RuntimeError, -3: MemoryError, -4: MemoryError}


class Paged(C.Structure):
    _fields_ = [("pool", C.c_void_p), ("block_table", C.c_void_p),
                ("batch", C.c_int32), ("n_layers", C.c_int32), ("n_kv_heads", C.c_int32),
                ("head_dim", C.c_int32), ("block_size", C.c_int32), ("max_blocks", C.c_int32),
                ("dtype", C.c_int32)]


class Drafter(C.Structure):
    _fields_ = [("pages", C.c_void_p), ("pos", C.c_void_p), ("score", C.c_void_p), ("n_rows", C.c_void_p),
                ("batch", C.c_int32), ("n_layers", C.c_int32), ("n_kv_heads", C.c_int32),
                ("head_dim", C.c_int32), ("cap", C.c_int32), ("page_stride", C.c_int64)]


class QCfg(C.Structure):
    _fields_ = [("bits", C.c_int32), ("group", C.c_int32), ("meta_f16", C.c_int32),
                ("sink", C.c_int32), ("recent", C.c_int32)]


P, I32, I64, F32, SZ = C.c_void_p, C.c_int32, C.c_int64, C.c_float, C.c_size_t
PPaged, PDrafter, PQCfg = C.POINTER(Paged), C.POINTER(Drafter), C.POINTER(QCfg)

_SIGS = {
    "dkv_quantize": (C.c_int, [P, I64, I32, I32, I32, I32, P, P, P, P, P]),
    "dkv_paged_append": (C.c_int, [PPaged, I32, P, P, I32, I32, P, P, P]),
    "dkv_paged_attention_workspace": (SZ, [PPaged, I32, I32, I32, I32]),
    "dkv_paged_attention": (C.c_int, [PPaged, I32, P, I32, I32, P, P, I32, I32, P, P, SZ, P]),
    "dkv_page_bytes": (I64, [I32, I32, I32, I32]),
    "dkv_drafter_append": (C.c_int, [PDrafter, I32, QCfg, P, P, I32, I32, P, P, P, P]),
    "dkv_drafter_truncate": (C.c_int, [PDrafter, PQCfg, P, P]),
    "dkv_drafter_sync": (C.c_int, [PDrafter, PPaged, PQCfg, P, P, P, P]),
    "dkv_drafter_rebuild": (C.c_int, [PDrafter, PPaged, C.POINTER(I32), I32, PQCfg, P, P, P]),
    "dkv_drafter_attention_workspace": (SZ, [PDrafter, I32, I32]),
    "dkv_drafter_attention": (C.c_int, [PDrafter, I32, QCfg, P, I32, I32, P, P, SZ, P]),
    "dkv_drafter_kernel_timing": (C.c_int, [I32]),
    "dkv_drafter_kernel_last_ms": (F32, []),
    "dkv_drafter_kernel_total_ms": (F32, [P]),
    "dkv_drafter_gather": (C.c_int, [PDrafter, I32, I32, QCfg, I32, P, P, P, P, P, P, P, P, P, P]),
    "dkv_sample_workspace": (SZ, [I32, I32]),
    "dkv_sample": (C.c_int, [P, I64, I32, I32, F32, P, P, P, P, SZ, P]),
    "dkv_accept_workspace": (SZ, [I32, I32, I32]),
    "dkv_accept": (C.c_int, [P, P, P, I32, I32, I32, F32, P, P, P, P, P, P, SZ, P]),
    "dkv_accept_noalloc": (C.c_int, [P, P, P, I32, I32, I32, F32, P, P, P, P, P, P]),
    "dkv_embed": (C.c_int, [P, I32, P, I32, I32, P, P, P, P]),
    "dkv_rmsnorm": (C.c_int, [P, P, I32, I32, I32, F32, P, I32, P]),
    "dkv_layernorm": (C.c_int, [P, P, P, I32, I32, I32, F32, P, I32, P]),
    "dkv_add_rmsnorm": (C.c_int, [P, P, I32, P, I32, P, I32, I32, I32, F32, P, I32, P]),
    "dkv_add_layernorm": (C.c_int, [P, P, I32, P, I32, P, P, I32, I32, I32, F32, P, I32, P]),
    "dkv_qkv_split": (C.c_int, [P, I32, P, I32, I32, I32, I32, I32, P, P, I32, P, P, P, P]),
    "dkv_add_norm_partials": (C.c_int, [P, P, I32, P, I32, P, P, I32, I32, I32, I32, F32, P, I32, P]),
    "dkv_qkv_split_partials": (C.c_int, [P, I32, P, I32, I32, I32, I32, I32, P, P, I32, P, P, P, P]),
    "dkv_silu_mul": (C.c_int, [P, I32, I32, I32, P, I32, P]),
    "dkv_bias_gelu": (C.c_int, [P, I32, P, I32, I32, I32, P, I32, P]),
    "dkv_relu": (C.c_int, [P, I32, I32, I32, P, I32, P]),
    "dkv_add": (C.c_int, [P, P, I32, P, I32, I32, I32, P]),
    "dkv_gemm_f32": (C.c_int, [P, P, I32, I32, I32, I32, P, I32, P, I32, P]),
    "dkv_gemm_bf16_workspace": (SZ, [I32, I32, I32]),
    "dkv_gemm_bf16_partials": (I32, [I32, I32, I32]),
    "dkv_gemm_bf16": (C.c_int, [P, I32, P, P, I32, I32, I32, P, I32, I32, P, SZ, P]),
    "dkv_last_error": (C.c_char_p, []),
    "dkv_version": (I32, []),
}

_lib = None


def lib():
    """Load the library once; raise loudly if it is not built."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"DRAFTKV HIP library not built: {LIB_PATH} is missing "
                               "(run `python draft-kv_amd/build.py`)")
        h = C.CDLL(LIB_PATH)
        for name, (res, args) in _SIGS.items():
            f = getattr(h, name)
            f.restype = res
            f.argtypes = args
        _lib = h
    return _lib


def exported_symbols() -> list[str]:
    return list(_SIGS)


def check(rc: int, fn: str) -> None:
    if rc != 0:
        msg = lib().dkv_last_error().decode(errors="replace")
        raise _ERRORS.get(rc, RuntimeError)(f"{fn}: {msg}")
