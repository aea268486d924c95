"""Group-wise asymmetric min/max quantization, restated with codes exposed.

Reference: draftkv/compress.py:21-46 (``quantize``). The reference returns only
the dequantized fp32 array; the codes, per-group scale and per-group minimum it
computes on the way are returned here as well, because the HIP library stores
exactly those and parity is checked on them bit for bit.

Operation order (all float32, two roundings in the dequant -- numpy does not
fuse multiply-add):

    flat  = x.reshape(-1, d).astype(float32), zero-padded to a multiple of
            ``group`` (the padding joins the last group, so it takes part in
            that group's min/max)                         compress.py:30-36
    lo    = min over the group, hi = max                  compress.py:38-39
    scale = max((hi - lo) / levels, 1e-8)                 compress.py:40-41
    q     = rint((g - lo) / scale).clip(0, levels)        compress.py:42
    deq   = q * scale + lo                                compress.py:43
    bits >= 16: an fp32 copy, no codes                    compress.py:28-29

Extensions the reference does not have (its ``quantize`` hard-wires group 64
through the default argument at compress.py:124-125 and keeps scale/lo in
fp32):

* ``group`` is a parameter (32 is used for the int4 drafter pages);
* ``meta="f16"`` stores scale and lo as IEEE half (round-to-nearest-even).
  The codes are then computed against the *stored* values, so the stored
  triple (codes, scale16, lo16) is self-consistent:
  ``lo16 = f16(lo)``, ``s16 = f16(scale)`` (raised to the smallest positive
  half, 2**-24, if it rounds to zero), ``q = rint((g - lo16)/s16).clip``,
  ``deq = q * s16 + lo16`` in float32.
"""

from __future__ import annotations

import numpy as np

F16_MIN_SUBNORMAL = np.float32(2.0 ** -24)


def n_groups(d: int, group: int) -> int:
    return -(-d // group)


def quantize_codes(x: np.ndarray, bits: int, group: int = 64, meta: str = "f32"):
    """Quantize the last axis of ``x`` in groups.

    Returns ``(codes, scale, lo, deq)``:
      codes  uint8, shape ``x.shape`` (one code per element, 0..2**bits-1)
      scale  float32, shape ``x.shape[:-1] + (n_groups,)``
      lo     float32, same shape as scale
      deq    float32, shape ``x.shape`` -- identical to the reference's
             ``quantize(x, bits, group)`` when ``meta == "f32"``.
    """
    if bits >= 16:
        raise ValueError("bits >= 16 has no codes; use quantize()")
    if meta not in ("f32", "f16"):
        raise ValueError(f"meta must be 'f32' or 'f16', got {meta!r}")
    shape = x.shape
    d = shape[-1]
    pad = (-d) % group
    flat = x.reshape(-1, d).astype(np.float32)
    if pad:
        flat = np.pad(flat, ((0, 0), (0, pad)))
    g = flat.reshape(flat.shape[0], -1, group)
    levels = (1 << bits) - 1

    lo = g.min(axis=-1, keepdims=True)
    hi = g.max(axis=-1, keepdims=True)
    scale = np.maximum((hi - lo) / levels, 1e-8)
    if meta == "f16":
        lo = lo.astype(np.float16).astype(np.float32)
        scale = scale.astype(np.float16).astype(np.float32)
        scale = np.where(scale == 0, F16_MIN_SUBNORMAL, scale).astype(np.float32)
    q = np.rint((g - lo) / scale).clip(0, levels)
    deq = (q * scale + lo).reshape(flat.shape)
    codes = q.astype(np.uint8).reshape(flat.shape)
    if pad:
        deq = deq[:, :d]
        codes = codes[:, :d]
    gshape = shape[:-1] + (g.shape[1],)
    return (
        codes.reshape(shape),
        scale.reshape(gshape).astype(np.float32),
        lo.reshape(gshape).astype(np.float32),
        deq.reshape(shape).astype(np.float32),
    )


def quantize(x: np.ndarray, bits: int, group: int = 64, meta: str = "f32") -> np.ndarray:
    """The reference's round trip (compress.py:21-46), plus the two extensions."""
    if bits >= 16:
        return x.astype(np.float32, copy=True)
    return quantize_codes(x, bits, group, meta)[3]


def dequantize(codes: np.ndarray, scale: np.ndarray, lo: np.ndarray, group: int) -> np.ndarray:
    """``codes * scale + lo`` per group, float32, two roundings (compress.py:43)."""
    d = codes.shape[-1]
    gi = np.arange(d) // group
    s = scale[..., gi]
    z = lo[..., gi]
    return (codes.astype(np.float32) * s + z).astype(np.float32)
