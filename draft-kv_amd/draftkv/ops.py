"""Torch-tensor front end of the HIP entry points (device buffers in, device
buffers out). Every function validates shapes/dtypes on the host, hands raw
device pointers to the C ABI on torch's current stream, and raises on a
non-zero status. There is no CPU path."""

from __future__ import annotations

import contextlib
import ctypes as C
from typing import Optional, Sequence

import torch

from . import _lib
from ._lib import DKV_BF16, DKV_F32, DKV_GEMM_DEFER, DKV_GEMM_SWIGLU, DKV_GEMM_WTILED, Drafter, Paged, QCfg, check, lib


_get_device = getattr(torch._C, "_cuda_getDevice", None)
_raw_stream = getattr(torch._C, "_cuda_getCurrentRawStream", None)


def _stream() -> int:
    """The current HIP stream of the current device (the capture stream while
    a graph is recorded). torch's C accessors, when present, skip the Python
    layers of torch.cuda.current_stream(), which cost several microseconds on
    every launch."""
    if _raw_stream is not None and _get_device is not None:
        return _raw_stream(_get_device())
    return torch.cuda.current_stream().cuda_stream


def _ptr(t: Optional[torch.Tensor]) -> Optional[int]:
    return None if t is None else t.data_ptr()


def _need(t: torch.Tensor, name: str, dtype=None, ndim=None) -> None:
    if not t.is_cuda:
        raise ValueError(f"{name} must be a GPU tensor")
    if not t.is_contiguous():
        raise ValueError(f"{name} must be contiguous")
    if dtype is not None and t.dtype != dtype:
        raise ValueError(f"{name} must be {dtype}, got {t.dtype}")
    if ndim is not None and t.dim() != ndim:
        raise ValueError(f"{name} must have {ndim} dims, got {tuple(t.shape)}")


def _dt(t: torch.Tensor) -> int:
    if t.dtype == torch.float32:
        return DKV_F32
    if t.dtype == torch.bfloat16:
        return DKV_BF16
    raise ValueError(f"unsupported dtype {t.dtype} (float32 or bfloat16)")


class Workspace:
    """Grow-only scratch buffer per device (allocates only when a call needs more)."""

    def __init__(self) -> None:
        self._buf: dict = {}

    def get(self, device: torch.device, nbytes: int) -> torch.Tensor:
        key = (device.type, device.index)
        b = self._buf.get(key)
        if b is None or b.numel() < nbytes:
            b = torch.empty(max(nbytes, 1 << 16), dtype=torch.uint8, device=device)
            self._buf[key] = b
        return b


_WS = Workspace()


class Stager:
    """Host-to-device copies through page-locked staging buffers: the copy is
    queued on the current stream and the host returns at once (a copy out of
    pageable memory makes the host wait until the GPU has drained the
    stream). Slots are reused round-robin; a slot is refilled only after its
    last copy has finished."""

    def __init__(self, n_slots: int = 64) -> None:
        self.slots: list = [None] * n_slots     # (pinned uint8 buffer, event of its last copy)
        self.i = 0

    def to_device(self, a, device) -> torch.Tensor:
        import numpy as np
        a = np.ascontiguousarray(a)
        if torch.device(device).type != "cuda":
            return torch.from_numpy(a.copy())
        out = torch.empty(a.shape, dtype=torch.from_numpy(a[:0].reshape(-1)).dtype, device=device)
        if a.nbytes == 0:
            return out
        k = self.i
        self.i = (k + 1) % len(self.slots)
        slot = self.slots[k]
        if slot is not None:
            slot[1].synchronize()
        buf = slot[0] if slot is not None and slot[0].numel() >= a.nbytes else \
            torch.empty(max(a.nbytes, 4096), dtype=torch.uint8, pin_memory=True)
        buf.numpy()[: a.nbytes] = a.reshape(-1).view(np.uint8)
        out.view(-1).view(torch.uint8).copy_(buf[: a.nbytes], non_blocking=True)
        ev = torch.cuda.Event()
        ev.record()
        self.slots[k] = (buf, ev)
        return out


_STAGER = Stager()


def to_device(a, device) -> torch.Tensor:
    """A numpy array (or anything np.asarray takes) as a new device tensor of
    its dtype, copied asynchronously on the current stream."""
    return _STAGER.to_device(a, device)


@contextlib.contextmanager
def private_workspace(ws: Workspace):
    """Route every op's scratch to ``ws`` inside the block (a captured HIP
    graph keeps the buffers it was recorded with, so it owns them)."""
    global _WS
    old, _WS = _WS, ws
    try:
        yield ws
    finally:
        _WS = old


def qcfg(bits: int, group: int = 64, meta_f16: bool = False, sink: int = 4, recent: int = 32) -> QCfg:
    return QCfg(int(bits), int(group), int(bool(meta_f16)), int(sink), int(recent))


# ------------------------------------------------------------------ quantize
def quantize_codes(x: torch.Tensor, bits: int, group: int = 64, meta_f16: bool = False):
    """Group quantization of the last axis (reference compress.py:21-46).
    Returns (codes u8, scale f32, lo f32, deq f32)."""
    _need(x, "x", torch.float32)
    if bits >= 16:
        raise ValueError("bits >= 16 has no codes")
    d = x.shape[-1]
    rows = x.numel() // d if d else 0
    ng = -(-d // group)
    codes = torch.empty(x.shape, dtype=torch.uint8, device=x.device)
    scale = torch.empty(x.shape[:-1] + (ng,), dtype=torch.float32, device=x.device)
    lo = torch.empty_like(scale)
    deq = torch.empty_like(x)
    check(lib().dkv_quantize(x.data_ptr(), rows, d, bits, group, int(bool(meta_f16)), codes.data_ptr(),
                             scale.data_ptr(), lo.data_ptr(), deq.data_ptr(), _stream()), "dkv_quantize")
    return codes, scale, lo, deq


# ------------------------------------------------------------------ paged full cache
def paged_append(desc: Paged, layer: int, k: torch.Tensor, v: torch.Tensor, start: torch.Tensor,
                 count: Optional[torch.Tensor] = None) -> None:
    _need(k, "k", ndim=4)
    _need(v, "v", ndim=4)
    _need(start, "start", torch.int32)
    if k.shape != v.shape or k.dtype != v.dtype:
        raise ValueError("k and v must match")
    b, T, H, D = k.shape
    if b != desc.batch or H != desc.n_kv_heads or D != desc.head_dim:
        raise ValueError(f"k shape {tuple(k.shape)} does not match the cache")
    check(lib().dkv_paged_append(C.byref(desc), layer, k.data_ptr(), v.data_ptr(), _dt(k), T,
                                 start.data_ptr(), _ptr(count), _stream()), "dkv_paged_append")


def paged_attention(desc: Paged, layer: int, q: torch.Tensor, start: torch.Tensor, max_len: int,
                    chunk_keys: int, out: Optional[torch.Tensor] = None,
                    count: Optional[torch.Tensor] = None) -> torch.Tensor:
    """Causal attention of q [batch, T, Hq, D] over the paged cache; count
    (int32 [batch], optional): the rows each sequence appended this forward
    (the cache ends at start + count; padding rows see the whole cache)."""
    _need(q, "q", torch.float32, 4)
    _need(start, "start", torch.int32)
    if count is not None:
        _need(count, "count", torch.int32)
    b, T, Hq, D = q.shape
    if b != desc.batch or D != desc.head_dim:
        raise ValueError(f"q shape {tuple(q.shape)} does not match the cache")
    if out is None:
        out = torch.empty_like(q)
    nbytes = lib().dkv_paged_attention_workspace(C.byref(desc), T, Hq, max_len, chunk_keys)
    ws = _WS.get(q.device, nbytes)
    check(lib().dkv_paged_attention(C.byref(desc), layer, q.data_ptr(), T, Hq, start.data_ptr(), _ptr(count),
                                    max_len, chunk_keys, out.data_ptr(), ws.data_ptr(), ws.numel(), _stream()),
          "dkv_paged_attention")
    return out


# ------------------------------------------------------------------ mirror
def _qarr(cfgs: Sequence[QCfg]):
    arr = (QCfg * len(cfgs))(*cfgs)
    return arr


def drafter_append(desc: Drafter, layer: int, cfg: QCfg, k: torch.Tensor, v: torch.Tensor,
                   start: torch.Tensor, budget: torch.Tensor, count: Optional[torch.Tensor] = None) -> None:
    _need(k, "k", ndim=4)
    _need(v, "v", ndim=4)
    _need(start, "start", torch.int32)
    _need(budget, "budget", torch.int32)
    b, T, H, D = k.shape
    if b != desc.batch or H != desc.n_kv_heads or D != desc.head_dim:
        raise ValueError(f"k shape {tuple(k.shape)} does not match the mirror")
    check(lib().dkv_drafter_append(C.byref(desc), layer, cfg, k.data_ptr(), v.data_ptr(), _dt(k), T,
                                   start.data_ptr(), _ptr(count), budget.data_ptr(), _stream()),
          "dkv_drafter_append")


def drafter_truncate(desc: Drafter, cfgs: Sequence[QCfg], start: torch.Tensor) -> None:
    _need(start, "start", torch.int32)
    check(lib().dkv_drafter_truncate(C.byref(desc), _qarr(cfgs), start.data_ptr(), _stream()),
          "dkv_drafter_truncate")


def drafter_sync(desc: Drafter, full: Paged, cfgs: Sequence[QCfg], start: torch.Tensor, end: torch.Tensor,
                 budget: torch.Tensor) -> None:
    for t, n in ((start, "start"), (end, "end"), (budget, "budget")):
        _need(t, n, torch.int32)
    check(lib().dkv_drafter_sync(C.byref(desc), C.byref(full), _qarr(cfgs), start.data_ptr(), end.data_ptr(),
                                 budget.data_ptr(), _stream()), "dkv_drafter_sync")


def drafter_rebuild(desc: Drafter, full: Paged, layers: Sequence[int], cfgs: Sequence[QCfg],
                    length: torch.Tensor, budget: torch.Tensor) -> None:
    _need(length, "length", torch.int32)
    _need(budget, "budget", torch.int32)
    la = (C.c_int32 * max(1, len(layers)))(*layers)
    check(lib().dkv_drafter_rebuild(C.byref(desc), C.byref(full), la, len(layers), _qarr(cfgs),
                                    length.data_ptr(), budget.data_ptr(), _stream()), "dkv_drafter_rebuild")


def drafter_attention(desc: Drafter, layer: int, cfg: QCfg, q: torch.Tensor, want_mass: bool,
                      out: Optional[torch.Tensor] = None) -> torch.Tensor:
    _need(q, "q", torch.float32, 3)
    b, Hq, D = q.shape
    if b != desc.batch or D != desc.head_dim:
        raise ValueError(f"q shape {tuple(q.shape)} does not match the mirror")
    if out is None:
        out = torch.empty_like(q)
    nbytes = lib().dkv_drafter_attention_workspace(C.byref(desc), Hq, int(want_mass))
    ws = _WS.get(q.device, nbytes)
    check(lib().dkv_drafter_attention(C.byref(desc), layer, cfg, q.data_ptr(), Hq, int(want_mass), out.data_ptr(),
                                      ws.data_ptr(), ws.numel(), _stream()), "dkv_drafter_attention")
    return out


def drafter_kernel_timing(on: bool) -> None:
    """Record HIP events around the split-K kernel of every drafter_attention
    call (a benchmark hook; drafter_kernel_last_ms reads the last pair)."""
    check(lib().dkv_drafter_kernel_timing(int(bool(on))), "dkv_drafter_kernel_timing")


def drafter_kernel_last_ms() -> float:
    return float(lib().dkv_drafter_kernel_last_ms())


def drafter_kernel_total_ms() -> tuple:
    """(milliseconds, pairs): the summed event pairs recorded since the hook
    was switched on (at most 1024 calls)."""
    n = C.c_int32(0)
    ms = float(lib().dkv_drafter_kernel_total_ms(C.byref(n)))
    return ms, int(n.value)


def drafter_gather(desc: Drafter, seq: int, layer: int, cfg: QCfg, rows: int, device) -> dict:
    H, D = desc.n_kv_heads, desc.head_dim
    ng = 0 if cfg.bits >= 16 else -(-D // cfg.group)
    o = {}
    for kv in ("k", "v"):
        o[kv + "_codes"] = torch.empty((rows, H, D), dtype=torch.uint8, device=device)
        o[kv + "_scale"] = torch.empty((rows, H, max(ng, 1)), dtype=torch.float32, device=device)
        o[kv + "_lo"] = torch.empty((rows, H, max(ng, 1)), dtype=torch.float32, device=device)
        o[kv + "_deq"] = torch.empty((rows, H, D), dtype=torch.float32, device=device)
    o["pos"] = torch.empty((rows,), dtype=torch.int32, device=device)
    check(lib().dkv_drafter_gather(C.byref(desc), seq, layer, cfg, rows,
                                   *(o[k].data_ptr() for k in ("k_codes", "k_scale", "k_lo", "k_deq",
                                                               "v_codes", "v_scale", "v_lo", "v_deq", "pos")),
                                   _stream()), "dkv_drafter_gather")
    return o


# ------------------------------------------------------------------ sampling and accept
ROW_STATS_WORDS = 4   # dkv_row_stats_t: 32 bytes, held as 4 float64 words per row


def row_stats(rows: int, device, lead: tuple = ()) -> torch.Tensor:
    """A buffer of dkv_row_stats_t for ``lead + (rows,)`` rows."""
    return torch.empty(lead + (rows, ROW_STATS_WORDS), dtype=torch.float64, device=device)


def sample(logits: torch.Tensor, temperature: float, u: torch.Tensor,
           out: Optional[torch.Tensor] = None, stats_out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """One draw per row; ``stats_out`` (a ``row_stats(b)`` buffer or a view
    of one) receives each row's normaliser, which ``accept`` takes back as
    ``draft_stats`` instead of recomputing it."""
    _need(logits, "logits", torch.float32, 2)
    _need(u, "u", torch.float64)
    b, V = logits.shape
    if out is None:
        out = torch.empty(b, dtype=torch.int32, device=logits.device)
    if stats_out is not None:
        _need(stats_out, "stats_out", torch.float64, 2)
        if stats_out.shape != (b, ROW_STATS_WORDS):
            raise ValueError("stats_out must be a row_stats(batch) buffer")
    ws = _WS.get(logits.device, lib().dkv_sample_workspace(b, V))
    check(lib().dkv_sample(logits.data_ptr(), V, b, V, float(temperature), u.data_ptr(), out.data_ptr(),
                           _ptr(stats_out), ws.data_ptr(), ws.numel(), _stream()), "dkv_sample")
    return out


def accept(target: torch.Tensor, draft: Optional[torch.Tensor], draft_tokens: torch.Tensor,
           temperature: float, u: torch.Tensor, draft_stats: Optional[torch.Tensor] = None):
    """Returns (accepted, next_token, n_uniforms) int32 [batch] device tensors.
    ``target`` [batch, gamma+1, vocab]; ``draft`` [gamma, batch, vocab] (the
    draft steps' logits, step-major); ``draft_stats``: the draft rows'
    normalisers from ``sample(..., stats_out=)``, [gamma, batch] rows of
    ``row_stats`` (step-major)."""
    _need(target, "target", torch.float32, 3)
    _need(draft_tokens, "draft_tokens", torch.int32, 2)
    _need(u, "u", torch.float64, 2)
    b, g1, V = target.shape
    gamma = g1 - 1
    if draft_tokens.shape != (b, gamma) or u.shape != (b, g1):
        raise ValueError("draft_tokens must be [batch, gamma] and u [batch, gamma+1]")
    if temperature > 0.0 and gamma > 0:
        if draft is None:
            raise ValueError("draft logits are needed when temperature > 0")
        _need(draft, "draft", torch.float32, 3)
        if draft.shape != (gamma, b, V):
            raise ValueError("draft must be [gamma, batch, vocab]")
    if draft_stats is not None:
        _need(draft_stats, "draft_stats", torch.float64, 3)
        if draft_stats.shape != (gamma, b, ROW_STATS_WORDS):
            raise ValueError("draft_stats must be [gamma, batch] row_stats")
    res = torch.empty((3, b), dtype=torch.int32, device=target.device)
    ws = _WS.get(target.device, lib().dkv_accept_workspace(b, gamma, V))
    check(lib().dkv_accept(target.data_ptr(), _ptr(draft), draft_tokens.data_ptr(), b, gamma, V,
                           float(temperature), u.data_ptr(), _ptr(draft_stats), res[0].data_ptr(), res[1].data_ptr(),
                           res[2].data_ptr(), ws.data_ptr(), ws.numel(), _stream()), "dkv_accept")
    return res[0], res[1], res[2]


# ------------------------------------------------------------------ model forward ops
def _odt(dtype) -> int:
    return DKV_BF16 if dtype == torch.bfloat16 else DKV_F32


def embed(table: torch.Tensor, tokens: torch.Tensor, pos_table: Optional[torch.Tensor] = None,
          positions: Optional[torch.Tensor] = None) -> torch.Tensor:
    _need(tokens, "tokens", torch.int32)
    rows, d = tokens.numel(), table.shape[1]
    out = torch.empty((rows, d), dtype=torch.float32, device=table.device)
    check(lib().dkv_embed(table.data_ptr(), _dt(table), tokens.data_ptr(), rows, d, _ptr(pos_table),
                          _ptr(positions), out.data_ptr(), _stream()), "dkv_embed")
    return out


def rmsnorm(x: torch.Tensor, w: torch.Tensor, eps: float, out_dtype=torch.float32) -> torch.Tensor:
    _need(x, "x", torch.float32, 2)
    out = torch.empty(x.shape, dtype=out_dtype, device=x.device)
    check(lib().dkv_rmsnorm(x.data_ptr(), w.data_ptr(), _dt(w), x.shape[0], x.shape[1], float(eps), out.data_ptr(),
                            _odt(out_dtype), _stream()), "dkv_rmsnorm")
    return out


def layernorm(x: torch.Tensor, w: torch.Tensor, b: torch.Tensor, eps: float, out_dtype=torch.float32) -> torch.Tensor:
    _need(x, "x", torch.float32, 2)
    out = torch.empty(x.shape, dtype=out_dtype, device=x.device)
    check(lib().dkv_layernorm(x.data_ptr(), w.data_ptr(), b.data_ptr(), _dt(w), x.shape[0], x.shape[1], float(eps),
                              out.data_ptr(), _odt(out_dtype), _stream()), "dkv_layernorm")
    return out


def add_norm(h: torch.Tensor, x: torch.Tensor, bias: Optional[torch.Tensor], w: torch.Tensor,
             b: Optional[torch.Tensor], eps: float, layer_norm: bool, out_dtype=torch.float32) -> torch.Tensor:
    """h += x (+ bias) in place, then return RMSNorm(h) (or LayerNorm when ``layer_norm``)."""
    _need(h, "h", torch.float32, 2)
    rows, d = h.shape
    if isinstance(x, Partials):
        if x.shape != (rows, d):
            raise ValueError("add_norm: shapes differ")
        out = torch.empty((rows, d), dtype=out_dtype, device=h.device)
        bp, bd = _bias(bias)
        check(lib().dkv_add_norm_partials(h.data_ptr(), x.data_ptr(), x.n_part, bp, bd, w.data_ptr(),
                                          _ptr(b) if layer_norm else None, _dt(w), 1 if layer_norm else 0, rows, d,
                                          float(eps), out.data_ptr(), _odt(out_dtype), _stream()),
              "dkv_add_norm_partials")
        return out
    _need(x, "x")
    if x.numel() != h.numel():
        raise ValueError("add_norm: shapes differ")
    out = torch.empty((rows, d), dtype=out_dtype, device=h.device)
    bp, bd = _bias(bias)
    if layer_norm:
        check(lib().dkv_add_layernorm(h.data_ptr(), x.data_ptr(), _dt(x), bp, bd, w.data_ptr(), b.data_ptr(), _dt(w),
                                      rows, d, float(eps), out.data_ptr(), _odt(out_dtype), _stream()),
              "dkv_add_layernorm")
    else:
        check(lib().dkv_add_rmsnorm(h.data_ptr(), x.data_ptr(), _dt(x), bp, bd, w.data_ptr(), _dt(w), rows, d,
                                    float(eps), out.data_ptr(), _odt(out_dtype), _stream()), "dkv_add_rmsnorm")
    return out


def _bias(b: Optional[torch.Tensor]):
    return (None, 0) if b is None else (b.data_ptr(), _dt(b))


def qkv_split(qkv: torch.Tensor, bias: Optional[torch.Tensor], n_q_heads: int, n_kv_heads: int, d: int,
              positions: Optional[torch.Tensor] = None, cos_sin: Optional[torch.Tensor] = None, max_pos: int = 0):
    """Fused projection rows [q | k | v] (+ bias) -> float32 q [rows, Hq, d], k, v [rows, Hkv, d];
    RoPE on q and k when ``cos_sin`` (cos table then sin table, [2, max_pos, d/2]) is given.
    ``qkv`` may be a bf16 GEMM's ``Partials``."""
    part = isinstance(qkv, Partials)
    if not part:
        _need(qkv, "qkv", ndim=2)
    rows = qkv.shape[0]
    if qkv.shape[1] != (n_q_heads + 2 * n_kv_heads) * d:
        raise ValueError(f"qkv width {qkv.shape[1]} != (Hq + 2 Hkv) * d")
    dev = qkv.device
    q = torch.empty((rows, n_q_heads, d), dtype=torch.float32, device=dev)
    k = torch.empty((rows, n_kv_heads, d), dtype=torch.float32, device=dev)
    v = torch.empty((rows, n_kv_heads, d), dtype=torch.float32, device=dev)
    bp, bd = _bias(bias)
    if part:
        check(lib().dkv_qkv_split_partials(qkv.data_ptr(), qkv.n_part, bp, bd, rows, n_q_heads, n_kv_heads, d,
                                           _ptr(positions), _ptr(cos_sin), max_pos, q.data_ptr(), k.data_ptr(),
                                           v.data_ptr(), _stream()), "dkv_qkv_split_partials")
        return q, k, v
    check(lib().dkv_qkv_split(qkv.data_ptr(), _dt(qkv), bp, bd, rows, n_q_heads, n_kv_heads, d, _ptr(positions),
                              _ptr(cos_sin), max_pos, q.data_ptr(), k.data_ptr(), v.data_ptr(), _stream()),
          "dkv_qkv_split")
    return q, k, v


def silu_mul(gate_up: torch.Tensor, out_dtype=torch.float32) -> torch.Tensor:
    _need(gate_up, "gate_up", ndim=2)
    rows, ff2 = gate_up.shape
    out = torch.empty((rows, ff2 // 2), dtype=out_dtype, device=gate_up.device)
    check(lib().dkv_silu_mul(gate_up.data_ptr(), _dt(gate_up), rows, ff2 // 2, out.data_ptr(), _odt(out_dtype),
                             _stream()), "dkv_silu_mul")
    return out


def bias_gelu(x: torch.Tensor, bias: Optional[torch.Tensor], out_dtype=torch.float32) -> torch.Tensor:
    _need(x, "x", ndim=2)
    rows, n = x.shape
    out = torch.empty((rows, n), dtype=out_dtype, device=x.device)
    bp, bd = _bias(bias)
    check(lib().dkv_bias_gelu(x.data_ptr(), _dt(x), bp, bd, rows, n, out.data_ptr(), _odt(out_dtype), _stream()),
          "dkv_bias_gelu")
    return out


def relu(x: torch.Tensor, out_dtype=torch.float32) -> torch.Tensor:
    _need(x, "x", ndim=2)
    rows, n = x.shape
    out = torch.empty((rows, n), dtype=out_dtype, device=x.device)
    check(lib().dkv_relu(x.data_ptr(), _dt(x), rows, n, out.data_ptr(), _odt(out_dtype), _stream()), "dkv_relu")
    return out


def add_(h: torch.Tensor, x: torch.Tensor, bias: Optional[torch.Tensor] = None) -> torch.Tensor:
    """h += x (+ bias); h float32 [rows, n], x float32 or bfloat16 of the same shape."""
    _need(h, "h", torch.float32, 2)
    _need(x, "x")
    if x.numel() != h.numel():
        raise ValueError("add_: shapes differ")
    rows, n = h.shape
    bp, bd = _bias(bias)
    check(lib().dkv_add(h.data_ptr(), x.data_ptr(), _dt(x), bp, bd, rows, n, _stream()), "dkv_add")
    return h


def gemm_f32(x: torch.Tensor, w: torch.Tensor, w_layout: int, bias: Optional[torch.Tensor] = None,
             out: Optional[torch.Tensor] = None, accumulate: bool = False) -> torch.Tensor:
    """out (+)= x @ w (+ bias), w [K, N] (layout 0) or [N, K] (layout 1); float32, batch-invariant."""
    _need(x, "x", torch.float32, 2)
    _need(w, "w", torch.float32, 2)
    M, K = x.shape
    N = w.shape[1] if w_layout == 0 else w.shape[0]
    if (w.shape[0] if w_layout == 0 else w.shape[1]) != K:
        raise ValueError(f"gemm_f32: x {tuple(x.shape)} and w {tuple(w.shape)} (layout {w_layout}) disagree")
    if out is None:
        if accumulate:
            raise ValueError("gemm_f32: accumulate needs an output")
        out = torch.empty((M, N), dtype=torch.float32, device=x.device)
    elif out.shape != (M, N) or out.dtype != torch.float32 or not out.is_contiguous():
        raise ValueError("gemm_f32: out must be contiguous float32 [M, N]")
    bp, bd = _bias(bias)
    check(lib().dkv_gemm_f32(x.data_ptr(), w.data_ptr(), w_layout, M, N, K, bp, bd, out.data_ptr(), int(accumulate),
                             _stream()), "dkv_gemm_f32")
    return out


class TiledW:
    """A bf16 weight [N, K] (N % 16 == 0, K % 128 == 0) stored for
    dkv_gemm_bf16's DKV_GEMM_WTILED: 16-row x 128-k tiles of 4 KB, a 16-row
    fragment's tiles consecutive along k, each tile in the MFMA A-operand
    order of its four 32-k steps (element (16 fn + c, 128 kb + 32 j + 8 q + e)
    at (fn * K/128 + kb) * 2048 + j * 512 + (16 q + c) * 8 + e). Every load
    of W is then 1 KB contiguous. ``rows()`` gives the [N, K] matrix back."""

    __slots__ = ("t", "shape")
    dtype = torch.bfloat16

    def __init__(self, w: torch.Tensor) -> None:
        if not tile_ok(w):
            raise ValueError(f"TiledW: needs a contiguous bf16 [N, K] with N % 16 == 0 and K % 128 == 0, "
                             f"got {tuple(w.shape)} {w.dtype}")
        N, K = w.shape
        self.shape = (N, K)
        self.t = w.view(N // 16, 16, K // 128, 4, 4, 8).permute(0, 2, 3, 4, 1, 5).contiguous()

    def rows(self) -> torch.Tensor:
        N, K = self.shape
        return self.t.permute(0, 4, 1, 2, 3, 5).reshape(N, K)

    @property
    def device(self):
        return self.t.device

    @property
    def is_cuda(self) -> bool:
        return self.t.is_cuda

    def numel(self) -> int:
        return self.t.numel()

    def element_size(self) -> int:
        return 2

    def data_ptr(self) -> int:
        return self.t.data_ptr()

    def dim(self) -> int:
        return 2


def tile_ok(w) -> bool:
    return (isinstance(w, torch.Tensor) and w.dtype == torch.bfloat16 and w.dim() == 2 and w.is_contiguous()
            and w.shape[0] % 16 == 0 and w.shape[1] % 128 == 0 and w.shape[0] > 0)


def gemm_bf16_ok(x: torch.Tensor, w, bias: Optional[torch.Tensor] = None) -> bool:
    """Whether dkv_gemm_bf16 takes this product (contiguous x [M, K], bf16 or
    float32, and bf16 w [N, K] (a tensor or a ``TiledW``), any N,
    K % 32 == 0, 16-byte aligned; bias None or bf16 contiguous [N], 8-byte
    aligned)."""
    if not isinstance(w, TiledW) and not (isinstance(w, torch.Tensor) and w.dim() == 2 and w.is_contiguous()):
        return False
    ok = (x.dtype in (torch.bfloat16, torch.float32) and w.dtype == torch.bfloat16 and x.dim() == 2
          and x.is_cuda and w.is_cuda and x.is_contiguous()
          and x.shape[1] == w.shape[1] and w.shape[0] > 0 and w.shape[1] % 32 == 0
          and x.data_ptr() % 16 == 0 and w.data_ptr() % 16 == 0)
    if ok and bias is not None:
        ok = (bias.dtype == torch.bfloat16 and bias.is_cuda and bias.dim() == 1 and bias.is_contiguous()
              and bias.shape[0] == w.shape[0] and bias.data_ptr() % 8 == 0)
    return ok


class Partials:
    """A bf16 GEMM's per-chunk float32 partials [S, M, N] left for its
    consumer (``add_norm``, ``qkv_split``), which sums them in chunk order and
    rounds to bf16: the values the GEMM would have stored. The buffer is the
    op workspace, valid until the next op that takes workspace."""

    __slots__ = ("part", "n_part", "shape")

    def __init__(self, part: torch.Tensor, n_part: int, shape: tuple) -> None:
        self.part, self.n_part, self.shape = part, n_part, shape

    @property
    def device(self):
        return self.part.device

    def numel(self) -> int:
        return self.shape[0] * self.shape[1]

    def data_ptr(self) -> int:
        return self.part.data_ptr()


def gemm_bf16(x: torch.Tensor, w, bias: Optional[torch.Tensor] = None,
              out_dtype=torch.bfloat16, swiglu: bool = False, defer: bool = False):
    """x [M, K] @ w[N, K]^T (+ bias), bf16 in (a float32 x is rounded to bf16
    as it is read), float32 accumulation, bf16 (or float32) out; a row's
    result is the same for any M. swiglu: w's rows interleave (gate_i, up_i)
    and the result is silu(gate) * up, bf16 [M, N / 2] (no bias). defer (bf16
    out, no bias or SwiGLU): when the launch plan makes per-chunk partials,
    return them as ``Partials`` for a consumer that sums them (one launch
    fewer); else the tensor as usual."""
    if not gemm_bf16_ok(x, w, bias):
        raise ValueError(f"gemm_bf16: unsupported operands x {tuple(x.shape)} {x.dtype}, w {tuple(w.shape)} {w.dtype}"
                         + ("" if bias is None else f", bias {tuple(bias.shape)} {bias.dtype}"))
    M, K = x.shape
    N = w.shape[0]
    if swiglu and (bias is not None or out_dtype != torch.bfloat16 or N % 16):
        raise ValueError("gemm_bf16: the SwiGLU epilogue writes bf16, takes no bias and needs N % 16 == 0")
    defer = defer and not swiglu and bias is None and out_dtype == torch.bfloat16 and M > 0
    S = lib().dkv_gemm_bf16_partials(M, N, K) if defer else 0
    nbytes = lib().dkv_gemm_bf16_workspace(M, N, K)
    ws = _WS.get(x.device, nbytes) if nbytes else None
    wflag = DKV_GEMM_WTILED if isinstance(w, TiledW) else 0
    if S > 0:
        check(lib().dkv_gemm_bf16(x.data_ptr(), _odt(x.dtype), w.data_ptr(), None, M, N, K, ws.data_ptr(),
                                  _odt(out_dtype), DKV_GEMM_DEFER | wflag, ws.data_ptr(), ws.numel(), _stream()),
              "dkv_gemm_bf16")
        return Partials(ws, S, (M, N))
    out = torch.empty((M, N // 2 if swiglu else N), dtype=out_dtype, device=x.device)
    check(lib().dkv_gemm_bf16(x.data_ptr(), _odt(x.dtype), w.data_ptr(), _ptr(bias), M, N, K, out.data_ptr(),
                              _odt(out_dtype), (DKV_GEMM_SWIGLU if swiglu else 0) | wflag,
                              _ptr(ws), 0 if ws is None else ws.numel(), _stream()), "dkv_gemm_bf16")
    return out
