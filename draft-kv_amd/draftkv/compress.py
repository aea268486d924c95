"""KV compression on the GPU: the quantizer, the full cache and the drafter mirror.

Reference: draftkv/compress.py:21-241. The mirror keeps the reference's
observable behaviour -- quantized rows, sink + recent + heavy-hitter eviction
by accumulated attention mass, ``truncate``, ``sync_from``, ``rebuild_layers``
-- with the rows in device memory (integer codes plus per-group scale/lo,
dequantized in registers by the attention kernel). Storage order inside a
(sequence, layer) segment is not position order; ``read`` sorts by position.
"""

from __future__ import annotations

from typing import Optional, Sequence

import numpy as np
import torch

from . import ops
from ._lib import Drafter, QCfg
from .config import CompressionConfig, LayerPlan
from .paged import PagedKVCache, default_device


def quantize(x, bits: int, group: int = 64, scale_fp16: bool = False):
    """Round-trip ``x`` through a ``bits``-wide grid per group of channels
    (compress.py:21-46), on the GPU. numpy in -> numpy out; tensor in ->
    tensor out."""
    as_np = not torch.is_tensor(x)
    t = torch.as_tensor(np.asarray(x, np.float32)) if as_np else x
    if bits >= 16:
        out = t.to(torch.float32).clone()
        return out.numpy() if as_np else out
    dev = t.device if t.is_cuda else default_device()
    deq = ops.quantize_codes(t.to(dev, torch.float32).contiguous(), bits, group, scale_fp16)[3]
    return deq.cpu().numpy() if as_np else deq


def _cfg_of(c: CompressionConfig, head_dim: int) -> QCfg:
    return ops.qcfg(c.bits, c.group, c.scale_fp16, c.sink, c.recent)


def _budget(c: CompressionConfig, seen: int) -> int:           # compress.py:154-157
    return max(int(round(c.keep_frac * max(seen, 1))), c.sink + c.recent)


class FullKVCache(PagedKVCache):
    """The exact cache (compress.py:49-92) as a growable device-paged cache.

    ``FullKVCache(n_layers)`` learns its head count and width from the first
    append and grows its block pool when it runs out, as the reference's
    list-backed cache never runs out."""

    def __init__(self, n_layers: int, n_heads: Optional[int] = None, d_head: Optional[int] = None, *,
                 dtype=np.float32, batch: int = 1, max_tokens: int = 1 << 20, device=None,
                 block_size: int = 16, chunk_keys: Optional[int] = None) -> None:
        self._lazy = dict(n_layers=n_layers, dtype=dtype, batch=batch, max_tokens=max_tokens, device=device,
                          block_size=block_size, chunk_keys=chunk_keys)
        self.n_layers = n_layers
        self._ready = False
        if n_heads is not None and d_head is not None:
            self._init(n_heads, d_head)

    def _init(self, n_heads: int, d_head: int, n_blocks: int = 64) -> None:
        a = self._lazy
        super().__init__(a["n_layers"], n_heads, d_head, a["block_size"], n_blocks, a["dtype"],
                         batch=a["batch"], max_tokens=a["max_tokens"], device=a["device"],
                         chunk_keys=a["chunk_keys"])
        self._ready = True

    def _grow(self) -> None:
        old = self.n_blocks
        new = old * 2
        per_block = self.store.shape[1]
        store = torch.empty((self.batch * new, per_block), dtype=self.dtype, device=self.device)
        for s in range(self.batch):
            store[s * new: s * new + old].copy_(self.store[s * old: (s + 1) * old])
        self.store = store
        for p in self.pools:
            p._stack = list(range(old, new)) + p._stack   # existing free ids are handed out first
            p.n_blocks = new
        self.n_blocks = new
        self._dirty = (0, self.max_blocks)

    def _make_room(self, s: int, n: int) -> None:
        # growing only adds ids under the free list, so the ids handed out, and
        # the final pool size, are those of growing block by block
        while self.pools[s].n_free < n:
            self._grow()

    def _ensure_capacity(self, s, layer, extra):
        while True:
            need_blocks = -(-(int(self.n_tokens[s, layer]) + extra) // self.block_size) - int(self.table_len[s, layer])
            if need_blocks <= self.pools[s].n_free:
                break
            self._grow()
        super()._ensure_capacity(s, layer, extra)

    def reserve(self, counts):
        if not self._ready:
            raise RuntimeError("FullKVCache: shape unknown before the first append")
        super().reserve(counts)

    def append(self, layer, k, v, pos):
        if not self._ready:
            self._init(int(np.shape(k)[1]), int(np.shape(k)[2]))
        super().append(layer, k, v, pos)

    @property
    def length(self) -> int:
        return int(self.n_tokens[0, 0]) if self._ready else 0


class CompressedKVCache:
    """The drafter's lossy view: quantized rows plus token eviction
    (compress.py:95-241), resident on the GPU.

    ``CompressedKVCache(n_layers, cfg)`` is the reference signature (cfg: one
    ``CompressionConfig``, a ``LayerPlan`` or a per-layer list); the device
    shape (``n_kv_heads``, ``d_head``, ``batch``, ``cap`` rows per segment) is
    learned from the first append unless given.
    """

    def __init__(self, n_layers: int, cfg, *, n_kv_heads: Optional[int] = None, d_head: Optional[int] = None,
                 batch: int = 1, cap: Optional[int] = None, device=None,
                 reserve_cfgs: Sequence[CompressionConfig] = ()) -> None:
        self.n_layers = n_layers
        if isinstance(cfg, LayerPlan):
            self.cfgs = list(cfg.cfgs)
        elif isinstance(cfg, CompressionConfig):
            self.cfgs = [cfg] * n_layers
        else:
            self.cfgs = list(cfg)
        if len(self.cfgs) != n_layers:
            raise ValueError(f"expected {n_layers} per-layer configs, got {len(self.cfgs)}")
        self.cfg = self.cfgs[0]
        self.batch = batch
        self.device = torch.device(device) if device is not None else default_device()
        self.seen = np.zeros(batch, np.int64)          # logical context length (layer-0 appends)
        self._reserve = list(dict.fromkeys(reserve_cfgs))     # distinct arms the pages must fit
        self._cap_hint = cap
        self._ready = False
        if n_kv_heads is not None and d_head is not None:
            self._alloc(n_kv_heads, d_head, cap or 4096)

    # ------------------------------------------------------------ storage
    PAGE = 32

    def _page_stride(self, cfgs) -> int:
        """Bytes per page slot: the widest page among the arms this mirror holds."""
        from ._lib import lib
        return max(int(lib().dkv_page_bytes(c.bits, self.d_head, c.group, int(c.scale_fp16)))
                   for c in dict.fromkeys(list(cfgs) + self._reserve))

    def _alloc(self, H: int, D: int, cap: int) -> None:
        cap = -(-cap // self.PAGE) * self.PAGE
        self.n_kv_heads, self.d_head, self.cap = H, D, cap
        self.page_stride = self._page_stride(self.cfgs)
        b, L, dev = self.batch, self.n_layers, self.device
        # one row of page_stride bytes per page slot; page_slots() maps (layer,
        # sequence, head, page) to its slot (the C ABI's layout)
        self.pages = torch.empty((L * b * H * (cap // self.PAGE), self.page_stride), dtype=torch.uint8, device=dev)
        self.pos = torch.full((b, L, cap), -1, dtype=torch.int32, device=dev)
        self.score = torch.zeros((b, L, cap), dtype=torch.float64, device=dev)
        self.n_rows = torch.zeros((b, L), dtype=torch.int32, device=dev)
        self._ready = True

    def _regrow(self, cap: int, cfgs=None) -> None:
        """Re-layout for a larger row capacity and/or wider pages, keeping rows."""
        cfgs = cfgs if cfgs is not None else self.cfgs
        self._reserve = list(dict.fromkeys(self._reserve + list(cfgs)))
        stride = self._page_stride(cfgs)
        if cap <= self.cap and stride <= self.page_stride:
            return
        old_pages, old_pos, old_score, ocap, ostride = self.pages, self.pos, self.score, self.cap, self.page_stride
        old_slots = self.page_slots(ocap)
        n_rows = self.n_rows
        self._alloc(self.n_kv_heads, self.d_head, max(cap, self.cap))
        self.n_rows = n_rows
        new_slots = self.page_slots(self.cap)[:, :, : ocap // self.PAGE]
        for L in range(self.n_layers):   # a layer at a time: the gather's temporary stays small
            self.pages[new_slots[L].reshape(-1), :ostride] = old_pages[old_slots[L].reshape(-1)]
        self.pos[..., :ocap].copy_(old_pos)
        self.score[..., :ocap].copy_(old_score)

    PAGE_CHUNK = 8   # pages per interleaved chunk (csrc/mirror_layout.h)

    def page_slots(self, cap: int) -> torch.Tensor:
        """Page slot of every (layer, sequence x KV head, page) at row capacity
        ``cap``, shape (n_layers, batch * n_kv_heads, cap / 32): a layer's
        pages are one range in which the segments interleave in chunks of
        PAGE_CHUNK pages, the last cap/32 % PAGE_CHUNK pages of each segment
        after the whole chunks (page_ptr in csrc/mirror_layout.h)."""
        L, nseg, npg, ch = self.n_layers, self.batch * self.n_kv_heads, cap // self.PAGE, self.PAGE_CHUNK
        nf = npg // ch
        rem = npg - nf * ch
        kw = dict(device=self.device, dtype=torch.int64)
        lay = torch.arange(L, **kw).view(L, 1, 1)
        seg = torch.arange(nseg, **kw).view(1, nseg, 1)
        p = torch.arange(npg, **kw).view(1, 1, npg)
        base = lay * npg * nseg
        whole = base + ((p // ch) * nseg + seg) * ch + p % ch
        tail = base + nf * ch * nseg + seg * rem + (p - nf * ch)
        return torch.where(p < nf * ch, whole, tail)

    def desc(self) -> Drafter:
        return Drafter(self.pages.data_ptr(), self.pos.data_ptr(), self.score.data_ptr(), self.n_rows.data_ptr(),
                       self.batch, self.n_layers, self.n_kv_heads, self.d_head, self.cap, self.page_stride)

    def qcfg(self, layer: int) -> QCfg:
        return _cfg_of(self.cfgs[layer], self.d_head)

    def qcfgs(self) -> list:
        return [self.qcfg(L) for L in range(self.n_layers)]

    def _i32(self, a) -> torch.Tensor:
        return ops.to_device(np.asarray(a, np.int32), self.device)

    # ------------------------------------------------------------ batched device ops
    def budgets(self) -> np.ndarray:
        """int32 [n_layers, batch] budgets at the current ``seen``: _budget of
        every (layer, sequence), one vector evaluation per distinct arm (numpy's
        rint rounds half to even, as Python's round does)."""
        seen = np.maximum(self.seen, 1).astype(np.float64)
        out = np.empty((self.n_layers, self.batch), np.int32)
        by_cfg: dict = {}
        for L, c in enumerate(self.cfgs):
            by_cfg.setdefault(c, []).append(L)
        for c, layers in by_cfg.items():
            out[layers] = np.maximum(np.rint(c.keep_frac * seen).astype(np.int64), c.sink + c.recent)
        return out

    def step_budgets(self, start: Sequence[int], count: Sequence[int]) -> np.ndarray:
        """Account a forward that appends ``count[s]`` rows at ``start[s]`` to
        every layer (layer 0 moves ``seen``, compress.py:131-132) and return the
        per-layer budgets, int32 [n_layers, batch] on the host."""
        st, ct = np.asarray(start, np.int64), np.asarray(count, np.int64)
        self.seen = np.where(ct > 0, np.maximum(self.seen, st + ct), self.seen)
        return self.budgets()

    def begin_step(self, start: Sequence[int], count: Sequence[int]) -> torch.Tensor:
        """step_budgets as a device int32 [n_layers, batch] tensor."""
        return self._i32(self.step_budgets(start, count))

    def append_layer(self, layer: int, k: torch.Tensor, v: torch.Tensor, start: torch.Tensor,
                     budget_row: torch.Tensor, count: Optional[torch.Tensor] = None) -> None:
        ops.drafter_append(self.desc(), layer, self.qcfg(layer), k, v, start, budget_row, count)

    def attend(self, layer: int, q: torch.Tensor, want_mass: Optional[bool] = None,
               out: Optional[torch.Tensor] = None) -> torch.Tensor:
        """Attention of one query row per sequence over the live rows (q:
        [batch, q_heads, d_head] float32); adds each row's attention mass to
        its score when the layer can evict (keep_frac < 1)."""
        if want_mass is None:
            want_mass = self.cfgs[layer].keep_frac < 1.0
        return ops.drafter_attention(self.desc(), layer, self.qcfg(layer), q, want_mass, out)

    def rows(self) -> np.ndarray:
        """Live rows per (sequence, layer) (one device read-back)."""
        return self.n_rows.cpu().numpy()

    # ------------------------------------------------------------ reference protocol
    def append(self, layer: int, k, v, pos) -> None:                   # compress.py:122-133
        if self.batch != 1:
            raise ValueError("append() is the batch-1 protocol; use begin_step/append_layer")
        kt = (k if torch.is_tensor(k) else torch.as_tensor(np.asarray(k, np.float32))).to(self.device, torch.float32)
        vt = (v if torch.is_tensor(v) else torch.as_tensor(np.asarray(v, np.float32))).to(self.device, torch.float32)
        pos = np.asarray(pos).reshape(-1)
        T = kt.shape[0]
        if T == 0:
            return
        if not np.array_equal(pos, np.arange(pos[0], pos[0] + T)):
            raise ValueError("rows must be appended at consecutive positions")
        if not self._ready:
            self._alloc(kt.shape[1], kt.shape[2], max(self._cap_hint or 0, 4096, 2 * T))
        n_now = int(self.n_rows[0, layer].item())
        if n_now + T > self.cap:
            self._regrow(max(2 * self.cap, n_now + T))
        if layer == 0:
            self.seen[0] = max(self.seen[0], int(pos[-1]) + 1)
        budget = self._i32([_budget(self.cfgs[layer], int(self.seen[0]))])
        ops.drafter_append(self.desc(), layer, self.qcfg(layer), kt.contiguous()[None], vt.contiguous()[None],
                           self._i32([pos[0]]), budget)

    def read(self, layer: int, seq: int = 0):                          # compress.py:135-142
        """(k, v, pos) of the live rows, dequantized, in position order."""
        if not self._ready:
            z = np.zeros((0, 0, 0), np.float32)
            return z, z.copy(), np.zeros(0, np.int64)
        n = int(self.n_rows[seq, layer].item())
        g = ops.drafter_gather(self.desc(), seq, layer, self.qcfg(layer), n, self.device)
        order = torch.argsort(g["pos"].long())
        k = g["k_deq"][order].cpu().numpy()
        v = g["v_deq"][order].cpu().numpy()
        return k, v, g["pos"][order].cpu().numpy().astype(np.int64)

    def read_codes(self, layer: int, seq: int = 0) -> dict:
        """Codes, scale, lo, dequantized values and positions of the live rows,
        in position order (numpy) -- the parity view."""
        n = int(self.n_rows[seq, layer].item())
        g = ops.drafter_gather(self.desc(), seq, layer, self.qcfg(layer), n, self.device)
        order = torch.argsort(g["pos"].long())
        out = {k: t[order].cpu().numpy() for k, t in g.items()}
        out["score"] = self.score[seq, layer, :n][order].cpu().numpy()
        return out

    def note_attention(self, layer: int, probs) -> None:               # compress.py:144-151
        """Add externally computed probabilities (T, heads, rows in position
        order) to the row scores. The GPU forward fuses this into ``attend``."""
        p = torch.as_tensor(np.asarray(probs, np.float32)) if not torch.is_tensor(probs) else probs
        if p.numel() == 0:
            return
        mass = p.to(torch.float32).sum(dim=(0, 1)).to(self.device)
        n = int(self.n_rows[0, layer].item())
        order = torch.argsort(self.pos[0, layer, :n].long())
        m = min(n, mass.shape[0])
        self.score[0, layer, order[:m]] += mass[:m].double()

    def budget(self, layer: int = 0) -> int:                           # compress.py:154-157
        return _budget(self.cfgs[layer], int(self.seen[0]))

    def truncate(self, n_pos) -> None:                                 # compress.py:181-188
        if not self._ready:
            self.seen = np.minimum(self.seen, np.asarray(n_pos, np.int64))
            return
        cut = np.broadcast_to(np.asarray(n_pos, np.int64), (self.batch,))
        ops.drafter_truncate(self.desc(), self.qcfgs(), self._i32(cut))
        self.seen = np.minimum(self.seen, cut)

    def sync_from(self, full: PagedKVCache, start_pos) -> int:         # compress.py:190-207
        """Overwrite positions >= start_pos with quantized true K/V from the
        full cache; returns the (layer, token) rows rewritten (summed over the
        batch). ``start_pos`` is an int or one per sequence."""
        lens = full.lengths() if hasattr(full, "lengths") else np.array([full.length])
        st = np.broadcast_to(np.asarray(start_pos, np.int64), (self.batch,)).copy()
        if not self._ready:
            self.batch = full.batch
            self._alloc(full.n_heads, full.d_head, max(self._cap_hint or 0, int(lens.max()) + 64))
        if int(lens.max()) > self.cap:
            self._regrow(int(lens.max()) + 64)
        rows = int(np.maximum(lens - st, 0).sum()) * self.n_layers
        if np.all(st == 0):
            # truncate(0) + append of everything with scores 0 == the closed-form rebuild
            self.seen = np.maximum(np.minimum(self.seen, 0), np.where(lens > 0, lens, 0))
            self._rebuild(full, list(range(self.n_layers)), lens)
            return rows
        end = lens
        self.seen = np.minimum(self.seen, st)
        has = end > st
        self.seen = np.where(has, np.maximum(self.seen, end), self.seen)
        bud = self.budgets()
        ops.drafter_sync(self.desc(), full.desc(), self.qcfgs(), self._i32(st), self._i32(end), self._i32(bud))
        return rows

    def _rebuild(self, full, layers, lens) -> None:
        bud = self.budgets()
        ops.drafter_rebuild(self.desc(), full.desc(), layers, self.qcfgs(), self._i32(lens), self._i32(bud))

    def rebuild_layers(self, full: PagedKVCache, layers, cfgs=None) -> int:   # compress.py:209-230
        layers = list(layers)
        if cfgs is not None:
            new = list(self.cfgs)
            for L in layers:
                new[L] = cfgs[L]
            if self._ready:
                self._regrow(self.cap, new)
            self.cfgs = new
        self.cfg = self.cfgs[0]
        lens = full.lengths() if hasattr(full, "lengths") else np.array([full.length])
        if not self._ready:
            self.batch = full.batch
            self._alloc(full.n_heads, full.d_head, max(self._cap_hint or 0, int(lens.max()) + 64))
        if int(lens.max()) > self.cap:
            self._regrow(int(lens.max()) + 64)
        if 0 in layers:
            self.seen = np.where(lens > 0, np.maximum(self.seen, lens), self.seen)
        if layers:
            self._rebuild(full, layers, lens)
        return int(lens.sum()) * len(layers)

    @property
    def length(self) -> int:                                           # compress.py:232-234
        return int(self.n_rows[0, 0].item()) if self._ready else 0

    def nbytes(self, n_heads: int, d_head: int) -> float:             # compress.py:236-241
        rows = self.rows() if self._ready else np.zeros((self.batch, self.n_layers))
        return float(sum(2.0 * rows[:, L].sum() * n_heads * self.cfgs[L].bytes_per_entry(d_head)
                         for L in range(self.n_layers)))

    @property
    def seen_positions(self) -> int:
        return int(self.seen[0])
