"""The three caches of the decode round, restated on numpy arrays.

* ``FullKVCache``       -- reference draftkv/compress.py:49-92
* ``CompressedKVCache`` -- reference draftkv/compress.py:95-241
* ``BlockPool``, ``PagedKVCache``, ``plan_blocks_needed``
                        -- reference draftkv/paged.py:29-181

The reference keeps per-layer Python lists of rows; here each layer holds
stacked arrays. The observable behaviour (``read`` order, eviction choice,
truncation, block ids handed out, errors raised) is the reference's.
"""

from __future__ import annotations

from typing import Sequence

import numpy as np

from .config import Cfg, budget
from .quant import quantize, quantize_codes


def _empty(h: int = 0, d: int = 0, dtype=np.float32):
    return np.zeros((0, h, d), dtype)


class FullKVCache:
    """compress.py:49-92. Stores rows as given (the Llama forward hands it
    float64 K after RoPE, llama.py:168-171,197-198)."""

    def __init__(self, n_layers: int) -> None:
        self.n_layers = n_layers
        self.k = [None] * n_layers
        self.v = [None] * n_layers
        self.pos = [np.zeros(0, np.int64) for _ in range(n_layers)]

    def append(self, layer, k, v, pos) -> None:                      # :59-63
        pos = np.asarray(pos, np.int64).reshape(-1)
        if self.k[layer] is None:
            self.k[layer], self.v[layer] = k.copy(), v.copy()
        else:
            self.k[layer] = np.concatenate([self.k[layer], k])
            self.v[layer] = np.concatenate([self.v[layer], v])
        self.pos[layer] = np.concatenate([self.pos[layer], pos])

    def read(self, layer):                                            # :65-73
        if self.k[layer] is None or self.pos[layer].size == 0:
            return _empty(), _empty(), np.zeros(0, np.int64)
        return self.k[layer].copy(), self.v[layer].copy(), self.pos[layer].copy()

    def note_attention(self, layer, probs) -> None:                   # :75-76
        pass

    def truncate(self, n_pos: int) -> None:                           # :79-85
        for L in range(self.n_layers):
            if self.k[L] is None:
                continue
            keep = self.pos[L] < n_pos
            self.k[L], self.v[L], self.pos[L] = self.k[L][keep], self.v[L][keep], self.pos[L][keep]

    @property
    def length(self) -> int:                                          # :87-89
        return int(self.pos[0].size)


class CompressedKVCache:
    """compress.py:95-241: quantized rows plus sink/recent/heavy-hitter eviction.

    Besides the dequantized rows the reference keeps, this restatement also
    keeps the integer codes and the per-group (scale, lo) of every row, so the
    HIP drafter pages can be compared with it bit for bit.
    """

    def __init__(self, n_layers: int, cfg) -> None:                   # :103-119
        self.n_layers = n_layers
        if isinstance(cfg, Cfg):
            self.cfgs = [cfg] * n_layers
        else:
            self.cfgs = list(cfg)
        if len(self.cfgs) != n_layers:
            raise ValueError(f"expected {n_layers} per-layer configs, got {len(self.cfgs)}")
        self.k = [None] * n_layers
        self.v = [None] * n_layers
        self.kq = [None] * n_layers     # (codes, scale, lo) for K, or None at 16 bits
        self.vq = [None] * n_layers
        self.pos = [np.zeros(0, np.int64) for _ in range(n_layers)]
        self.score = [np.zeros(0, np.float64) for _ in range(n_layers)]
        self.seen_positions = 0

    # -- model-facing ------------------------------------------------------
    def append(self, layer, k, v, pos) -> None:                       # :122-133
        cfg = self.cfgs[layer]
        pos = np.asarray(pos, np.int64).reshape(-1)
        if cfg.bits >= 16:
            kd, vd = quantize(k, 16), quantize(v, 16)
            kq = vq = None
        else:
            kq = quantize_codes(k, cfg.bits, cfg.group, cfg.meta)
            vq = quantize_codes(v, cfg.bits, cfg.group, cfg.meta)
            kd, vd = kq[3], vq[3]
        self._cat(layer, kd, vd, kq, vq, pos, np.zeros(pos.size, np.float64))
        if layer == 0:
            self.seen_positions = max(self.seen_positions, int(pos[-1]) + 1)
        self._evict(layer)

    def _cat(self, L, kd, vd, kq, vq, pos, score) -> None:
        if self.k[L] is None or self.pos[L].size == 0:
            self.k[L], self.v[L] = kd, vd
            self.kq[L] = None if kq is None else tuple(a for a in kq[:3])
            self.vq[L] = None if vq is None else tuple(a for a in vq[:3])
            self.pos[L], self.score[L] = pos, score
            return
        self.k[L] = np.concatenate([self.k[L], kd])
        self.v[L] = np.concatenate([self.v[L], vd])
        if kq is not None:
            self.kq[L] = tuple(np.concatenate([a, b]) for a, b in zip(self.kq[L], kq[:3]))
            self.vq[L] = tuple(np.concatenate([a, b]) for a, b in zip(self.vq[L], vq[:3]))
        self.pos[L] = np.concatenate([self.pos[L], pos])
        self.score[L] = np.concatenate([self.score[L], score])

    def _select(self, L, keep: np.ndarray) -> None:
        self.k[L], self.v[L] = self.k[L][keep], self.v[L][keep]
        if self.kq[L] is not None:
            self.kq[L] = tuple(a[keep] for a in self.kq[L])
            self.vq[L] = tuple(a[keep] for a in self.vq[L])
        self.pos[L], self.score[L] = self.pos[L][keep], self.score[L][keep]

    def read(self, layer):                                            # :135-142
        if self.k[layer] is None or self.pos[layer].size == 0:
            return _empty(), _empty(), np.zeros(0, np.int64)
        return self.k[layer].copy(), self.v[layer].copy(), self.pos[layer].copy()

    def note_attention(self, layer, probs) -> None:                   # :144-151
        if probs.size == 0:
            return
        mass = probs.sum(axis=(0, 1))                 # float32 sum over (Tq, heads)
        n = min(self.score[layer].size, mass.shape[0])
        self.score[layer][:n] += mass[:n].astype(np.float64)

    # -- control -----------------------------------------------------------
    def budget(self, layer: int = 0) -> int:                          # :154-157
        return budget(self.cfgs[layer], self.seen_positions)

    def victims(self, layer: int) -> np.ndarray:
        """Storage indices ``_evict`` would drop now (compress.py:159-174)."""
        cfg = self.cfgs[layer]
        n = self.pos[layer].size
        B = self.budget(layer)
        if n <= B:
            return np.zeros(0, np.int64)
        order = np.argsort(self.pos[layer])
        protected = np.zeros(n, bool)
        protected[order[: cfg.sink]] = True
        protected[order[-cfg.recent:]] = True        # recent == 0 -> every row (as :167)
        free = np.flatnonzero(~protected)
        n_drop = n - B
        if n_drop <= 0 or free.size == 0:
            return np.zeros(0, np.int64)
        # stable by score; ties keep storage order (== position order)
        ranked = free[np.argsort(self.score[layer][free], kind="stable")]
        return np.sort(ranked[:n_drop])

    def _evict(self, layer: int) -> None:                             # :159-179
        drop = self.victims(layer)
        if drop.size:
            keep = np.ones(self.pos[layer].size, bool)
            keep[drop] = False
            self._select(layer, keep)

    def truncate(self, n_pos: int) -> None:                           # :181-188
        for L in range(self.n_layers):
            if self.k[L] is None:
                continue
            self._select(L, self.pos[L] < n_pos)
        self.seen_positions = min(self.seen_positions, n_pos)

    def sync_from(self, full, start_pos: int) -> int:                 # :190-207
        self.truncate(start_pos)
        rows = 0
        for L in range(self.n_layers):
            k, v, pos = full.read(L)
            sel = np.flatnonzero(pos >= start_pos)
            if sel.size == 0:
                continue
            self.append(L, k[sel], v[sel], pos[sel])
            rows += int(sel.size)
        return rows

    def rebuild_layers(self, full, layers, cfgs=None) -> int:         # :209-230
        rows = 0
        for L in layers:
            if cfgs is not None:
                self.cfgs[L] = cfgs[L]
            self.k[L] = self.v[L] = self.kq[L] = self.vq[L] = None
            self.pos[L] = np.zeros(0, np.int64)
            self.score[L] = np.zeros(0, np.float64)
            k, v, pos = full.read(L)
            if pos.size:
                self.append(L, k, v, pos)
                rows += int(pos.size)
        return rows

    @property
    def length(self) -> int:                                          # :232-234
        return int(self.pos[0].size)

    def nbytes(self, n_heads: int, d_head: int) -> float:             # :236-241
        return sum(2.0 * self.pos[L].size * n_heads * self.cfgs[L].bytes_per_entry(d_head)
                   for L in range(self.n_layers))


# ----------------------------------------------------------------- paging
class BlockPoolExhausted(RuntimeError):
    """paged.py:29-31."""


class BlockPool:
    """paged.py:33-73: LIFO free list over ``range(n_blocks)``; ``pop()`` from
    the end, so the first block handed out is ``n_blocks - 1`` and a freed
    block is the next one handed out."""

    def __init__(self, n_blocks: int, block_size: int) -> None:
        self.n_blocks, self.block_size = n_blocks, block_size
        self.free_list = list(range(n_blocks))
        self.allocated: set[int] = set()

    def allocate(self) -> int:
        if not self.free_list:
            raise BlockPoolExhausted(f"all {self.n_blocks} blocks of size {self.block_size} are in use")
        b = self.free_list.pop()
        self.allocated.add(b)
        return b

    def free(self, block: int) -> None:
        if block not in self.allocated:
            raise RuntimeError(f"double free of block {block}")
        self.allocated.discard(block)
        self.free_list.append(block)

    @property
    def n_free(self) -> int:
        return len(self.free_list)

    @property
    def n_used(self) -> int:
        return len(self.allocated)

    def check_invariants(self) -> None:
        assert len(set(self.free_list)) == len(self.free_list), "duplicate in free list"
        assert not (set(self.free_list) & self.allocated), "block both free and allocated"
        assert len(self.free_list) + len(self.allocated) == self.n_blocks, "blocks leaked"


class PagedKVCache:
    """paged.py:76-176: per-layer block tables over one shared pool; slot =
    block * block_size + offset; truncate frees whole emptied blocks from the
    tail and keeps a partly filled tail block."""

    def __init__(self, n_layers, n_heads, d_head, block_size=16, n_blocks=512, dtype=np.float32):
        self.n_layers, self.n_heads, self.d_head = n_layers, n_heads, d_head
        self.block_size = block_size
        self.pool = BlockPool(n_blocks, block_size)
        shape = (n_blocks * block_size, n_heads, d_head)
        self.k_store = [np.zeros(shape, dtype) for _ in range(n_layers)]
        self.v_store = [np.zeros(shape, dtype) for _ in range(n_layers)]
        self.block_table: list[list[int]] = [[] for _ in range(n_layers)]
        self.n_tokens = [0] * n_layers
        self.pos: list[list[int]] = [[] for _ in range(n_layers)]

    def _slot(self, layer, index):                                    # :108-110
        return self.block_table[layer][index // self.block_size] * self.block_size + index % self.block_size

    def _ensure_capacity(self, layer, extra):                         # :112-117
        while len(self.block_table[layer]) * self.block_size < self.n_tokens[layer] + extra:
            self.block_table[layer].append(self.pool.allocate())

    def append(self, layer, k, v, pos) -> None:                       # :120-128
        n = k.shape[0]
        self._ensure_capacity(layer, n)
        for i in range(n):
            s = self._slot(layer, self.n_tokens[layer])
            self.k_store[layer][s] = k[i]
            self.v_store[layer][s] = v[i]
            self.pos[layer].append(int(pos[i]))
            self.n_tokens[layer] += 1

    def read(self, layer):                                            # :130-138
        n = self.n_tokens[layer]
        if n == 0:
            return (_empty(self.n_heads, self.d_head), _empty(self.n_heads, self.d_head),
                    np.zeros(0, np.int64))
        slots = np.array([self._slot(layer, i) for i in range(n)], np.int64)
        return self.k_store[layer][slots], self.v_store[layer][slots], np.asarray(self.pos[layer], np.int64)

    def note_attention(self, layer, probs) -> None:                   # :140-141
        pass

    def truncate(self, n_pos: int) -> None:                           # :144-162
        for L in range(self.n_layers):
            keep = sum(1 for p in self.pos[L] if p < n_pos)
            if keep == self.n_tokens[L]:
                continue
            assert all(p < n_pos for p in self.pos[L][:keep]), "positions not monotone"
            self.pos[L] = self.pos[L][:keep]
            self.n_tokens[L] = keep
            need = -(-keep // self.block_size)
            while len(self.block_table[L]) > need:
                self.pool.free(self.block_table[L].pop())

    @property
    def length(self) -> int:
        return self.n_tokens[0]

    @property
    def blocks_in_use(self) -> int:
        return self.pool.n_used

    def fragmentation(self) -> float:                                 # :172-176
        cap = self.pool.n_used * self.block_size
        return 0.0 if cap == 0 else 1.0 - sum(self.n_tokens) / cap


def plan_blocks_needed(ctx: int, n_layers: int, block_size: int) -> int:   # :179-181
    return n_layers * (-(-ctx // block_size))
