"""Paged full (authoritative) KV cache on the GPU, with host block pools.

Reference: draftkv/paged.py:29-181. Same allocator semantics -- a LIFO free
list over ``range(n_blocks)`` (first block handed out is ``n_blocks - 1``, a
freed block is reused next), per-layer block tables, ``truncate`` frees whole
emptied blocks from the tail and keeps a partly filled tail block,
``BlockPoolExhausted`` instead of corruption, ``RuntimeError`` on a double
free. The block *contents* live in one device pool:

    pool[phys_block] = K [n_kv_heads][block_size][d_head]  ++  V [n_kv_heads][d_head][block_size]

A batched cache gives every sequence its own ``BlockPool`` over its own range
of physical blocks, so each sequence's block ids are exactly those of a
batch-1 reference run. Block tables are mirrored to the device (int32
``[batch][n_layers][max_blocks]``) once per forward, before the kernels read
them.
"""

from __future__ import annotations

import math
from typing import Optional, Sequence

import numpy as np
import torch

from . import ops
from ._lib import DKV_BF16, DKV_F32, Paged


class BlockPoolExhausted(RuntimeError):
    """Raised instead of silently corrupting state when the pool runs dry (paged.py:29-31)."""


class BlockPool:
    """Fixed pool of KV blocks handed out and returned whole (paged.py:33-73)."""

    def __init__(self, n_blocks: int, block_size: int) -> None:
        self.n_blocks = n_blocks
        self.block_size = block_size
        self._stack = list(range(n_blocks))      # pop() from the end: LIFO
        self._live: set[int] = set()

    def allocate(self) -> int:
        if not self._stack:
            raise BlockPoolExhausted(f"all {self.n_blocks} blocks of size {self.block_size} are in use")
        b = self._stack.pop()
        self._live.add(b)
        return b

    def allocate_many(self, n: int) -> list:
        """n allocate() calls at once: the blocks in the order they would be
        handed out. Raises (allocating nothing) when fewer than n are free."""
        if n > len(self._stack):
            raise BlockPoolExhausted(f"{n} blocks wanted, {len(self._stack)} of {self.n_blocks} free")
        if n <= 0:
            return []
        got = self._stack[-n:][::-1]
        del self._stack[-n:]
        self._live.update(got)
        return got

    def free(self, block: int) -> None:
        if block not in self._live:
            raise RuntimeError(f"double free of block {block}")
        self._live.remove(block)
        self._stack.append(block)

    @property
    def n_free(self) -> int:
        return len(self._stack)

    @property
    def n_used(self) -> int:
        return len(self._live)

    def check_invariants(self) -> None:
        assert len(set(self._stack)) == len(self._stack), "duplicate in free list"
        assert not (set(self._stack) & self._live), "block both free and allocated"
        assert len(self._stack) + len(self._live) == self.n_blocks, "blocks leaked"


def _torch_dtype(dtype) -> torch.dtype:
    if dtype in (None, np.float32, torch.float32, "float32", "f32"):
        return torch.float32
    if dtype in (torch.bfloat16, "bfloat16", "bf16"):
        return torch.bfloat16
    raise ValueError(f"unsupported cache dtype {dtype!r} (float32 or bfloat16)")


def auto_chunk_keys(batch: int, n_heads: int, max_tokens: int) -> int:
    """Keys per work unit of the verify/decode attention kernel: about 1024
    units (four per CU) over the cache's capacity, a power of two in
    [2048, 8192]. Measured on one MI355X (bf16, head_dim 128): at batch 32,
    ctx 32k, 8192-key units are 2.5-4% faster than 2048; at batch 1, ctx 262k,
    2048 is best. Verify and decode use the cache's one value, so their rows
    stay bit-identical whatever it is."""
    units = max(1.0, batch * n_heads * max_tokens / 1024.0)
    return int(min(8192, max(2048, 1 << int(round(math.log2(units))))))


def default_device() -> torch.device:
    if not torch.cuda.is_available():
        raise RuntimeError("draftkv needs a ROCm GPU (torch.cuda.is_available() is False)")
    return torch.device("cuda", torch.cuda.current_device())


class PagedKVCache:
    """The full cache, in device blocks, behind the reference cache protocol.

    ``PagedKVCache(n_layers, n_heads, d_head, block_size=16, n_blocks=512,
    dtype=np.float32)`` is the reference signature (n_heads = KV heads);
    ``batch``, ``max_tokens``, ``device`` and ``chunk_keys`` (the fixed key
    chunk of the attention kernel; by default ``auto_chunk_keys``) are
    additions.
    """

    def __init__(self, n_layers: int, n_heads: int, d_head: int, block_size: int = 16,
                 n_blocks: int = 512, dtype=np.float32, *, batch: int = 1,
                 max_tokens: Optional[int] = None, device=None, chunk_keys: Optional[int] = None) -> None:
        self.n_layers, self.n_heads, self.d_head = n_layers, n_heads, d_head
        self.block_size, self.n_blocks, self.batch = block_size, n_blocks, batch
        self.dtype = _torch_dtype(dtype)
        self.device = torch.device(device) if device is not None else default_device()
        self.max_tokens = max_tokens if max_tokens is not None else n_blocks * block_size
        self.chunk_keys = chunk_keys if chunk_keys is not None else auto_chunk_keys(batch, n_heads, self.max_tokens)
        self.max_blocks = -(-self.max_tokens // block_size)
        self.pools = [BlockPool(n_blocks, block_size) for _ in range(batch)]
        per_block = 2 * n_heads * block_size * d_head
        self.store = torch.empty((batch * n_blocks, per_block), dtype=self.dtype, device=self.device)
        self.tables = np.full((batch, n_layers, self.max_blocks), -1, np.int32)   # local ids
        self.table_len = np.zeros((batch, n_layers), np.int64)
        self.n_tokens = np.zeros((batch, n_layers), np.int64)
        self.d_tables = torch.full((batch, n_layers, self.max_blocks), 0, dtype=torch.int32, device=self.device)
        self._dirty: Optional[tuple[int, int]] = None   # [lo, hi) block-index range to upload

    # ------------------------------------------------------------ descriptor
    def desc(self) -> Paged:
        return Paged(self.store.data_ptr(), self.d_tables.data_ptr(), self.batch, self.n_layers, self.n_heads,
                     self.d_head, self.block_size, self.max_blocks,
                     DKV_BF16 if self.dtype == torch.bfloat16 else DKV_F32)

    # ------------------------------------------------------------ allocation
    def _ensure_capacity(self, s: int, layer: int, extra: int) -> None:   # paged.py:112-117
        need = self.n_tokens[s, layer] + extra
        while self.table_len[s, layer] * self.block_size < need:
            idx = int(self.table_len[s, layer])
            if idx >= self.max_blocks:
                raise BlockPoolExhausted(f"sequence {s} exceeds max_tokens={self.max_tokens}")
            self.tables[s, layer, idx] = self.pools[s].allocate()
            self.table_len[s, layer] += 1
            lo, hi = self._dirty or (idx, idx + 1)
            self._dirty = (min(lo, idx), max(hi, idx + 1))

    def _make_room(self, s: int, n: int) -> None:
        """Hook before sequence s takes n blocks (a fixed pool raises when short)."""

    def reserve(self, counts: Sequence[int]) -> None:
        """Allocate blocks for ``counts[s]`` more tokens in every layer, layer by
        layer as the reference's per-layer appends would (each sequence's pool
        hands its blocks to layer 0 first, then layer 1, ...), and push the new
        table entries to the device. Vectorized over (sequence, layer): only the
        pairs that need a block are visited."""
        cnt = np.asarray(counts, np.int64).reshape(self.batch)
        grow = cnt > 0
        if not grow.any():
            return
        bs = self.block_size
        need = self.n_tokens + cnt[:, None]
        want = np.where(grow[:, None], np.maximum(-(-need // bs), self.table_len), self.table_len)
        if int(want.max()) > self.max_blocks:
            s = int(np.flatnonzero((want > self.max_blocks).any(axis=1))[0])
            raise BlockPoolExhausted(f"sequence {s} exceeds max_tokens={self.max_tokens}")
        add = want - self.table_len
        for s in np.flatnonzero(add.any(axis=1)):
            self._make_room(int(s), int(add[s].sum()))
            got = self.pools[s].allocate_many(int(add[s].sum()))
            i = 0
            for L in np.flatnonzero(add[s]):
                k, t0 = int(add[s, L]), int(self.table_len[s, L])
                self.tables[s, L, t0: t0 + k] = got[i: i + k]
                i += k
        if add.any():
            lo = int(self.table_len[add > 0].min())
            hi = int(want.max())
            dl, dh = self._dirty or (lo, hi)
            self._dirty = (min(dl, lo), max(dh, hi))
            self.table_len = want
        self._upload()

    def _upload(self) -> None:
        if self._dirty is None:
            return
        lo, hi = self._dirty
        phys = self.tables[:, :, lo:hi] + (np.arange(self.batch, dtype=np.int32) * self.n_blocks)[:, None, None]
        phys = np.where(self.tables[:, :, lo:hi] >= 0, phys, 0).astype(np.int32)
        self.d_tables[:, :, lo:hi].copy_(ops.to_device(phys, self.device))
        self._dirty = None

    # ------------------------------------------------------------ batched device ops
    def append_layer(self, layer: int, k: torch.Tensor, v: torch.Tensor, start: torch.Tensor,
                     count: Optional[torch.Tensor] = None) -> None:
        """Write ``k, v`` [batch, T, heads, d_head] at positions start[s]..; blocks
        must have been reserved."""
        ops.paged_append(self.desc(), layer, k, v, start, count)

    def attend(self, layer: int, q: torch.Tensor, start: torch.Tensor, max_len: int,
               out: Optional[torch.Tensor] = None, count: Optional[torch.Tensor] = None) -> torch.Tensor:
        """Causal attention of q [batch, T, heads, d_head] at positions start[s]..;
        count: the rows appended this forward when not all T (see append_layer)."""
        return ops.paged_attention(self.desc(), layer, q, start, max_len, self.chunk_keys, out, count)

    def commit(self, counts: Sequence[int]) -> None:
        """Record that ``counts[s]`` rows were appended to every layer."""
        self.n_tokens += np.asarray(counts, np.int64)[:, None]

    # ------------------------------------------------------------ reference protocol (batch 1 view)
    def append(self, layer: int, k, v, pos) -> None:                  # paged.py:120-128
        """Reference-protocol append for sequence 0 (k, v: (T, heads, d_head))."""
        if self.batch != 1:
            raise ValueError("append() is the batch-1 protocol; use reserve/append_layer/commit")
        k = torch.as_tensor(np.asarray(k, np.float32) if not torch.is_tensor(k) else k, device=self.device)
        v = torch.as_tensor(np.asarray(v, np.float32) if not torch.is_tensor(v) else v, device=self.device)
        pos = np.asarray(pos).reshape(-1)
        T = k.shape[0]
        if T == 0:
            return
        start = int(self.n_tokens[0, layer])
        if not np.array_equal(pos, np.arange(start, start + T)):
            raise ValueError("the device cache stores positions contiguously from 0")
        self._ensure_capacity(0, layer, T)
        self._upload()
        st = torch.tensor([start], dtype=torch.int32, device=self.device)
        ops.paged_append(self.desc(), layer, k.float().contiguous()[None], v.float().contiguous()[None], st)
        self.n_tokens[0, layer] += T

    def read(self, layer: int, seq: int = 0):                          # paged.py:130-138
        n = int(self.n_tokens[seq, layer])
        if n == 0:
            z = np.zeros((0, self.n_heads, self.d_head), np.float32)
            return z, z.copy(), np.zeros(0, np.int64)
        H, D, bs = self.n_heads, self.d_head, self.block_size
        nb = -(-n // bs)
        phys = self.tables[seq, layer, :nb].astype(np.int64) + seq * self.n_blocks
        blocks = self.store[torch.from_numpy(phys).to(self.device)].float().cpu().numpy()
        kb = blocks[:, : H * bs * D].reshape(nb, H, bs, D).transpose(0, 2, 1, 3).reshape(nb * bs, H, D)
        vb = blocks[:, H * bs * D:].reshape(nb, H, D, bs).transpose(0, 3, 1, 2).reshape(nb * bs, H, D)
        return kb[:n].copy(), vb[:n].copy(), np.arange(n, dtype=np.int64)

    def note_attention(self, layer: int, probs) -> None:               # paged.py:140-141
        pass

    def truncate(self, n_pos) -> None:                                 # paged.py:144-162
        """Drop positions >= n_pos (an int for every sequence, or one per sequence)."""
        cut = np.broadcast_to(np.asarray(n_pos, np.int64), (self.batch,))
        keep = np.minimum(self.n_tokens, cut[:, None])
        changed = keep != self.n_tokens
        if not changed.any():
            return
        self.n_tokens = np.where(changed, keep, self.n_tokens)
        need = np.where(changed, -(-keep // self.block_size), self.table_len)
        # emptied tail blocks go back per sequence, layer by layer, last first
        for s, L in zip(*np.nonzero(self.table_len > need)):
            for idx in range(int(self.table_len[s, L]) - 1, int(need[s, L]) - 1, -1):
                self.pools[s].free(int(self.tables[s, L, idx]))
                self.tables[s, L, idx] = -1
            self.table_len[s, L] = need[s, L]

    @property
    def block_table(self) -> list:
        """Sequence 0's per-layer block ids (reference attribute)."""
        return [self.tables[0, L, : self.table_len[0, L]].tolist() for L in range(self.n_layers)]

    @property
    def pool(self) -> BlockPool:
        """Sequence 0's block pool (the reference's single pool)."""
        return self.pools[0]

    @property
    def length(self) -> int:
        return int(self.n_tokens[0, 0])

    def lengths(self) -> np.ndarray:
        return self.n_tokens[:, 0].copy()

    @property
    def blocks_in_use(self) -> int:
        return sum(p.n_used for p in self.pools)

    def fragmentation(self) -> float:                                  # paged.py:172-176
        cap = self.blocks_in_use * self.block_size
        return 0.0 if cap == 0 else 1.0 - float(self.n_tokens.sum()) / cap


def plan_blocks_needed(ctx: int, n_layers: int, block_size: int) -> int:   # paged.py:179-181
    """Blocks a context of ``ctx`` tokens occupies across all layers."""
    return n_layers * (-(-ctx // block_size))
