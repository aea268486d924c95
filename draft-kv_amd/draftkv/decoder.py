"""One decoder forward for the three model families, on the GPU.

The reference has three numpy forwards that differ only in their pieces
(draftkv/model.py:100-133, draftkv/gpt2.py:182-213, draftkv/llama.py:175-225):
norm (RMSNorm / LayerNorm), positions (sinusoidal or learned table added to the
embedding / RoPE on q and k), MLP (ReLU / GELU-tanh with biases / SwiGLU),
optional projection biases, and the LM head (own matrix / tied embedding).
``Decoder`` runs any combination on device buffers:

* float32 weights: every product goes through ``dkv_gemm_f32`` (one in-order
  reduction per output), so a row's logits do not depend on how many rows
  share the pass -- the verify pass and one-token decoding agree bit for bit,
  which is what makes greedy self-speculative decoding exactly lossless.
* bfloat16 weights: the projections and the head run as the library's bf16
  MFMA GEMM (``dkv_gemm_bf16``, K chunks fixed by the shape, so a row's result
  does not depend on the batch either); norms, RoPE, activations and residual
  adds stay in the HIP kernels with float32 activations. There is no other
  backend: a product the library GEMM does not take raises.

Attention and the K/V writes go to the cache the forward is handed: the
device-paged full cache (``PagedKVCache`` / ``FullKVCache``) or the drafter
mirror (``CompressedKVCache``). ``forward(tokens, cache, start_pos)`` is the
reference's single-sequence signature (numpy in, numpy (T, V) float32 out);
``forward_batch`` is the batched device form the engine uses.
"""

from __future__ import annotations

from typing import Optional, Sequence

import numpy as np
import torch

from . import ops
from .compress import CompressedKVCache, FullKVCache
from .paged import PagedKVCache, default_device


def _t(x, device, dtype) -> Optional[torch.Tensor]:
    if x is None:
        return None
    if torch.is_tensor(x):
        return x.to(device=device, dtype=dtype).contiguous()
    return torch.as_tensor(np.ascontiguousarray(np.asarray(x, np.float32))).to(device=device, dtype=dtype)


class Layer:
    """Device weights of one block. ``w*`` are stored [N, K] (layout 1) or
    [K, N] (layout 0) as given; bf16 models always hold [N, K]."""

    __slots__ = ("n1w", "n1b", "wqkv", "bqkv", "wo", "bo", "n2w", "n2b", "w1", "b1", "w2", "b2")


class Decoder:
    """Shared forward; subclasses fill the spec in their constructors.

    Spec attributes: ``n_layers, d_model, n_heads, n_kv_heads, d_head,
    vocab_size, eps, norm ('rms'|'layer'), mlp ('relu'|'gelu'|'swiglu'),
    layout`` (0: weights [K, N] as ``x @ W``; 1: [N, K] as ``x @ W.T``),
    ``emb, pos_table, rope_theta, head, head_layout, layers, nfw, nfb``.
    """

    norm = "rms"
    mlp = "swiglu"
    rope_theta: Optional[float] = None

    # ------------------------------------------------------------ setup
    def _setup_device(self, dtype, device) -> None:
        self.device = torch.device(device) if device is not None else default_device()
        self.wdtype = dtype
        if dtype not in (torch.float32, torch.bfloat16):
            raise ValueError("dtype must be torch.float32 or torch.bfloat16")
        self.act_dtype = dtype           # dtype of GEMM inputs
        self.kv_dtype = dtype            # dtype of the full cache
        self._cs: Optional[torch.Tensor] = None
        self._cs_len = 0

    def _w(self, x, layout: int) -> torch.Tensor:
        """Upload a weight matrix; bf16 models keep every matrix as [N, K]."""
        t = _t(x, self.device, self.wdtype)
        if self.wdtype == torch.bfloat16 and layout == 0:
            t = t.t().contiguous()
        return t

    def _v(self, x) -> Optional[torch.Tensor]:
        return _t(x, self.device, self.wdtype)

    @property
    def w_layout(self) -> int:
        return 1 if self.wdtype == torch.bfloat16 else self.layout

    def new_cache(self, batch: int = 1, max_tokens: int = 1 << 20, chunk_keys: Optional[int] = None) -> FullKVCache:
        """The full cache for ``batch`` sequences of up to ``max_tokens`` rows;
        ``chunk_keys`` fixes the attention kernel's key chunk (by default
        chosen from the shape, ``paged.auto_chunk_keys``)."""
        return FullKVCache(self.n_layers, self.n_kv_heads, self.d_head, dtype=self.kv_dtype, batch=batch,
                           max_tokens=max_tokens, device=self.device, chunk_keys=chunk_keys)

    # ------------------------------------------------------------ RoPE table
    def _cos_sin(self, need: int):
        """cos table then sin table, float32 [2, n, d/2], computed in float64 as
        llama.py:164-172 does (the two halves of the reference's table are equal)."""
        if self._cs is None or self._cs_len < need:
            n = max(1024, 1 << (need - 1).bit_length())
            D = self.d_head
            inv = 1.0 / (self.rope_theta ** (np.arange(0, D, 2) / D))
            ang = np.outer(np.arange(n), inv)
            cs = np.stack([np.cos(ang), np.sin(ang)]).astype(np.float32)
            self._cs = torch.as_tensor(cs).to(self.device)
            self._cs_len = n
        return self._cs, self._cs_len

    # ------------------------------------------------------------ pieces
    def _norm(self, h: torch.Tensor, w, b) -> torch.Tensor:
        if self.norm == "rms":
            return ops.rmsnorm(h, w, self.eps, self.act_dtype)
        return ops.layernorm(h, w, b, self.eps, self.act_dtype)

    def _proj(self, x: torch.Tensor, w: torch.Tensor, bias=None, defer: bool = False):
        """x @ W (+ bias); float32 out for float32 models, bf16 out for bf16 models
        (with ``defer``, possibly the bf16 GEMM's partials for a consumer that takes them)."""
        if self.wdtype == torch.float32:
            return ops.gemm_f32(x, w, self.layout, bias)
        return self._linear(x, w, bias, defer=defer)

    @staticmethod
    def _linear(x: torch.Tensor, w: torch.Tensor, bias=None, out_dtype=torch.bfloat16, defer: bool = False):
        """bf16 x @ W^T (+ b) (W as [N, K]) by the library's batch-invariant
        GEMM (any N; K a multiple of 32). ``defer``: the caller takes
        ``ops.Partials`` (qkv_split, add_norm), so the GEMM may leave its
        per-chunk partials to it instead of reducing them itself. Raises
        ValueError for a product the GEMM does not take (a second backend
        would break the batch invariance greedy losslessness rests on)."""
        return ops.gemm_bf16(x, w, bias, out_dtype, defer=defer)

    def _residual(self, h: torch.Tensor, x: torch.Tensor, w: torch.Tensor, bias, nw, nb) -> torch.Tensor:
        """h += x @ W (+ bias), then return the next norm of h (weights nw, nb).
        float32: the GEMM accumulates into h; bf16: the add is fused into the norm."""
        if self.wdtype == torch.float32:
            ops.gemm_f32(x, w, self.layout, bias, out=h, accumulate=True)
            return self._norm(h, nw, nb)
        return ops.add_norm(h, self._linear(x, w, defer=True), bias, nw, nb, self.eps, self.norm == "layer",
                            self.act_dtype)

    def _tile_weights(self) -> None:
        """bf16 models: store every projection weight the bf16 GEMM takes in its
        tiled form (``ops.TiledW``: 1 KB contiguous per load of W), and the LM
        head too unless it is the (tied) embedding table. The arithmetic is
        unchanged; ``TiledW.rows()`` gives a matrix back."""
        if self.wdtype != torch.bfloat16:
            return
        for i, p in enumerate(self.layers):   # the bf16 GEMM's k step is 32
            for name in ("wqkv", "wo", "w1", "w2"):
                if getattr(p, name).shape[1] % 32:
                    raise ValueError(f"bf16 weights: layer {i} {name} has input width {getattr(p, name).shape[1]}, "
                                     "not a multiple of 32 (the bf16 GEMM's k step)")
        if self.head.shape[1] % 32:
            raise ValueError(f"bf16 weights: the head's input width {self.head.shape[1]} is not a multiple of 32")
        if self.device.type != "cuda":
            return
        for p in self.layers:
            for name in ("wqkv", "wo", "w1", "w2"):
                w = getattr(p, name)
                if ops.tile_ok(w):
                    setattr(p, name, ops.TiledW(w))
        if self.head is not self.emb and ops.tile_ok(self.head):
            self.head = ops.TiledW(self.head)

    def _interleave_gate_up(self) -> None:
        """bf16 SwiGLU models: reorder each fused [gate; up] weight to rows
        (gate_0, up_0, gate_1, up_1, ...), so the GEMM's epilogue holds both
        halves of a pair and writes silu(gate) * up directly (when the width
        is a multiple of 8, so the fused weight's rows come in whole 16-row
        fragments; else the GEMM writes [gate | up] and the SwiGLU kernel
        combines them)."""
        if self.mlp != "swiglu" or self.wdtype != torch.bfloat16:
            return
        if self.layers and self.layers[0].w1.shape[0] % 16:
            return
        for p in self.layers:
            ff2, k = p.w1.shape
            p.w1 = p.w1.view(2, ff2 // 2, k).transpose(0, 1).reshape(ff2, k).contiguous()
        self.gate_up_interleaved = True

    def _mlp_inner(self, x: torch.Tensor, p: Layer) -> torch.Tensor:
        if self.mlp == "swiglu":
            if getattr(self, "gate_up_interleaved", False):
                return ops.gemm_bf16(x, p.w1, swiglu=True)
            return ops.silu_mul(self._proj(x, p.w1), self.act_dtype)
        if self.mlp == "gelu":
            return ops.bias_gelu(self._proj(x, p.w1), p.b1, self.act_dtype)
        return ops.relu(self._proj(x, p.w1), self.act_dtype)

    def _head(self, x: torch.Tensor) -> torch.Tensor:
        if self.wdtype == torch.float32:
            return ops.gemm_f32(x, self.head, self.head_layout)
        return self._linear(x, self.head, out_dtype=torch.float32)

    # ------------------------------------------------------------ forward
    def forward_batch(self, tokens: torch.Tensor, cache, start: Sequence[int],
                      count: Optional[Sequence[int]] = None) -> torch.Tensor:
        """Run ``tokens`` [batch, T] (int32, on the device) at positions
        start[s] .. start[s]+T-1 and return float32 logits [batch, T, vocab].

        The first ``count[s]`` rows of sequence s (default all T) are appended to
        ``cache``; the other rows are computed and their outputs are undefined
        (the engine uses count 0 for sequences that are done). With the drafter
        mirror T must be 1."""
        b, T = tokens.shape
        st = np.asarray(start, np.int64).reshape(b)
        ct = np.full(b, T, np.int64) if count is None else np.asarray(count, np.int64).reshape(b)
        if np.any(ct < 0) or np.any(ct > T):
            raise ValueError("count must lie in [0, T]")
        st = np.where(ct > 0, st, 0)          # finished sequences attend over a harmless prefix
        pos = (st[:, None] + np.arange(T)[None, :]).astype(np.int32)
        max_pos = int(pos.max()) + 1 if pos.size else 0
        if self.pos_table is not None and max_pos > self.pos_table.shape[0]:
            raise IndexError(f"position {max_pos - 1} beyond the position table ({self.pos_table.shape[0]})")
        dev = self.device
        positions = ops.to_device(pos.reshape(-1), dev)
        tok = tokens.reshape(-1).to(torch.int32).contiguous()
        cs, cs_len = (None, 0)
        if self.rope_theta is not None:
            cs, cs_len = self._cos_sin(max_pos)

        if isinstance(cache, CompressedKVCache):
            attn = self._mirror_attention(cache, b, T, st, ct)
        elif isinstance(cache, PagedKVCache):
            attn = self._paged_attention(cache, b, T, st, ct, max_pos)
        else:
            raise TypeError(f"unsupported cache type {type(cache).__name__}: the GPU forward runs against "
                            "draftkv.paged.PagedKVCache / compress.FullKVCache / compress.CompressedKVCache")

        logits = self._core(tok, positions, b, T, attn, cs, cs_len)
        attn.finish()
        return logits

    def _core(self, tok: torch.Tensor, positions: torch.Tensor, b: int, T: int, attn, cs, cs_len) -> torch.Tensor:
        """The device part of a forward: embed, the decoder layers (attention
        through ``attn(L, q, k, v)``), final norm and head; no host sync and no
        host-dependent shapes, so a HIP graph can record it."""
        R = b * T
        h = ops.embed(self.emb, tok, self.pos_table, positions if self.pos_table is not None else None)
        Hq, Hkv, D = self.n_heads, self.n_kv_heads, self.d_head
        nL = len(self.layers)
        x = self._norm(h, self.layers[0].n1w, self.layers[0].n1b)
        for L, p in enumerate(self.layers):
            q, k, v = ops.qkv_split(self._proj(x, p.wqkv, defer=True), p.bqkv, Hq, Hkv, D, positions, cs, cs_len)
            a = attn(L, q.view(b, T, Hq, D), k.view(b, T, Hkv, D), v.view(b, T, Hkv, D)).view(R, Hq * D)
            # float32 attention output: a bf16 model's o-proj GEMM rounds it to
            # bf16 as it reads it (the same bits as converting it first)
            x = self._residual(h, a, p.wo, p.bo, p.n2w, p.n2b)
            nxt = self.layers[L + 1] if L + 1 < nL else None
            nw, nb = (nxt.n1w, nxt.n1b) if nxt is not None else (self.nfw, self.nfb)
            x = self._residual(h, self._mlp_inner(x, p), p.w2, p.b2, nw, nb)
        return self._head(x).view(b, T, self.vocab_size)

    # ------------------------------------------------------------ caches
    def _paged_attention(self, cache: PagedKVCache, b, T, st, ct, max_pos):
        if isinstance(cache, FullKVCache) and not cache._ready:
            cache._init(self.n_kv_heads, self.d_head)
        if cache.batch != b:
            raise ValueError(f"cache batch {cache.batch} != token batch {b}")
        if cache.n_heads != self.n_kv_heads or cache.d_head != self.d_head:
            raise ValueError("cache heads/width do not match the model")
        if max_pos > cache.max_tokens:
            raise ValueError(f"positions up to {max_pos} exceed the cache's max_tokens={cache.max_tokens}")
        have = cache.n_tokens[:, 0]
        for s in range(b):
            if ct[s] > 0 and st[s] != have[s]:
                raise ValueError(f"sequence {s}: rows must be appended at the cache end "
                                 f"(start {st[s]}, cache holds {have[s]})")
        cache.reserve(ct)
        start_d = ops.to_device(st.astype(np.int32), self.device)
        count_d = None if np.all(ct == T) else ops.to_device(ct.astype(np.int32), self.device)
        attn = self.paged_attn(cache, start_d, count_d, max_pos)
        attn.finish = lambda: cache.commit(ct)
        return attn

    @staticmethod
    def paged_attn(cache: PagedKVCache, start_d, count_d, max_len: int):
        """attn(L, q, k, v) of a forward over the full cache, device tensors
        only: append the rows to layer L at start_d (count_d rows, or all),
        then attend the queries over keys 0 .. start + t. max_len bounds the
        key count of every sequence (it sizes the launch, not the arithmetic)."""
        def attn(L, q, k, v):
            cache.append_layer(L, k, v, start_d, count_d)
            return cache.attend(L, q, start_d, max_len, count=count_d)

        attn.finish = lambda: None
        return attn

    def _mirror_attention(self, cache: CompressedKVCache, b, T, st, ct):
        if T != 1:
            raise ValueError("the drafter mirror takes one row per sequence per forward")
        # a segment never holds more rows than positions
        self.prepare_mirror(cache, b, int((st + ct).max()) if b else 0)
        budgets = cache.begin_step(st, ct)
        start_d = ops.to_device(st.astype(np.int32), self.device)
        count_d = None if np.all(ct == 1) else ops.to_device(ct.astype(np.int32), self.device)
        return self.mirror_attn(cache, b, start_d, budgets, count_d)

    def mirror_attn(self, cache: CompressedKVCache, b: int, start_d, budgets_d, count_d):
        """attn(L, q, k, v) of a draft forward over device tensors: append the
        step's row to layer L of the mirror (evicting to budgets_d[L]), then
        attend its query over the live rows."""
        def attn(L, q, k, v):
            cache.append_layer(L, k, v, start_d, budgets_d[L], count_d)
            return cache.attend(L, q.view(b, self.n_heads, self.d_head))

        attn.finish = lambda: None
        return attn

    def prepare_mirror(self, cache: CompressedKVCache, b: int, need: int) -> None:
        """Allocate the mirror on first use and grow it to hold ``need`` rows
        per segment (the host half of a draft forward's setup)."""
        if not cache._ready:
            cache.batch = b
            cache.seen = np.zeros(b, np.int64)
            cache._alloc(self.n_kv_heads, self.d_head, max(cache._cap_hint or 0, 4096))
        if cache.batch != b:
            raise ValueError(f"mirror batch {cache.batch} != token batch {b}")
        if need > cache.cap:
            cache._regrow(max(2 * cache.cap, need))

    # ------------------------------------------------------------ reference protocol
    def forward(self, tokens, cache, start_pos: int) -> np.ndarray:
        """Reference signature: ``tokens`` (T,) at positions [start_pos,
        start_pos+T) of a batch-1 cache; returns numpy logits (T, vocab) float32."""
        tok = np.asarray(tokens, np.int64).reshape(-1)
        if tok.size and (tok.min() < 0 or tok.max() >= self.vocab_size):
            raise IndexError("token id out of range")
        t = torch.as_tensor(tok.astype(np.int32)).to(self.device)[None]
        if isinstance(cache, PagedKVCache) and getattr(cache, "batch", 1) != 1:
            raise ValueError("forward() is the batch-1 protocol; use forward_batch")
        return self.forward_batch(t, cache, [start_pos]).cpu().numpy()[0]

    def logits_to_probs(self, logits: np.ndarray, temperature: float = 1.0) -> np.ndarray:   # model.py:135-140
        if temperature <= 0:
            out = np.zeros_like(logits)
            out[..., int(np.argmax(logits, -1))] = 1.0
            return out
        x = logits / temperature
        x = x - x.max(-1, keepdims=True)
        e = np.exp(x)
        return e / e.sum(-1, keepdims=True)
