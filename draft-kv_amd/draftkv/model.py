"""The small random-weight transformer of the reference, on the GPU.

Reference: draftkv/model.py:28-156. Same constructor, same weights for a given
seed (drawn from ``np.random.default_rng(seed)`` in the reference's order),
same ``forward(tokens, cache, start_pos)``; the forward runs in ``Decoder``.
"""

from __future__ import annotations

import numpy as np
import torch

from .decoder import Decoder, Layer


def sinusoidal(n: int, d: int) -> np.ndarray:                   # model.py:86-94
    """Sinusoidal position table [n, d] in float64: sin on even, cos on odd channels."""
    p = np.arange(n)[:, None]
    i = np.arange(0, d, 2)[None, :]
    ang = p / np.power(10000.0, i / d)
    out = np.zeros((n, d))
    out[:, 0::2] = np.sin(ang)
    out[:, 1::2] = np.cos(ang)
    return out


class TinyTransformer(Decoder):
    """RMSNorm (eps 1e-6), sinusoidal positions added to the embedding, ReLU
    MLP, untied head; weights used as ``x @ W`` (model.py:100-133)."""

    norm = "rms"
    mlp = "relu"
    layout = 0

    def __init__(self, vocab_size: int = 256, d_model: int = 64, n_heads: int = 4, n_layers: int = 4,
                 d_ff=None, max_pos: int = 4096, attn_sharpness: float = 1.0, attn_gain: float = 1.0,
                 seed: int = 0, *, dtype=torch.float32, device=None) -> None:
        self._setup_device(dtype, device)
        rng = np.random.default_rng(seed)
        self.vocab_size, self.d_model, self.n_heads, self.n_layers = vocab_size, d_model, n_heads, n_layers
        self.n_kv_heads = n_heads
        self.d_head = d_model // n_heads
        self.attn_sharpness, self.attn_gain = attn_sharpness, attn_gain
        self.eps = 1e-6
        d_ff = d_ff or 2 * d_model
        s = 1.0 / np.sqrt(d_model)
        f32 = np.float32
        emb = (rng.standard_normal((vocab_size, d_model)) * s).astype(f32)
        self.emb = self._v(emb)
        self.pos_table = self._v(sinusoidal(max_pos, d_model).astype(f32))
        self.layers = []
        for _ in range(n_layers):
            wq = (rng.standard_normal((d_model, d_model)) * s * attn_sharpness).astype(f32)
            wk = (rng.standard_normal((d_model, d_model)) * s).astype(f32)
            wv = (rng.standard_normal((d_model, d_model)) * s).astype(f32)
            wo = (rng.standard_normal((d_model, d_model)) * s * attn_gain).astype(f32)
            w1 = (rng.standard_normal((d_model, d_ff)) * s).astype(f32)
            w2 = (rng.standard_normal((d_ff, d_model)) * s).astype(f32)
            p = Layer()
            p.n1w, p.n1b = self._v(np.ones(d_model, f32)), None
            p.wqkv, p.bqkv = self._w(np.concatenate([wq, wk, wv], axis=1), 0), None
            p.wo, p.bo = self._w(wo, 0), None
            p.n2w, p.n2b = self._v(np.ones(d_model, f32)), None
            p.w1, p.b1 = self._w(w1, 0), None
            p.w2, p.b2 = self._w(w2, 0), None
            self.layers.append(p)
        self.nfw, self.nfb = self._v(np.ones(d_model, f32)), None
        self.head = self._w((rng.standard_normal((d_model, vocab_size)) * s).astype(f32), 0)
        self.head_layout = self.w_layout
        self._tile_weights()


def demo_model(seed: int = 1, **kw) -> TinyTransformer:            # model.py:143-156
    """The reference's test/benchmark model: vocab 128, d 64, 4 heads, 3 layers,
    attention sharpness and gain 4."""
    params = dict(vocab_size=128, d_model=64, n_heads=4, n_layers=3, attn_sharpness=4.0, attn_gain=4.0, seed=seed)
    params.update(kw)
    return TinyTransformer(**params)
