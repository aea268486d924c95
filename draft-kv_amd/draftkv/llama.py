"""Llama / Qwen2-style decoder behind the reference's interface, on the GPU.

Reference: draftkv/llama.py:112-225 (model), :228-245 (checkpoint lookup),
:247-298 (random-weight demo model). RMSNorm, RoPE (rotate-half, float64
tables), GQA (the caches hold KV heads), optional q/k/v biases, SwiGLU MLP,
untied head unless ``lm_head.weight`` is absent. Weights are ``[out, in]`` and
used as ``x @ W.T``.
"""

from __future__ import annotations

import json
import os
from pathlib import Path
from typing import Optional

import numpy as np
import torch

from .bpe import ByteLevelBPE  # noqa: F401  (llama.py:29; re-exported here)
from .decoder import Decoder, Layer
from .gpt2 import load_safetensors

LLAMA3_8B = dict(num_hidden_layers=32, hidden_size=4096, num_attention_heads=32, num_key_value_heads=8,
                 head_dim=128, intermediate_size=14336, vocab_size=128256, rms_norm_eps=1e-5,
                 rope_theta=500000.0)
SMOLLM2_135M = dict(num_hidden_layers=30, hidden_size=576, num_attention_heads=9, num_key_value_heads=3,
                    head_dim=64, intermediate_size=1536, vocab_size=49152, rms_norm_eps=1e-5,
                    rope_theta=10000.0)


def _cat(parts):
    if torch.is_tensor(parts[0]):
        return torch.cat(parts, 0)
    return np.concatenate(parts, 0)


class LlamaLike(Decoder):
    """llama.py:112-225 on the GPU."""

    norm = "rms"
    mlp = "swiglu"
    layout = 1

    def __init__(self, weights: dict, config: dict, *, dtype=torch.float32, device=None) -> None:
        self._setup_device(dtype, device)
        c = config
        self.cfg = c
        self.n_layers = c["num_hidden_layers"]
        self.d_model = c["hidden_size"]
        self.n_heads = c["num_attention_heads"]
        self.n_kv_heads = c.get("num_key_value_heads", self.n_heads)
        self.d_head = c.get("head_dim", self.d_model // self.n_heads)
        self.n_rep = self.n_heads // self.n_kv_heads
        self.vocab_size = c["vocab_size"]
        self.eps = c.get("rms_norm_eps", 1e-5)
        self.theta = float(c.get("rope_theta") or 10000.0)
        self.rope_theta = self.theta
        if self.n_heads % self.n_kv_heads:
            raise ValueError("num_attention_heads must be a multiple of num_key_value_heads")
        w = weights
        self.emb = self._v(w["model.embed_tokens.weight"])
        self.pos_table = None
        self.layers = []
        for i in range(self.n_layers):
            pre = f"model.layers.{i}."
            g = lambda n: w.get(pre + n)
            p = Layer()
            p.n1w, p.n1b = self._v(g("input_layernorm.weight")), None
            p.wqkv = self._w(_cat([g("self_attn.q_proj.weight"), g("self_attn.k_proj.weight"),
                                   g("self_attn.v_proj.weight")]), 1)
            qb = g("self_attn.q_proj.bias")
            p.bqkv = None if qb is None else self._v(_cat([qb, g("self_attn.k_proj.bias"),
                                                           g("self_attn.v_proj.bias")]))
            p.wo, p.bo = self._w(g("self_attn.o_proj.weight"), 1), self._v(g("self_attn.o_proj.bias"))
            p.n2w, p.n2b = self._v(g("post_attention_layernorm.weight")), None
            p.w1, p.b1 = self._w(_cat([g("mlp.gate_proj.weight"), g("mlp.up_proj.weight")]), 1), None
            p.w2, p.b2 = self._w(g("mlp.down_proj.weight"), 1), None
            self.layers.append(p)
        self.nfw, self.nfb = self._v(w["model.norm.weight"]), None
        head = w.get("lm_head.weight")
        self.head = self.emb if head is None else self._w(head, 1)        # tied when absent
        self.head_layout = 1
        self._interleave_gate_up()
        self._tile_weights()

    @classmethod
    def from_dir(cls, d, **kw) -> "LlamaLike":                          # llama.py:152-156
        d = Path(d)
        cfg = json.loads((d / "config.json").read_text())
        return cls(load_safetensors(d / "model.safetensors"), cfg, **kw)

    @classmethod
    def random(cls, config: dict, seed: int = 0, std: float = 0.02, *, dtype=torch.bfloat16,
               device=None) -> "LlamaLike":
        """Random-init model of the given shape with matrices ~ N(0, std) drawn on
        the device (torch generator seeded with ``seed``); norm weights 1."""
        from .paged import default_device
        dev = torch.device(device) if device is not None else default_device()
        gen = torch.Generator(device=dev)
        gen.manual_seed(seed)
        c = config
        d, H, KV = c["hidden_size"], c["num_attention_heads"], c.get("num_key_value_heads", c["num_attention_heads"])
        D = c.get("head_dim", d // H)
        ff, V = c["intermediate_size"], c["vocab_size"]

        def R(*shape):
            t = torch.empty(shape, dtype=dtype, device=dev)
            return t.normal_(0.0, std, generator=gen)

        ones = lambda n: torch.ones(n, dtype=dtype, device=dev)
        w = {"model.embed_tokens.weight": R(V, d), "model.norm.weight": ones(d), "lm_head.weight": R(V, d)}
        for i in range(c["num_hidden_layers"]):
            p = f"model.layers.{i}."
            w[p + "input_layernorm.weight"] = ones(d)
            w[p + "post_attention_layernorm.weight"] = ones(d)
            w[p + "self_attn.q_proj.weight"] = R(H * D, d)
            w[p + "self_attn.k_proj.weight"] = R(KV * D, d)
            w[p + "self_attn.v_proj.weight"] = R(KV * D, d)
            w[p + "self_attn.o_proj.weight"] = R(d, H * D)
            w[p + "mlp.gate_proj.weight"] = R(ff, d)
            w[p + "mlp.up_proj.weight"] = R(ff, d)
            w[p + "mlp.down_proj.weight"] = R(d, ff)
        return cls(w, c, dtype=dtype, device=dev)


def load_llama(d, **kw):                                                   # llama.py:228-234
    """Returns (model, tokenizer) for a local Llama/Qwen2-style checkpoint
    directory; the tokenizer is None when it has no tokenizer.json."""
    d = Path(d)
    if not (d / "model.safetensors").exists():
        raise FileNotFoundError(f"no checkpoint at {d} (no download here)")
    tok = ByteLevelBPE(d / "tokenizer.json") if (d / "tokenizer.json").exists() else None
    return LlamaLike.from_dir(d, **kw), tok


def default_llama_dir(name: str = "smollm2-135m") -> Optional[Path]:       # llama.py:237-244
    env = os.environ.get("DRAFTKV_LLAMA_DIR")
    for c in ([Path(env)] if env else []) + [Path.home() / ".cache" / "draftkv" / name]:
        if (c / "model.safetensors").exists():
            return c
    return None


def demo_llama_weights(n_layers: int = 4, d_model: int = 64, n_heads: int = 8, n_kv_heads: int = 2,
                       vocab_size: int = 128, intermediate: int = 128, attn_bias: bool = False, seed: int = 0,
                       attn_gain: float = 4.0, attn_sharpness: float = 4.0):
    """Weights and config of the random-weight demo model (llama.py:247-298),
    drawn from ``np.random.default_rng(seed)`` in the reference's order,
    including the draw the reference makes and discards for the q bias."""
    rng = np.random.default_rng(seed)
    dh = d_model // n_heads
    s = 1.0 / np.sqrt(d_model)
    f32 = np.float32

    def R(*shape, k=1.0):
        return (rng.standard_normal(shape) * s * k).astype(f32)

    w = {"model.embed_tokens.weight": R(vocab_size, d_model), "model.norm.weight": np.ones(d_model, f32)}
    for i in range(n_layers):
        p = f"model.layers.{i}."
        w[p + "input_layernorm.weight"] = np.ones(d_model, f32)
        w[p + "post_attention_layernorm.weight"] = np.ones(d_model, f32)
        w[p + "self_attn.q_proj.weight"] = R(n_heads * dh, d_model, k=attn_sharpness)
        w[p + "self_attn.k_proj.weight"] = R(n_kv_heads * dh, d_model)
        w[p + "self_attn.v_proj.weight"] = R(n_kv_heads * dh, d_model)
        w[p + "self_attn.o_proj.weight"] = R(d_model, n_heads * dh, k=attn_gain)
        if attn_bias:
            R(n_heads * dh)                        # drawn and discarded, as the reference does
            w[p + "self_attn.k_proj.bias"] = np.zeros(n_kv_heads * dh, f32) + 0.01
            w[p + "self_attn.v_proj.bias"] = np.zeros(n_kv_heads * dh, f32) + 0.01
            w[p + "self_attn.q_proj.bias"] = np.zeros(n_heads * dh, f32) + 0.01
        w[p + "mlp.gate_proj.weight"] = R(intermediate, d_model)
        w[p + "mlp.up_proj.weight"] = R(intermediate, d_model)
        w[p + "mlp.down_proj.weight"] = R(d_model, intermediate)
    cfg = dict(num_hidden_layers=n_layers, hidden_size=d_model, num_attention_heads=n_heads,
               num_key_value_heads=n_kv_heads, vocab_size=vocab_size, rms_norm_eps=1e-5, rope_theta=10000.0)
    return w, cfg


def demo_llama(n_layers: int = 4, d_model: int = 64, n_heads: int = 8, n_kv_heads: int = 2, vocab_size: int = 128,
               intermediate: int = 128, attn_bias: bool = False, seed: int = 0, attn_gain: float = 4.0,
               attn_sharpness: float = 4.0, *, dtype=torch.float32, device=None) -> LlamaLike:
    """Random-weight Llama-style model: RoPE + GQA + RMSNorm + SwiGLU (llama.py:247-298)."""
    w, cfg = demo_llama_weights(n_layers, d_model, n_heads, n_kv_heads, vocab_size, intermediate, attn_bias, seed,
                                attn_gain, attn_sharpness)
    return LlamaLike(w, cfg, dtype=dtype, device=device)
