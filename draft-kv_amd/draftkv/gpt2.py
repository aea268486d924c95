"""GPT-2 / distilgpt2 behind the reference's interface, on the GPU.

Reference: draftkv/gpt2.py:25-44 (safetensors reader), :130-213 (model),
:216-245 (checkpoint lookup). LayerNorm, learned positions, fused QKV Conv1D
weights used as ``x @ W``, GELU-tanh MLP with biases, head tied to the token
embedding. No network fetch: checkpoints are read from a local directory.
"""

from __future__ import annotations

import json
import os
from pathlib import Path
from typing import Optional

import numpy as np
import torch

from .bpe import BPETokenizer  # noqa: F401  (gpt2.py:65; re-exported here)
from .decoder import Decoder, Layer

_NP = {"F32": np.float32, "F16": np.float16, "I64": np.int64, "I32": np.int32}

DISTILGPT2 = dict(n_layer=6, n_head=12, n_embd=768, vocab_size=50257, n_positions=1024, n_inner=None,
                  layer_norm_epsilon=1e-5)


def load_safetensors(path) -> dict:
    """Read a .safetensors file (8-byte little-endian header length, JSON
    header, raw little-endian tensors) into float32 numpy arrays; bf16 is
    widened exactly (gpt2.py:25-44). Nothing in the file is executed."""
    path = Path(path)
    with open(path, "rb") as f:
        n = int.from_bytes(f.read(8), "little")
        header = json.loads(f.read(n))
        blob = f.read()
    out = {}
    for name, meta in header.items():
        if name == "__metadata__":
            continue
        lo, hi = meta["data_offsets"]
        raw = blob[lo:hi]
        if meta["dtype"] == "BF16":
            a = (np.frombuffer(raw, np.uint16).astype(np.uint32) << 16).view(np.float32)
        elif meta["dtype"] in _NP:
            a = np.frombuffer(raw, _NP[meta["dtype"]]).astype(np.float32)
        else:
            raise ValueError(f"{path}: unsupported dtype {meta['dtype']} for {name}")
        out[name] = a.reshape(meta["shape"])
    return out


def gpt2_random_weights(cfg: dict, seed: int = 0, std: float = 0.02) -> dict:
    """Random-init GPT-2 weights (no checkpoint offline): matrices and
    embeddings ~ N(0, std) from ``np.random.default_rng(seed)`` in the order
    wte, wpe, then per block c_attn, attn c_proj, c_fc, mlp c_proj; LayerNorm
    weights 1, biases 0; float32."""
    rng = np.random.default_rng(seed)
    d, V, P, L = cfg["n_embd"], cfg["vocab_size"], cfg["n_positions"], cfg["n_layer"]
    ff = cfg.get("n_inner") or 4 * d
    f32 = np.float32

    def R(*s):
        return (rng.standard_normal(s) * std).astype(f32)

    w = {"wte.weight": R(V, d), "wpe.weight": R(P, d)}
    for i in range(L):
        p = f"h.{i}."
        w[p + "attn.c_attn.weight"] = R(d, 3 * d)
        w[p + "attn.c_proj.weight"] = R(d, d)
        w[p + "mlp.c_fc.weight"] = R(d, ff)
        w[p + "mlp.c_proj.weight"] = R(ff, d)
        w[p + "attn.c_attn.bias"] = np.zeros(3 * d, f32)
        w[p + "attn.c_proj.bias"] = np.zeros(d, f32)
        w[p + "mlp.c_fc.bias"] = np.zeros(ff, f32)
        w[p + "mlp.c_proj.bias"] = np.zeros(d, f32)
        for n in ("ln_1", "ln_2"):
            w[p + n + ".weight"] = np.ones(d, f32)
            w[p + n + ".bias"] = np.zeros(d, f32)
    w["ln_f.weight"] = np.ones(d, f32)
    w["ln_f.bias"] = np.zeros(d, f32)
    return w


class GPT2(Decoder):
    """gpt2.py:130-213 on the GPU."""

    norm = "layer"
    mlp = "gelu"
    layout = 0

    def __init__(self, weights: dict, config: dict, *, dtype=torch.float32, device=None) -> None:
        self._setup_device(dtype, device)
        self.cfg = config
        self.n_layers = config["n_layer"]
        self.n_heads = config["n_head"]
        self.n_kv_heads = self.n_heads
        self.d_model = config["n_embd"]
        self.d_head = self.d_model // self.n_heads
        self.vocab_size = config["vocab_size"]
        self.eps = config.get("layer_norm_epsilon", 1e-5)
        w = weights
        pre = "transformer." if "transformer.wte.weight" in w else ""
        self.emb = self._v(w[f"{pre}wte.weight"])
        self.pos_table = self._v(w[f"{pre}wpe.weight"])
        self.layers = []
        for i in range(self.n_layers):
            g = lambda n: w[f"{pre}h.{i}.{n}"]
            p = Layer()
            p.n1w, p.n1b = self._v(g("ln_1.weight")), self._v(g("ln_1.bias"))
            p.wqkv, p.bqkv = self._w(g("attn.c_attn.weight"), 0), self._v(g("attn.c_attn.bias"))
            p.wo, p.bo = self._w(g("attn.c_proj.weight"), 0), self._v(g("attn.c_proj.bias"))
            p.n2w, p.n2b = self._v(g("ln_2.weight")), self._v(g("ln_2.bias"))
            p.w1, p.b1 = self._w(g("mlp.c_fc.weight"), 0), self._v(g("mlp.c_fc.bias"))
            p.w2, p.b2 = self._w(g("mlp.c_proj.weight"), 0), self._v(g("mlp.c_proj.bias"))
            self.layers.append(p)
        self.nfw, self.nfb = self._v(w[f"{pre}ln_f.weight"]), self._v(w[f"{pre}ln_f.bias"])
        self.head = self.emb                       # tied: logits = h @ wte.T (gpt2.py:213)
        self.head_layout = 1
        self._tile_weights()

    @classmethod
    def from_dir(cls, d, **kw) -> "GPT2":                             # gpt2.py:169-174
        d = Path(d)
        cfg = json.loads((d / "config.json").read_text())
        cfg.setdefault("vocab_size", 50257)
        return cls(load_safetensors(d / "model.safetensors"), cfg, **kw)

    @classmethod
    def random(cls, config: Optional[dict] = None, seed: int = 0, std: float = 0.02, **kw) -> "GPT2":
        """Random-init model of the given shape (distilgpt2 by default)."""
        cfg = dict(config or DISTILGPT2)
        return cls(gpt2_random_weights(cfg, seed, std), cfg, **kw)


def default_model_dir() -> Optional[Path]:                               # gpt2.py:216-229
    """A local distilgpt2 checkpoint: $DRAFTKV_GPT2_DIR or ~/.cache/draftkv/distilgpt2; None if absent."""
    env = os.environ.get("DRAFTKV_GPT2_DIR")
    for c in ([Path(env)] if env else []) + [Path.home() / ".cache" / "draftkv" / "distilgpt2"]:
        if (c / "model.safetensors").exists() and (c / "config.json").exists():
            return c
    return None


def load_real_model(d=None, **kw):                                       # gpt2.py:232-245
    """Returns (model, tokenizer) from a local checkpoint; raises FileNotFoundError
    when there is none. The tokenizer is None when the directory has no
    vocab.json / merges.txt."""
    d = Path(d) if d else default_model_dir()
    if d is None:
        raise FileNotFoundError("no distilgpt2 checkpoint; set DRAFTKV_GPT2_DIR (no download here)")
    tok = None
    if (d / "vocab.json").exists() and (d / "merges.txt").exists():
        tok = BPETokenizer(d / "vocab.json", d / "merges.txt")
    return GPT2.from_dir(d, **kw), tok
