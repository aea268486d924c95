"""The three model forwards that drive the decode round, restated in numpy.

* ``TinyTransformer`` / ``demo_model``  -- reference draftkv/model.py:18-156
* ``GPT2``                              -- reference draftkv/gpt2.py:114-213
* ``LlamaLike`` / ``demo_llama``        -- reference draftkv/llama.py:93-298

Each ``forward(tokens, cache, start_pos)`` appends K/V to ``cache`` and reads
it back exactly as the reference does, so it runs against either oracle cache.
``GPT2`` and ``LlamaLike`` take an optional ``act_round`` (e.g. ``bf16_round``)
that models a bf16 forward's storage points -- every matrix product's inputs
and result, and the K/V rows cached -- in otherwise unchanged arithmetic; it
measures how far bf16 storage alone moves the logits. Without it the forward
is the reference's.
The weight initialisers consume ``np.random.default_rng(seed)`` in the
reference's order, so a given seed yields the reference's weights.
"""

from __future__ import annotations

import numpy as np

from .attention import attend


def rms_norm(x, w, eps):                      # model.py:18-19, llama.py:93-94
    return x / np.sqrt((x * x).mean(-1, keepdims=True) + eps) * w


def layer_norm(x, w, b, eps=1e-5):            # gpt2.py:120-123
    mu = x.mean(-1, keepdims=True)
    var = x.var(-1, keepdims=True)
    return (x - mu) / np.sqrt(var + eps) * w + b


def gelu_new(x):                              # gpt2.py:126-127
    return 0.5 * x * (1.0 + np.tanh(0.7978845608028654 * (x + 0.044715 * x ** 3)))


def silu(x):                                  # llama.py:102-103
    return x / (1.0 + np.exp(-x))


def rotate_half(x):                           # llama.py:106-109
    h = x.shape[-1] // 2
    return np.concatenate([-x[..., h:], x[..., :h]], axis=-1)


def bf16_round(x) -> np.ndarray:
    """Round to the nearest bfloat16 value, ties to even (the top 16 bits of a
    float32 after adding 0x7FFF plus the lowest kept bit); float32 result.
    Inputs in float64 are first rounded to float32. Used by the forwards'
    ``act_round`` to model a bf16 device forward's storage points; the
    reference itself has no bf16 arithmetic."""
    u = np.ascontiguousarray(np.asarray(x, np.float32)).view(np.uint32).astype(np.uint64)
    u = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16) << 16
    return u.astype(np.uint32).view(np.float32)


def _keep(x):
    return x


def sinusoidal(n: int, d: int) -> np.ndarray:   # model.py:86-94
    p = np.arange(n)[:, None]
    i = np.arange(0, d, 2)[None, :]
    ang = p / np.power(10000.0, i / d)
    out = np.zeros((n, d))
    out[:, 0::2] = np.sin(ang)
    out[:, 1::2] = np.cos(ang)
    return out


# --------------------------------------------------------------------- tiny
class TinyTransformer:
    """model.py:28-133."""

    def __init__(self, vocab_size=256, d_model=64, n_heads=4, n_layers=4, d_ff=None,
                 max_pos=4096, attn_sharpness=1.0, attn_gain=1.0, seed=0):
        rng = np.random.default_rng(seed)
        self.vocab_size, self.d_model, self.n_heads, self.n_layers = vocab_size, d_model, n_heads, n_layers
        self.n_kv_heads = n_heads
        self.d_head = d_model // n_heads
        d_ff = d_ff or 2 * d_model
        s = 1.0 / np.sqrt(d_model)
        f32 = np.float32
        self.emb = (rng.standard_normal((vocab_size, d_model)) * s).astype(f32)
        self.pos_emb = sinusoidal(max_pos, d_model).astype(f32)
        self.layers = []
        for _ in range(n_layers):
            wq = (rng.standard_normal((d_model, d_model)) * s * attn_sharpness).astype(f32)
            wk = (rng.standard_normal((d_model, d_model)) * s).astype(f32)
            wv = (rng.standard_normal((d_model, d_model)) * s).astype(f32)
            wo = (rng.standard_normal((d_model, d_model)) * s * attn_gain).astype(f32)
            w1 = (rng.standard_normal((d_model, d_ff)) * s).astype(f32)
            w2 = (rng.standard_normal((d_ff, d_model)) * s).astype(f32)
            self.layers.append(dict(n1=np.ones(d_model, f32), wq=wq, wk=wk, wv=wv, wo=wo,
                                    n2=np.ones(d_model, f32), w1=w1, w2=w2))
        self.nf = np.ones(d_model, f32)
        self.head = (rng.standard_normal((d_model, vocab_size)) * s).astype(f32)

    def forward(self, tokens, cache, start_pos):
        tokens = np.asarray(tokens, np.int64).reshape(-1)
        T = tokens.size
        pos = np.arange(start_pos, start_pos + T)
        h = self.emb[tokens] + self.pos_emb[pos]
        H, D = self.n_heads, self.d_head
        for L, p in enumerate(self.layers):
            x = rms_norm(h, p["n1"], 1e-6)
            q = (x @ p["wq"]).reshape(T, H, D)
            k = (x @ p["wk"]).reshape(T, H, D)
            v = (x @ p["wv"]).reshape(T, H, D)
            cache.append(L, k, v, pos)
            ck, cv, cpos = cache.read(L)
            attn, _, mp = attend(q, ck, cv, cpos, pos)
            cache.note_attention(L, mp)
            h = h + attn.reshape(T, H * D) @ p["wo"]
            x = rms_norm(h, p["n2"], 1e-6)
            h = h + np.maximum(x @ p["w1"], 0.0) @ p["w2"]
        return (rms_norm(h, self.nf, 1e-6) @ self.head).astype(np.float32)


def demo_model(seed: int = 1, **kw) -> TinyTransformer:     # model.py:143-156
    params = dict(vocab_size=128, d_model=64, n_heads=4, n_layers=3,
                  attn_sharpness=4.0, attn_gain=4.0, seed=seed)
    params.update(kw)
    return TinyTransformer(**params)


# --------------------------------------------------------------------- gpt2
class GPT2:
    """gpt2.py:130-213 (LayerNorm, fused QKV Conv1D ``x @ W``, GELU-tanh, tied head)."""

    def __init__(self, weights: dict, config: dict, act_round=None):
        self.r = act_round or _keep     # applied to every matrix product's input and output, and K/V
        self.n_layers = config["n_layer"]
        self.n_heads = config["n_head"]
        self.n_kv_heads = self.n_heads
        self.d_model = config["n_embd"]
        self.d_head = self.d_model // self.n_heads
        self.vocab_size = config["vocab_size"]
        self.eps = config.get("layer_norm_epsilon", 1e-5)
        w = weights
        pre = "transformer." if "transformer.wte.weight" in w else ""
        self.wte, self.wpe = w[f"{pre}wte.weight"], w[f"{pre}wpe.weight"]
        self.blocks = []
        for i in range(self.n_layers):
            p = f"{pre}h.{i}."
            self.blocks.append({k: w[p + n] for k, n in (
                ("ln1w", "ln_1.weight"), ("ln1b", "ln_1.bias"),
                ("qkvw", "attn.c_attn.weight"), ("qkvb", "attn.c_attn.bias"),
                ("ow", "attn.c_proj.weight"), ("ob", "attn.c_proj.bias"),
                ("ln2w", "ln_2.weight"), ("ln2b", "ln_2.bias"),
                ("fcw", "mlp.c_fc.weight"), ("fcb", "mlp.c_fc.bias"),
                ("pw", "mlp.c_proj.weight"), ("pb", "mlp.c_proj.bias"))})
        self.lnfw, self.lnfb = w[f"{pre}ln_f.weight"], w[f"{pre}ln_f.bias"]

    def forward(self, tokens, cache, start_pos):
        tokens = np.asarray(tokens, np.int64).reshape(-1)
        T = tokens.size
        pos = np.arange(start_pos, start_pos + T)
        h = self.wte[tokens] + self.wpe[pos]
        H, D = self.n_heads, self.d_head
        r = self.r
        if r is _keep:
            for L, p in enumerate(self.blocks):
                x = layer_norm(h, p["ln1w"], p["ln1b"], self.eps)
                qkv = x @ p["qkvw"] + p["qkvb"]
                q, k, v = np.split(qkv, 3, axis=-1)
                q, k, v = q.reshape(T, H, D), k.reshape(T, H, D), v.reshape(T, H, D)
                cache.append(L, k, v, pos)
                ck, cv, cpos = cache.read(L)
                attn, _, mp = attend(q, ck, cv, cpos, pos)
                cache.note_attention(L, mp)
                h = h + attn.reshape(T, H * D) @ p["ow"] + p["ob"]
                x = layer_norm(h, p["ln2w"], p["ln2b"], self.eps)
                h = h + gelu_new(x @ p["fcw"] + p["fcb"]) @ p["pw"] + p["pb"]
            h = layer_norm(h, self.lnfw, self.lnfb, self.eps)
            return (h @ self.wte.T).astype(np.float32)
        # the same forward with every product's operands and result passed through r
        for L, p in enumerate(self.blocks):
            x = r(layer_norm(h, p["ln1w"], p["ln1b"], self.eps))
            qkv = r(x @ p["qkvw"]) + p["qkvb"]
            q, k, v = np.split(qkv, 3, axis=-1)
            q, k, v = q.reshape(T, H, D), r(k.reshape(T, H, D)), r(v.reshape(T, H, D))
            cache.append(L, k, v, pos)
            ck, cv, cpos = cache.read(L)
            attn, _, mp = attend(q, ck, cv, cpos, pos)
            cache.note_attention(L, mp)
            h = h + r(r(attn.reshape(T, H * D)) @ p["ow"]) + p["ob"]
            x = r(layer_norm(h, p["ln2w"], p["ln2b"], self.eps))
            h = h + r(r(gelu_new(r(x @ p["fcw"]) + p["fcb"])) @ p["pw"]) + p["pb"]
        h = r(layer_norm(h, self.lnfw, self.lnfb, self.eps))
        return (h @ self.wte.T).astype(np.float32)


def gpt2_random_weights(cfg: dict, seed: int = 0, std: float = 0.02) -> dict:
    """Random-init GPT-2 weights (no checkpoint offline). Matrices and
    embeddings ~ N(0, std) drawn from ``default_rng(seed)`` in this order:
    wte, wpe, then per block c_attn.weight, c_proj.weight, c_fc.weight,
    mlp.c_proj.weight. LayerNorm weights 1, all biases 0. float32."""
    rng = np.random.default_rng(seed)
    d, V, P, L = cfg["n_embd"], cfg["vocab_size"], cfg["n_positions"], cfg["n_layer"]
    ff = cfg.get("n_inner") or 4 * d
    f32 = np.float32
    R = lambda *s: (rng.standard_normal(s) * std).astype(f32)
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


# -------------------------------------------------------------------- llama
class LlamaLike:
    """llama.py:112-225 (RMSNorm, RoPE with float64 tables, GQA by repeat, SwiGLU)."""

    def __init__(self, weights: dict, config: dict, act_round=None):
        c = config
        self.r = act_round or _keep     # applied to every matrix product's input and output, and K/V
        self.n_layers = c["num_hidden_layers"]
        self.d_model = c["hidden_size"]
        self.n_heads = c["num_attention_heads"]
        self.n_kv_heads = c.get("num_key_value_heads", self.n_heads)
        self.d_head = c.get("head_dim", self.d_model // self.n_heads)
        self.n_rep = self.n_heads // self.n_kv_heads
        self.vocab_size = c["vocab_size"]
        self.eps = c.get("rms_norm_eps", 1e-5)
        self.theta = float(c.get("rope_theta") or 10000.0)
        w = weights
        self.emb = w["model.embed_tokens.weight"]
        self.head = w.get("lm_head.weight", self.emb)
        self.final_norm = w["model.norm.weight"]
        self.layers = []
        for i in range(self.n_layers):
            p = f"model.layers.{i}."
            g = lambda n: w.get(p + n)
            self.layers.append(dict(
                n1=g("input_layernorm.weight"),
                q=g("self_attn.q_proj.weight"), qb=g("self_attn.q_proj.bias"),
                k=g("self_attn.k_proj.weight"), kb=g("self_attn.k_proj.bias"),
                v=g("self_attn.v_proj.weight"), vb=g("self_attn.v_proj.bias"),
                o=g("self_attn.o_proj.weight"), ob=g("self_attn.o_proj.bias"),
                n2=g("post_attention_layernorm.weight"),
                gate=g("mlp.gate_proj.weight"), up=g("mlp.up_proj.weight"),
                down=g("mlp.down_proj.weight")))

    def rope(self, pos):                                   # llama.py:164-172
        inv = 1.0 / (self.theta ** (np.arange(0, self.d_head, 2) / self.d_head))
        ang = np.outer(np.asarray(pos), inv)
        emb = np.concatenate([ang, ang], axis=-1)
        return np.cos(emb), np.sin(emb)

    def forward(self, tokens, cache, start_pos):
        tokens = np.asarray(tokens, np.int64).reshape(-1)
        T = tokens.size
        pos = np.arange(start_pos, start_pos + T)
        h = self.emb[tokens].astype(np.float32)
        H, KV, D = self.n_heads, self.n_kv_heads, self.d_head
        cos, sin = self.rope(pos)
        cos, sin = cos[:, None, :], sin[:, None, :]
        if self.r is not _keep:
            return self._forward_rounded(h, cache, pos, cos, sin)
        for L, p in enumerate(self.layers):
            x = rms_norm(h, p["n1"], self.eps)
            q, k, v = x @ p["q"].T, x @ p["k"].T, x @ p["v"].T
            if p["qb"] is not None:
                q, k, v = q + p["qb"], k + p["kb"], v + p["vb"]
            q, k, v = q.reshape(T, H, D), k.reshape(T, KV, D), v.reshape(T, KV, D)
            q = q * cos + rotate_half(q) * sin             # float64 from here
            k = k * cos + rotate_half(k) * sin
            cache.append(L, k, v, pos)
            ck, cv, cpos = cache.read(L)
            attn, _, mp = attend(q, ck, cv, cpos, pos, self.n_rep)
            cache.note_attention(L, mp)
            h = h + attn.reshape(T, H * D) @ p["o"].T + (p["ob"] if p["ob"] is not None else 0.0)
            x = rms_norm(h, p["n2"], self.eps)
            h = h + (silu(x @ p["gate"].T) * (x @ p["up"].T)) @ p["down"].T
        h = rms_norm(h, self.final_norm, self.eps)
        return (h @ self.head.T).astype(np.float32)


    def _forward_rounded(self, h, cache, pos, cos, sin):
        """``forward`` with every matrix product's operands and result, and the
        K/V rows appended, passed through ``self.r``."""
        r, T = self.r, h.shape[0]
        H, KV, D = self.n_heads, self.n_kv_heads, self.d_head
        for L, p in enumerate(self.layers):
            x = r(rms_norm(h, p["n1"], self.eps))
            q, k, v = r(x @ p["q"].T), r(x @ p["k"].T), r(x @ p["v"].T)
            if p["qb"] is not None:
                q, k, v = q + p["qb"], k + p["kb"], v + p["vb"]
            q, k, v = q.reshape(T, H, D), k.reshape(T, KV, D), v.reshape(T, KV, D)
            q = q * cos + rotate_half(q) * sin
            k = r(k * cos + rotate_half(k) * sin)
            v = r(v)
            cache.append(L, k, v, pos)
            ck, cv, cpos = cache.read(L)
            attn, _, mp = attend(q, ck, cv, cpos, pos, self.n_rep)
            cache.note_attention(L, mp)
            h = h + r(r(attn.reshape(T, H * D)) @ p["o"].T) + (p["ob"] if p["ob"] is not None else 0.0)
            x = r(rms_norm(h, p["n2"], self.eps))
            h = h + r(r(silu(r(x @ p["gate"].T)) * r(x @ p["up"].T)) @ p["down"].T)
        h = r(rms_norm(h, self.final_norm, self.eps))
        return (h @ self.head.T).astype(np.float32)


def demo_llama_weights(n_layers=4, d_model=64, n_heads=8, n_kv_heads=2, vocab_size=128,
                       intermediate=128, attn_bias=False, seed=0, attn_gain=4.0,
                       attn_sharpness=4.0):
    """llama.py:247-298: weights and config of the random-weight demo model,
    drawing from ``default_rng(seed)`` in the reference's order (including the
    throw-away draw the reference makes for the q bias when ``attn_bias``)."""
    rng = np.random.default_rng(seed)
    dh = d_model // n_heads
    s = 1.0 / np.sqrt(d_model)
    f32 = np.float32

    def R(*shape, k=1.0):
        return (rng.standard_normal(shape) * s * k).astype(f32)

    w = {"model.embed_tokens.weight": R(vocab_size, d_model),
         "model.norm.weight": np.ones(d_model, f32)}
    for i in range(n_layers):
        p = f"model.layers.{i}."
        w[p + "input_layernorm.weight"] = np.ones(d_model, f32)
        w[p + "post_attention_layernorm.weight"] = np.ones(d_model, f32)
        w[p + "self_attn.q_proj.weight"] = R(n_heads * dh, d_model, k=attn_sharpness)
        w[p + "self_attn.k_proj.weight"] = R(n_kv_heads * dh, d_model)
        w[p + "self_attn.v_proj.weight"] = R(n_kv_heads * dh, d_model)
        w[p + "self_attn.o_proj.weight"] = R(d_model, n_heads * dh, k=attn_gain)
        if attn_bias:
            R(n_heads * dh)                       # consumed and discarded, as the reference does
            w[p + "self_attn.k_proj.bias"] = np.zeros(n_kv_heads * dh, f32) + 0.01
            w[p + "self_attn.v_proj.bias"] = np.zeros(n_kv_heads * dh, f32) + 0.01
            w[p + "self_attn.q_proj.bias"] = np.zeros(n_heads * dh, f32) + 0.01
        w[p + "mlp.gate_proj.weight"] = R(intermediate, d_model)
        w[p + "mlp.up_proj.weight"] = R(intermediate, d_model)
        w[p + "mlp.down_proj.weight"] = R(d_model, intermediate)
    cfg = dict(num_hidden_layers=n_layers, hidden_size=d_model, num_attention_heads=n_heads,
               num_key_value_heads=n_kv_heads, vocab_size=vocab_size, rms_norm_eps=1e-5,
               rope_theta=10000.0)
    return w, cfg


def demo_llama(**kw) -> LlamaLike:
    w, cfg = demo_llama_weights(**kw)
    return LlamaLike(w, cfg)
