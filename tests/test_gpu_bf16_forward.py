"""bf16 model forwards against the float32 oracle on the same bf16 weights,
and models built on the GPU from checkpoints written to disk.

The device's bf16 forward stores every matrix product's operands and result
in bf16, and the full cache's K/V rows; it accumulates in float32. The
oracle runs the reference's arithmetic (float32, float64 where numpy
promotes) on the same bf16 weight values. The tolerance comes from bf16
storage itself: the oracle's forward with bf16 rounding at those storage
points (``act_round=bf16_round``) moves the logits by delta = max |z_bf16 -
z_f32| (and rho in RMS). The device logits must lie within 2 delta of the
float32 oracle at every entry and within 2 rho in RMS, and must pick the
oracle's argmax in every row whose top-two margin exceeds 4 delta. Float32
models keep the 2e-3 relative / 1e-3 absolute bound.

Reference: draftkv/llama.py:175-225, draftkv/gpt2.py:25-44 (checkpoint
reader), :182-213, tests/test_gpt2.py:25-38 (a fake checkpoint on disk).
"""

import gc
import json

import numpy as np
import pytest
import torch

import oracle.models as om
from oracle.caches import FullKVCache as OFull

pytestmark = pytest.mark.gpu

RTOL, ATOL = 2e-3, 1e-3


def _rms(a) -> float:
    return float(np.sqrt((np.asarray(a, np.float64) ** 2).mean()))


def check_bf16_logits(z_dev, z32, zr, what):
    """The bf16 tolerance rule above; returns (delta, max device error)."""
    assert z_dev.shape == z32.shape == zr.shape, what
    d_r = np.abs(zr.astype(np.float64) - z32)
    d = np.abs(z_dev.astype(np.float64) - z32)
    delta = float(d_r.max())
    assert delta > 0, f"{what}: bf16 storage left the logits unchanged (no rounding modelled?)"
    assert d.max() <= 2 * delta, f"{what}: max error {d.max():.3g} > 2 x {delta:.3g}"
    assert _rms(d) <= 2 * _rms(d_r), f"{what}: RMS error {_rms(d):.3g} > 2 x {_rms(d_r):.3g}"
    top = np.sort(z32, -1)[:, -2:]
    sure = (top[:, 1] - top[:, 0]) > 4 * delta
    assert np.array_equal(z_dev.argmax(-1)[sure], z32.argmax(-1)[sure]), f"{what}: argmax differs"
    return delta, float(d.max())


def _run(model, toks, cache, split):
    """Logits of a prefill of toks[:split] then one-token steps over the rest."""
    rows = [model.forward(toks[:split], cache, 0)]
    for i in range(split, len(toks)):
        rows.append(model.forward(toks[i:i + 1], cache, i))
    return np.concatenate(rows, 0)


def _llama_weights(cfg, seed, dev, tied):
    """bf16 weights ~ N(0, 0.02) drawn on the device (norm weights 1)."""
    g = torch.Generator(device=dev)
    g.manual_seed(seed)
    d, H, KV = cfg["hidden_size"], cfg["num_attention_heads"], cfg["num_key_value_heads"]
    D, ff, V = cfg["head_dim"], cfg["intermediate_size"], cfg["vocab_size"]

    def R(*shape):
        return torch.empty(shape, dtype=torch.bfloat16, device=dev).normal_(0.0, 0.02, generator=g)

    ones = lambda n: torch.ones(n, dtype=torch.bfloat16, device=dev)
    w = {"model.embed_tokens.weight": R(V, d), "model.norm.weight": ones(d)}
    if not tied:
        w["lm_head.weight"] = R(V, d)
    for i in range(cfg["num_hidden_layers"]):
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
    return w


def _shapes():
    from draftkv.llama import LLAMA3_8B, SMOLLM2_135M
    return {"llama3_8b_width_2_layers": (dict(LLAMA3_8B, num_hidden_layers=2), False),
            "smollm2_135m": (dict(SMOLLM2_135M), True)}


@pytest.mark.parametrize("shape", ["llama3_8b_width_2_layers", "smollm2_135m"])
def test_bf16_llama_forward_matches_oracle(dev, shape):
    """A 2-layer model of Llama-3-8B's width (4096 hidden, 32/8 heads of 128,
    SwiGLU 14336, 128256-token untied head, RoPE theta 5e5) and the SmolLM2-135M
    shape (30 layers, 576 hidden, 9/3 heads of 64, tied head): 23 prefill rows
    and 3 decode steps, by the bf16 tolerance rule."""
    from draftkv.llama import LlamaLike
    cfg, tied = _shapes()[shape]
    w = _llama_weights(cfg, 3, dev, tied)
    g = LlamaLike(w, cfg, dtype=torch.bfloat16)
    wn = {k: v.float().cpu().numpy() for k, v in w.items()}
    toks = np.random.default_rng(4).integers(0, cfg["vocab_size"], 26)
    z_dev = _run(g, toks, g.new_cache(), 23)
    del g, w
    gc.collect()
    torch.cuda.empty_cache()
    L = cfg["num_hidden_layers"]
    z32 = _run(om.LlamaLike(wn, cfg), toks, OFull(L), 23)
    zr = _run(om.LlamaLike(wn, cfg, act_round=om.bf16_round), toks, OFull(L), 23)
    delta, err = check_bf16_logits(z_dev, z32, zr, shape)
    print(f"{shape}: bf16 storage moves the logits by up to {delta:.4g}; device error {err:.4g}")


def test_bf16_gpt2_forward_matches_oracle(dev):
    """A 2-layer GPT-2 of distilgpt2's width (768 hidden, 12 heads, GELU 3072,
    learned positions, LayerNorm with biases) whose head is the tied
    50257-row embedding, by the bf16 tolerance rule."""
    from draftkv import gpt2
    cfg = dict(gpt2.DISTILGPT2, n_layer=2)
    w = {k: om.bf16_round(v) for k, v in gpt2.gpt2_random_weights(cfg, seed=5, std=0.05).items()}
    rng = np.random.default_rng(6)
    for k in w:   # nonzero biases and LayerNorm affine terms, so every bias path counts
        if k.endswith("bias"):
            w[k] = om.bf16_round(0.02 * rng.standard_normal(w[k].shape))
    g = gpt2.GPT2(w, cfg, dtype=torch.bfloat16)
    toks = rng.integers(0, cfg["vocab_size"], 26)
    z_dev = _run(g, toks, g.new_cache(), 23)
    z32 = _run(om.GPT2(w, cfg), toks, OFull(2), 23)
    zr = _run(om.GPT2(w, cfg, act_round=om.bf16_round), toks, OFull(2), 23)
    check_bf16_logits(z_dev, z32, zr, "gpt2 bf16")


# ------------------------------------------------------------------ checkpoints on disk
def test_gpt2_f32_checkpoint_from_dir_matches_oracle(dev, tmp_path):
    """A float32 GPT-2 checkpoint (HF key names under ``transformer.``,
    written by the safetensors package) and its config.json: GPT2.from_dir
    builds the model on the GPU and its logits match the oracle's on the
    weights written."""
    from safetensors.numpy import save_file

    from draftkv import gpt2
    cfg = dict(n_layer=2, n_head=4, n_embd=64, vocab_size=97, n_positions=128, n_inner=None,
               layer_norm_epsilon=1e-5)
    w = om.gpt2_random_weights(cfg, seed=7, std=0.2)
    rng = np.random.default_rng(8)
    for k in w:
        if k.endswith("bias"):
            w[k] = (0.05 * rng.standard_normal(w[k].shape)).astype(np.float32)
    save_file({"transformer." + k: v for k, v in w.items()}, str(tmp_path / "model.safetensors"))
    (tmp_path / "config.json").write_text(json.dumps({k: v for k, v in cfg.items() if v is not None}))
    g = gpt2.GPT2.from_dir(tmp_path)
    assert g.wdtype == torch.float32 and g.n_layers == 2 and g.vocab_size == 97
    toks = rng.integers(0, 97, 40)
    z = _run(g, toks, g.new_cache(), 37)
    want = _run(om.GPT2(w, cfg), toks, OFull(2), 37)
    np.testing.assert_allclose(z, want, rtol=RTOL, atol=ATOL)
    m, tok = gpt2.load_real_model(tmp_path)
    assert tok is None and m.n_layers == 2


def test_llama_bf16_checkpoint_from_dir_matches_oracle(dev, tmp_path):
    """A bf16 Llama checkpoint (GQA, q/k/v biases, untied head; written by
    the safetensors package from torch bf16 tensors) and its config.json:
    LlamaLike.from_dir builds it on the GPU as a float32 model (logits within
    2e-3 / 1e-3 of the oracle on the stored values) and as a bf16 model (the
    bf16 tolerance rule)."""
    from safetensors.torch import save_file

    from draftkv import llama
    cfg = dict(num_hidden_layers=2, hidden_size=128, num_attention_heads=8, num_key_value_heads=2, head_dim=16,
               intermediate_size=256, vocab_size=300, rms_norm_eps=1e-5, rope_theta=10000.0)
    g0 = torch.Generator().manual_seed(9)
    R = lambda *s: (0.1 * torch.randn(s, generator=g0)).to(torch.bfloat16)
    w = {"model.embed_tokens.weight": R(300, 128), "model.norm.weight": (1 + R(128)).to(torch.bfloat16),
         "lm_head.weight": R(300, 128)}
    for i in range(2):
        p = f"model.layers.{i}."
        w[p + "input_layernorm.weight"] = (1 + R(128)).to(torch.bfloat16)
        w[p + "post_attention_layernorm.weight"] = (1 + R(128)).to(torch.bfloat16)
        w[p + "self_attn.q_proj.weight"], w[p + "self_attn.q_proj.bias"] = R(128, 128), R(128)
        w[p + "self_attn.k_proj.weight"], w[p + "self_attn.k_proj.bias"] = R(32, 128), R(32)
        w[p + "self_attn.v_proj.weight"], w[p + "self_attn.v_proj.bias"] = R(32, 128), R(32)
        w[p + "self_attn.o_proj.weight"] = R(128, 128)
        w[p + "mlp.gate_proj.weight"], w[p + "mlp.up_proj.weight"] = R(256, 128), R(256, 128)
        w[p + "mlp.down_proj.weight"] = R(128, 256)
    save_file(w, str(tmp_path / "model.safetensors"))
    (tmp_path / "config.json").write_text(json.dumps(cfg))
    wn = {k: v.float().numpy() for k, v in w.items()}
    toks = np.random.default_rng(10).integers(0, 300, 40)
    z32 = _run(om.LlamaLike(wn, cfg), toks, OFull(2), 37)
    g = llama.LlamaLike.from_dir(tmp_path)
    assert g.wdtype == torch.float32 and g.n_kv_heads == 2
    np.testing.assert_allclose(_run(g, toks, g.new_cache(), 37), z32, rtol=RTOL, atol=ATOL)
    gb = llama.LlamaLike.from_dir(tmp_path, dtype=torch.bfloat16)
    zr = _run(om.LlamaLike(wn, cfg, act_round=om.bf16_round), toks, OFull(2), 37)
    check_bf16_logits(_run(gb, toks, gb.new_cache(), 37), z32, zr, "llama bf16 checkpoint")
    m, tok = llama.load_llama(tmp_path, dtype=torch.bfloat16)
    assert tok is None and m.wdtype == torch.bfloat16
