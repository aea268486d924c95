"""The oracle's bf16 storage model on the CPU: ``bf16_round`` against
torch's float32 -> bfloat16 conversion (round to nearest even, on normal,
subnormal, tie, infinite and NaN inputs), and the rounded forwards' basic
properties (identity rounding is the reference forward; bf16 rounding moves
the logits by a small amount that shrinks with the rounding's own size)."""

import numpy as np
import pytest
import torch

import oracle.models as om
from oracle.caches import FullKVCache


def test_bf16_round_equals_torch_conversion():
    rng = np.random.default_rng(0)
    x = np.concatenate([
        rng.standard_normal(100000).astype(np.float32) * 10.0 ** rng.integers(-30, 30, 100000),
        np.array([0.0, -0.0, 1.0, -1.0, np.inf, -np.inf, 3.4e38, -3.4e38, 1e-40, -1e-40, 1.17e-38], np.float32),
        # exact ties: low 16 bits 0x8000 with even and odd kept bits
        (np.array([0x3F808000, 0x3F818000, 0xBF808000, 0x00018000], np.uint32)).view(np.float32),
    ]).astype(np.float32)
    want = torch.from_numpy(x).to(torch.bfloat16).float().numpy()
    got = om.bf16_round(x)
    assert got.dtype == np.float32
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    nan = om.bf16_round(np.array([np.nan], np.float32))
    assert np.isnan(nan).all()


def test_bf16_round_of_float64_rounds_through_float32():
    x = np.random.default_rng(1).standard_normal(1000)
    assert np.array_equal(om.bf16_round(x), om.bf16_round(x.astype(np.float32)))


@pytest.mark.parametrize("family", ["llama", "gpt2"])
def test_rounded_forward(family):
    if family == "llama":
        w, cfg = om.demo_llama_weights(n_layers=2, d_model=64, n_heads=8, n_kv_heads=2, vocab_size=97,
                                       attn_bias=True, attn_gain=1.0, attn_sharpness=1.0)
        w = {k: om.bf16_round(v) for k, v in w.items()}
        mk = lambda r: om.LlamaLike(w, cfg, act_round=r)
    else:
        cfg = dict(n_layer=2, n_head=4, n_embd=64, vocab_size=97, n_positions=128)
        w = {k: om.bf16_round(v) for k, v in om.gpt2_random_weights(cfg, seed=0, std=0.2).items()}
        mk = lambda r: om.GPT2(w, cfg, act_round=r)
    toks = np.random.default_rng(2).integers(0, 97, 30)
    z = mk(None).forward(toks, FullKVCache(2), 0)
    assert np.array_equal(mk(lambda a: a).forward(toks, FullKVCache(2), 0), z)
    zb = mk(om.bf16_round).forward(toks, FullKVCache(2), 0)
    d = np.abs(zb - z)
    # bf16 storage moves the logits by a few bf16 roundings' worth, never by their size
    assert 0 < d.max() < 0.05 * np.abs(z).max()
    # a finer rounding (12 dropped bits instead of 16) moves them ~16x less
    def r12(a):
        u = np.ascontiguousarray(np.asarray(a, np.float32)).view(np.uint32).astype(np.uint64)
        return ((((u + 0x7FF + ((u >> 12) & 1)) >> 12) << 12).astype(np.uint32)).view(np.float32)
    d12 = np.abs(mk(r12).forward(toks, FullKVCache(2), 0) - z)
    assert np.sqrt((d12 ** 2).mean()) < np.sqrt((d ** 2).mean()) / 4
