"""Whole decodes at the model shapes of the benchmark configurations.

* distilgpt2 shape (6 layers, d_model 768, 12 heads, vocab 50257, float32,
  seed-0 weights N(0, 0.02)), a 512-token prompt, 128 greedy tokens, int8
  keep 1, gamma 4, 16-token pages: tokens and per-round accepted runs equal the
  oracle engine's on the same weights and prompt, and equal the GPU's own
  full-KV decoding (reference tests/test_lossless.py:28-35).
* SmolLM2-135M shape (30 layers, 576 wide, 9/3 GQA heads, head_dim 64),
  bf16, batch 4 of 4096-token prompts, int4 group-32 fp16-meta keep 0.5,
  gamma 8: greedy output equals full-KV decoding, and the mirror's kept rows
  of layers 0 and 1 hold the oracle's quantization of the full cache's rows
  at their positions, bit for bit, with the sink and recent rows kept.
* Llama-3-8B layer shape (head_dim 128, 32/8 heads, SwiGLU 14336, vocab
  128256), 3 layers, bf16, batch 4 of ragged ~4k-token prompts, arms
  switched between int8 group-64 keep 1 and int4 group-32 keep 0.25 every 3
  rounds: greedy output equals full-KV decoding. These are the head_dim-128
  kernels the benchmark runs (LDS-ring int4 drafter, register-staged int8
  drafter, MFMA verify attention, compile-time requantize).
"""

import numpy as np
import pytest
import torch

from oracle.config import Cfg
from oracle.quant import quantize_codes

pytestmark = pytest.mark.gpu


class Switch:
    """Arms switched every ``period`` rounds, fixed gamma (the controller protocol)."""

    def __init__(self, arms, gamma, period):
        self.arms, self.gamma, self.period, self.n = list(arms), gamma, period, 0

    def select(self, ctx, key=None):
        arm = self.arms[(self.n // self.period) % len(self.arms)]
        self.n += 1
        return arm, self.gamma

    def update(self, cfg, gamma, accepted, ctx, key=None):
        pass


def _prompt(seed, n, vocab):
    return [int(x) for x in np.random.default_rng(seed).integers(0, vocab, n)]


@pytest.fixture(autouse=True)
def _free():
    yield
    import gc
    gc.collect()
    torch.cuda.empty_cache()


@pytest.mark.timeout(600)
def test_distilgpt2_shape_matches_oracle_engine(dev):
    import oracle.models as om
    from draftkv import CompressionConfig, DraftKVEngine, FixedPolicy
    from draftkv.gpt2 import DISTILGPT2, GPT2
    from oracle.engine import Engine, fixed
    cfg = dict(DISTILGPT2)
    w = om.gpt2_random_weights(cfg, seed=0, std=0.02)
    prompt = [int(x) for x in np.random.default_rng(1).integers(0, cfg["vocab_size"], 512)]
    m = GPT2(w, cfg)
    arm = CompressionConfig(8, 1.0)
    r = DraftKVEngine(m, FixedPolicy(arm, 4), seed=0).generate(prompt, 128, 0.0)
    base = DraftKVEngine(m, seed=0).generate_baseline(prompt, 128, 0.0)
    assert r.tokens == base
    assert r.new_tokens == 128 and len(r.tokens) == 512 + 128
    ro = Engine(om.GPT2(w, cfg), fixed(Cfg(8, 1.0), 4), seed=0).generate(prompt, 128, 0.0)
    assert r.tokens == ro.tokens
    assert [x.accepted for x in r.rounds] == [x.accepted for x in ro.rounds]
    assert [x.gamma for x in r.rounds] == [x.gamma for x in ro.rounds]


@pytest.mark.timeout(600)
def test_smollm2_shape_bf16_lossless_and_mirror_codes(dev):
    from draftkv import CompressionConfig, DraftKVEngine, FixedPolicy
    from draftkv.llama import SMOLLM2_135M, LlamaLike
    m = LlamaLike.random(SMOLLM2_135M, seed=0, std=0.02, dtype=torch.bfloat16)
    V = m.vocab_size
    prompts = [_prompt(100 + s, 4096, V) for s in range(4)]
    arm = CompressionConfig(4, 0.5, group=32, scale_fp16=True)
    eng = DraftKVEngine(m, FixedPolicy(arm, 8), seed=0)
    res = eng.generate_batch(prompts, 40, 0.0)
    base = DraftKVEngine(m, seed=0).generate_baseline_batch(prompts, 40, 0.0)
    assert [r.tokens for r in res] == base
    assert all(len(r.tokens) == 4096 + 40 and r.new_tokens >= 40 for r in res)
    md, full = eng.last_mirror, eng.last_full
    ocfg = Cfg(4, 0.5, group=32, meta="f16")
    lens = full.lengths()
    bud = md.budgets()
    for layer in (0, 1):
        for s in range(4):
            g = md.read_codes(layer, s)
            pos = g["pos"].astype(np.int64)
            n = int(lens[s])
            # at most the budget (a resync truncates the drafted rows and appends
            # the accepted ones, which may leave it a few rows short)
            assert int(bud[layer, s]) - 9 <= pos.size <= min(n, int(bud[layer, s])), (layer, s)
            assert pos.tolist() == sorted(set(pos.tolist())) and pos.max() == n - 1
            # the sink rows stay; the recent window protects the newest rows at
            # each eviction, drafted rows included, so after a rollback the
            # oldest of the last 32 positions may be gone
            assert set(range(4)) <= set(pos.tolist())
            k, v, p = full.read(layer, s)
            assert p.tolist() == list(range(n))
            for name, x in (("k", k), ("v", v)):
                codes, scale, lo, _ = quantize_codes(x[pos], 4, 32, "f16")
                assert np.array_equal(g[name + "_codes"], codes), (layer, s, name)
                assert np.array_equal(g[name + "_scale"].view(np.uint32), scale.view(np.uint32)), (layer, s, name)
                assert np.array_equal(g[name + "_lo"].view(np.uint32), lo.view(np.uint32)), (layer, s, name)


@pytest.mark.timeout(600)
def test_llama8b_layer_shape_lossless_across_arm_switch(dev):
    from draftkv import CompressionConfig, DraftKVEngine
    from draftkv.llama import LLAMA3_8B, LlamaLike
    m = LlamaLike.random(dict(LLAMA3_8B, num_hidden_layers=3), seed=1, std=0.02, dtype=torch.bfloat16)
    prompts = [_prompt(200 + s, n, m.vocab_size) for s, n in enumerate((4096, 4100, 4500, 4999))]
    arms = [CompressionConfig(8, 1.0, group=64, scale_fp16=True),
            CompressionConfig(4, 0.25, group=32, scale_fp16=True)]
    eng = DraftKVEngine(m, Switch(arms, 5, 3), seed=0)
    res = eng.generate_batch(prompts, 48, 0.0)
    base = DraftKVEngine(m, seed=0).generate_baseline_batch(prompts, 48, 0.0)
    assert [r.tokens for r in res] == base
    used = {x.cfg for x in res[0].rounds}
    assert used == set(arms), used
    assert res[0].cache_rebuilds >= 3
