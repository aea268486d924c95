"""The GPU model forwards and the decode-round engine against the oracle.

* logits of the three model families (tiny ReLU transformer, GPT-2, Llama with
  GQA and biases) within 2e-3 relative / 1e-3 absolute of the numpy oracle;
* batch invariance of the float32 forward: a verify block's rows equal the
  one-token decode rows bit for bit (the property exact greedy losslessness
  rests on);
* greedy losslessness, the reference's own test (tests/test_lossless.py:28-35,
  tests/test_paged.py:103-116): speculative output == full-KV decoding, for
  every reference config and gamma, with contiguous and paged full caches;
* token and accepted-run parity with the oracle engine on the same seed
  (greedy and temperature sampling);
* a batch of ragged prompts decodes to the same tokens as one at a time.
"""

import numpy as np
import pytest
import torch

import oracle.models as om
from oracle.caches import FullKVCache as OFull
from oracle.config import Cfg
from oracle.engine import Engine, fixed

pytestmark = pytest.mark.gpu

RTOL, ATOL = 2e-3, 1e-3

GPT2_SMALL = dict(n_layer=2, n_head=4, n_embd=64, vocab_size=97, n_positions=512, n_inner=None,
                  layer_norm_epsilon=1e-5)


def _pair(name):
    """(gpu model, oracle model) with identical weights."""
    from draftkv import gpt2, llama, model
    if name == "tiny":
        return model.demo_model(), om.demo_model()
    if name == "llama":
        return llama.demo_llama(), om.demo_llama()
    if name == "llama_bias":
        return llama.demo_llama(attn_bias=True, n_layers=2), om.demo_llama(attn_bias=True, n_layers=2)
    if name == "gpt2":
        w = om.gpt2_random_weights(GPT2_SMALL, seed=0, std=0.2)
        return gpt2.GPT2(w, GPT2_SMALL), om.GPT2(w, GPT2_SMALL)
    raise KeyError(name)


def _ocfg(c):
    return Cfg(c.bits, c.keep_frac, c.sink, c.recent, c.group, "f16" if c.scale_fp16 else "f32")


def _prompt(seed, n, vocab):
    return [int(x) for x in np.random.default_rng(seed).integers(0, vocab, n)]


MODELS = ["tiny", "llama", "llama_bias", "gpt2"]


@pytest.mark.parametrize("name", MODELS)
def test_forward_matches_oracle(dev, name):
    g, o = _pair(name)
    toks = np.array(_prompt(1, 41, g.vocab_size))
    oc = OFull(o.n_layers)
    want = o.forward(toks[:-1], oc, 0)
    want1 = o.forward(toks[-1:], oc, 40)
    gc = g.new_cache()
    got = g.forward(toks[:-1], gc, 0)
    got1 = g.forward(toks[-1:], gc, 40)
    assert got.shape == want.shape and got.dtype == np.float32
    np.testing.assert_allclose(got, want, rtol=RTOL, atol=ATOL)
    np.testing.assert_allclose(got1, want1, rtol=RTOL, atol=ATOL)
    assert gc.length == 41


@pytest.mark.parametrize("name", MODELS)
def test_verify_block_equals_decode_rows(dev, name):
    """The float32 forward is batch-invariant: T rows in one pass == T one-row passes."""
    g, _ = _pair(name)
    toks = np.array(_prompt(2, 37, g.vocab_size))
    a, b = g.new_cache(), g.new_cache()
    g.forward(toks[:30], a, 0)
    g.forward(toks[:30], b, 0)
    block = g.forward(toks[30:], a, 30)
    rows = np.stack([g.forward(toks[30 + i: 31 + i], b, 30 + i)[0] for i in range(7)])
    assert np.array_equal(block.view(np.uint32), rows.view(np.uint32))


@pytest.fixture(scope="module")
def tiny_setup():
    from draftkv import DraftKVEngine
    from draftkv.model import demo_model
    m = demo_model()
    prompt = _prompt(0, 192, m.vocab_size)
    base = DraftKVEngine(m, seed=0).generate_baseline(prompt, 32, 0.0)
    return m, prompt, base


def _configs():
    from draftkv import CompressionConfig as C
    return [C(16, 1.0), C(8, 1.0), C(4, 1.0), C(4, 0.5), C(3, 0.5), C(2, 0.25)]


@pytest.mark.parametrize("ci", range(6))
@pytest.mark.parametrize("gamma", [1, 3, 6])
def test_greedy_output_identical(dev, tiny_setup, ci, gamma):
    from draftkv import DraftKVEngine, FixedPolicy
    m, prompt, base = tiny_setup
    cfg = _configs()[ci]
    r = DraftKVEngine(m, FixedPolicy(cfg, gamma), seed=0).generate(prompt, 32, 0.0)
    assert r.tokens == base, f"{cfg.label()} gamma={gamma} diverged from full-KV decoding"
    assert r.new_tokens == 32 and r.verify_passes <= 32


def test_baseline_matches_oracle_tokens(dev, tiny_setup):
    m, prompt, base = tiny_setup
    assert Engine(om.demo_model(), fixed(Cfg(), 1), seed=0).generate_baseline(prompt, 32, 0.0) == base


@pytest.mark.parametrize("block_size", [4, 16])
def test_lossless_with_paged_authoritative_cache(dev, tiny_setup, block_size):
    from draftkv import CompressionConfig, DraftKVEngine, FixedPolicy, PagedKVCache
    m, _, _ = tiny_setup
    prompt = _prompt(3, 192, m.vocab_size)
    base = DraftKVEngine(m, seed=0).generate_baseline(prompt, 32, 0.0)
    eng = DraftKVEngine(m, FixedPolicy(CompressionConfig(4, 0.5), 5), seed=0,
                        full_cache_factory=lambda: PagedKVCache(m.n_layers, m.n_heads, m.d_head,
                                                                block_size=block_size, n_blocks=2048))
    r = eng.generate(prompt, 32, 0.0)
    assert r.tokens == base
    eng.last_full.pool.check_invariants()


@pytest.mark.parametrize("name", ["llama", "llama_bias", "gpt2"])
def test_lossless_other_families(dev, name):
    from draftkv import CompressionConfig, DraftKVEngine, FixedPolicy
    g, _ = _pair(name)
    prompt = _prompt(4, 100, g.vocab_size)
    base = DraftKVEngine(g, seed=0).generate_baseline(prompt, 24, 0.0)
    for cfg, gamma in ((CompressionConfig(4, 0.5), 4), (CompressionConfig(2, 0.25, group=32, scale_fp16=True), 6)):
        r = DraftKVEngine(g, FixedPolicy(cfg, gamma), seed=0).generate(prompt, 24, 0.0)
        assert r.tokens == base, f"{name} {cfg.label()}"


@pytest.mark.parametrize("ci,gamma", [(1, 4), (2, 3), (3, 5), (5, 4)])
def test_rounds_match_oracle_engine(dev, tiny_setup, ci, gamma):
    """Same tokens and the same accepted count in every round as the oracle engine."""
    from draftkv import DraftKVEngine, FixedPolicy
    m, prompt, _ = tiny_setup
    cfg = _configs()[ci]
    r = DraftKVEngine(m, FixedPolicy(cfg, gamma), seed=0).generate(prompt, 32, 0.0)
    o = Engine(om.demo_model(), fixed(_ocfg(cfg), gamma), seed=0).generate(prompt, 32, 0.0)
    assert r.tokens == o.tokens
    assert [x.accepted for x in r.rounds] == [x.accepted for x in o.rounds]
    assert r.cache_rebuilds == o.cache_rebuilds == 1


@pytest.mark.parametrize("temperature", [0.7, 1.0])
def test_sampling_matches_oracle_engine(dev, tiny_setup, temperature):
    """Temperature sampling with the same seed: same draws, same tokens, same accepted runs."""
    from draftkv import CompressionConfig, DraftKVEngine, FixedPolicy
    m, prompt, _ = tiny_setup
    cfg = CompressionConfig(4, 1.0)
    r = DraftKVEngine(m, FixedPolicy(cfg, 4), seed=7).generate(prompt, 32, temperature)
    o = Engine(om.demo_model(), fixed(_ocfg(cfg), 4), seed=7).generate(prompt, 32, temperature)
    assert r.tokens == o.tokens
    assert [x.accepted for x in r.rounds] == [x.accepted for x in o.rounds]
    base = Engine(om.demo_model(), fixed(_ocfg(cfg), 4), seed=7).generate_baseline(prompt, 16, temperature)
    from draftkv import DraftKVEngine as E
    assert E(m, seed=7).generate_baseline(prompt, 16, temperature) == base


def test_batched_generate_equals_one_at_a_time(dev, tiny_setup):
    from draftkv import CompressionConfig, DraftKVEngine, FixedPolicy
    m, _, _ = tiny_setup
    prompts = [_prompt(10 + s, n, m.vocab_size) for s, n in enumerate((50, 64, 31))]
    single = [DraftKVEngine(m, seed=0).generate_baseline(p, 20, 0.0) for p in prompts]
    batch_base = DraftKVEngine(m, seed=0).generate_baseline_batch(prompts, 20, 0.0)
    assert batch_base == single
    res = DraftKVEngine(m, FixedPolicy(CompressionConfig(4, 0.5), 4), seed=0).generate_batch(prompts, 20, 0.0)
    assert [r.tokens for r in res] == single


class _Gamma:
    """A controller with no stated bound (no gamma / gamma_max attribute): one
    arm, gamma 20 every round."""

    def __init__(self, arm):
        self.arm = arm

    def select(self, ctx, key=None):
        return self.arm, 20

    def update(self, cfg, gamma, accepted, ctx, key=None):
        pass


@pytest.mark.parametrize("bounded", [True, False])
def test_batched_long_drafts_with_uneven_progress_fit_the_caches(dev, tiny_setup, bounded):
    """One gamma serves the batch and is capped only by the largest remaining
    budget, so with gamma 20 a sequence one token short of its budget still
    verifies 21 rows while another has many left: the caches are sized for
    that (the controller's bound, or the budget when it states none), and the
    output equals plain decoding of each prompt."""
    from draftkv import CompressionConfig, DraftKVEngine, FixedPolicy
    m, _, _ = tiny_setup
    prompts = [_prompt(40 + s, n, m.vocab_size) for s, n in enumerate((57, 23, 90, 41))]
    cfg = CompressionConfig(4, 0.5)
    single = [DraftKVEngine(m, seed=0).generate_baseline(p, 26, 0.0) for p in prompts]
    ctrl = FixedPolicy(cfg, 20) if bounded else _Gamma(cfg)
    res = DraftKVEngine(m, ctrl, seed=0).generate_batch(prompts, 26, 0.0)
    assert [r.tokens for r in res] == single
    # progress was uneven (the sequences accepted different runs), and long drafts ran
    assert len({tuple(x.accepted for x in r.rounds) for r in res}) > 1
    assert max(x.gamma for r in res for x in r.rounds) >= 18


def test_draft_longer_than_64_is_lossless(dev, tiny_setup):
    """FixedPolicy(cfg, 80), which the reference accepts: rounds draft up to
    80 tokens (the accept kernel decides any gamma) and the output equals
    plain decoding."""
    from draftkv import CompressionConfig, DraftKVEngine, FixedPolicy
    m, prompt, _ = tiny_setup
    base = DraftKVEngine(m, seed=0).generate_baseline(prompt, 100, 0.0)
    r = DraftKVEngine(m, FixedPolicy(CompressionConfig(8, 1.0), 80), seed=0).generate(prompt, 100, 0.0)
    assert r.tokens == base
    assert r.rounds[0].gamma == 80


class _Adaptive:
    """A test-local controller (the select/update protocol): cycles through the
    arms, lengthens the draft after a fully accepted round and shortens it
    (down to 0, a plain full-KV step) after a rejection."""

    def __init__(self, arms, gamma=2, gamma_max=9):
        self.arms, self.gamma, self.gamma_max, self.n = list(arms), gamma, gamma_max, 0

    def select(self, ctx, key=None):
        arm = self.arms[self.n % len(self.arms)]
        self.n += 1
        return arm, self.gamma

    def update(self, cfg, gamma, accepted, ctx, key=None):
        if gamma == 0:
            self.gamma = 1
        elif accepted == gamma:
            self.gamma = min(self.gamma_max, gamma + 2)
        else:
            self.gamma = max(0, accepted - 1)


def test_controller_driven_run_is_lossless(dev, tiny_setup):
    from draftkv import DraftKVEngine, default_arms
    m, prompt, base = tiny_setup
    ctrl = _Adaptive(default_arms())
    r = DraftKVEngine(m, ctrl, seed=0).generate(prompt, 32, 0.0)
    assert r.tokens == base
    assert r.verify_passes <= r.new_tokens
    assert len({x.cfg for x in r.rounds}) > 3 and len({x.gamma for x in r.rounds}) > 2


@pytest.mark.parametrize("attn_bias", [False, True])
def test_bf16_verify_block_equals_decode_rows(dev, attn_bias):
    """The bf16 forward (MFMA GEMMs with K chunks fixed by the shape, per-row
    norms, batch-invariant verify attention) is batch-invariant too: T rows
    in one pass == T one-row passes, bit for bit."""
    from draftkv.llama import LlamaLike, demo_llama_weights
    w, c = demo_llama_weights(attn_sharpness=1.0, attn_gain=1.0, attn_bias=attn_bias)
    g = LlamaLike(w, c, dtype=torch.bfloat16)
    toks = np.array(_prompt(6, 40, c["vocab_size"]))
    a, b = g.new_cache(), g.new_cache()
    g.forward(toks[:31], a, 0)
    g.forward(toks[:31], b, 0)
    block = g.forward(toks[31:], a, 31)
    rows = np.stack([g.forward(toks[31 + i: 32 + i], b, 31 + i)[0] for i in range(9)])
    assert np.array_equal(block.view(np.uint32), rows.view(np.uint32))


@pytest.mark.parametrize("attn_bias", [False, True])
def test_bf16_greedy_output_identical(dev, attn_bias):
    """Greedy losslessness with bf16 weights and a bf16 paged cache: the
    speculative output equals full-KV decoding token for token, for several
    drafter arms and gammas."""
    from draftkv import CompressionConfig, DraftKVEngine, FixedPolicy
    from draftkv.llama import LlamaLike, demo_llama_weights
    w, c = demo_llama_weights(attn_sharpness=1.0, attn_gain=1.0, attn_bias=attn_bias)
    g = LlamaLike(w, c, dtype=torch.bfloat16)
    prompt = _prompt(7, 150, c["vocab_size"])
    base = DraftKVEngine(g, seed=0).generate_baseline(prompt, 40, 0.0)
    for cfg, gamma in ((CompressionConfig(8, 1.0), 3), (CompressionConfig(4, 0.5, group=32, scale_fp16=True), 6),
                       (CompressionConfig(2, 0.25), 4)):
        r = DraftKVEngine(g, FixedPolicy(cfg, gamma), seed=0).generate(prompt, 40, 0.0)
        assert r.tokens == base, f"bf16 {cfg.label()} gamma={gamma} diverged from full-KV decoding"


def test_bf16_gpt2_tied_head_batch_invariant_and_lossless(dev):
    """A bf16 GPT-2 of distilgpt2's width whose head is the tied 50257-row
    embedding (gpt2.py:213): the library GEMM takes the head's last partial
    16-row fragment, verify rows equal one-token decode rows bit for bit, and
    greedy speculative output equals full-KV decoding."""
    from draftkv import CompressionConfig, DraftKVEngine, FixedPolicy, gpt2
    cfg = dict(gpt2.DISTILGPT2, n_layer=2)
    g = gpt2.GPT2.random(cfg, seed=0, std=0.05, dtype=torch.bfloat16)
    assert g.head is g.emb and g.head.shape[0] == 50257
    toks = np.array(_prompt(8, 40, 50257))
    a, b = g.new_cache(), g.new_cache()
    g.forward(toks[:31], a, 0)
    g.forward(toks[:31], b, 0)
    block = g.forward(toks[31:], a, 31)
    rows = np.stack([g.forward(toks[31 + i: 32 + i], b, 31 + i)[0] for i in range(9)])
    assert np.array_equal(block.view(np.uint32), rows.view(np.uint32))
    prompt = _prompt(9, 120, 50257)
    base = DraftKVEngine(g, seed=0).generate_baseline(prompt, 24, 0.0)
    for cfg_, gamma in ((CompressionConfig(8, 1.0), 4), (CompressionConfig(4, 0.5, group=32, scale_fp16=True), 6)):
        r = DraftKVEngine(g, FixedPolicy(cfg_, gamma), seed=0).generate(prompt, 24, 0.0)
        assert r.tokens == base, f"bf16 gpt2 {cfg_.label()} gamma={gamma}"


def test_bf16_llama_runs_and_is_self_consistent(dev):
    """bf16 weights + bf16 paged cache (the serving configuration): logits stay
    close to the float32 model and speculative decoding runs end to end."""
    from draftkv import CompressionConfig, DraftKVEngine, FixedPolicy
    from draftkv.llama import LlamaLike, demo_llama_weights
    w, c = demo_llama_weights(attn_sharpness=1.0, attn_gain=1.0)
    g16 = LlamaLike(w, c, dtype=torch.bfloat16)
    g32 = LlamaLike(w, c)
    toks = np.array(_prompt(5, 33, c["vocab_size"]))
    a = g16.forward(toks, g16.new_cache(), 0)
    b = g32.forward(toks, g32.new_cache(), 0)
    assert np.abs(a - b).max() < 0.05 * max(1.0, np.abs(b).max())
    r = DraftKVEngine(g16, FixedPolicy(CompressionConfig(4, 0.5, group=32, scale_fp16=True), 4),
                      seed=0).generate(list(toks), 16, 0.0)
    assert len(r.tokens) == 33 + 16 and r.new_tokens == 16
