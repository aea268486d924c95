"""Decode rounds of the full Llama-3-8B shape (32 layers, d_model 4096, 32/8
GQA heads, head_dim 128, SwiGLU 14336, vocab 128256, bf16 random weights
N(0, 0.02)) over a synthetic full cache written straight into shuffled
16-token pages, at the two context shapes of the benchmark:

* batch 32 at 32768 positions, arms int8 group-64 keep 1 and int4 group-32
  keep 0.25 (fp16 meta) switched every 2 rounds (each switch requantizes
  all 32 layers);
* batch 1 at 262144 positions (a 34 GB full cache), int4 group-32 keep 0.25
  with gamma 16, then int8 keep 1.

No oracle runs a model of this size; the checks are the properties the
reference's own tests use: greedy speculative output equals plain full-KV
decoding on the same cache (tests/test_lossless.py:28-35), across the arm
switch, and temperature-0.8 (batch 32) and temperature-1.0 (batch 1) runs
decode valid tokens with accepted runs within gamma.
"""

import gc

import numpy as np
import pytest
import torch

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


@pytest.fixture(autouse=True)
def _free():
    gc.collect()
    torch.cuda.empty_cache()
    yield
    gc.collect()
    torch.cuda.empty_cache()


@pytest.fixture(scope="module")
def model(dev):
    from draftkv.llama import LLAMA3_8B, LlamaLike
    m = LlamaLike.random(LLAMA3_8B, seed=0, std=0.02, dtype=torch.bfloat16)
    yield m
    del m
    gc.collect()
    torch.cuda.empty_cache()


def _synthetic_cache(model, batch, ctx, extra, seed):
    """ctx-1 rows of N(0,1) bf16 K/V per sequence and layer in 16-token pages
    from shuffled free lists (the prefill of a ctx-token prompt, without
    running it)."""
    from draftkv import PagedKVCache
    L, H, D = model.n_layers, model.n_kv_heads, model.d_head
    max_tokens = ctx + extra
    full = PagedKVCache(L, H, D, block_size=16, n_blocks=L * -(-max_tokens // 16), dtype="bf16", batch=batch,
                        max_tokens=max_tokens, device=model.device)
    rng = np.random.default_rng(seed)
    for p in full.pools:
        rng.shuffle(p._stack)
    full.reserve([ctx - 1] * batch)
    g = torch.Generator(device=model.device)
    g.manual_seed(seed)
    step = max(1, (1 << 30) // (full.store.shape[1] * 2))
    for i in range(0, full.store.shape[0], step):
        blk = full.store[i: i + step]
        blk.copy_(torch.randn(blk.shape, generator=g, device=model.device, dtype=torch.float32))
    full.commit([ctx - 1] * batch)
    return full


def _greedy_full_kv(model, full, toks, n_new):
    """Plain decoding on the full cache from each sequence's pending token."""
    from draftkv import ops
    b = len(toks)
    start = np.array([len(t) - 1 for t in toks], np.int64)
    x = torch.as_tensor(np.array([t[-1] for t in toks], np.int32)).to(model.device)
    u = torch.zeros((n_new, b), dtype=torch.float64, device=model.device)
    out = []
    for i in range(n_new):
        lg = model.forward_batch(x[:, None], full, start + i)[:, 0]
        x = ops.sample(lg, 0.0, u[i])
        out.append(x)
    return torch.stack(out, 1).cpu().numpy()


def _speculative(model, full, toks, ctrl, n_new, T, reserve, seed=0):
    from draftkv import DraftKVEngine
    from draftkv.engine import DecodeBatch
    eng = DraftKVEngine(model, ctrl, seed=seed)
    batch = DecodeBatch(eng, [list(t) for t in toks], full, n_new, T, reserve_cfgs=reserve)
    while batch.step():
        pass
    res = batch.results()
    del batch
    return res


@pytest.mark.timeout(900)
def test_b32_ctx32k_greedy_lossless_across_arm_switches(dev, model):
    from draftkv import CompressionConfig
    b, ctx, n_new = 32, 32768, 16
    full = _synthetic_cache(model, b, ctx, 64, seed=1)
    rng = np.random.default_rng(0)
    toks = [[int(x) for x in rng.integers(0, model.vocab_size, ctx)] for _ in range(b)]
    arms = [CompressionConfig(8, 1.0, group=64, scale_fp16=True),
            CompressionConfig(4, 0.25, group=32, scale_fp16=True)]
    res = _speculative(model, full, toks, Switch(arms, 3, 2), n_new, 0.0, arms)
    assert {x.cfg for x in res[0].rounds} == set(arms)
    assert res[0].cache_rebuilds >= 2
    spec = np.array([r.tokens[ctx:] for r in res])
    assert spec.shape == (b, n_new)
    full.truncate(ctx - 1)
    base = _greedy_full_kv(model, full, toks, n_new)
    assert np.array_equal(spec, base)
    # temperature 0.8 rejection sampling (the benchmark's operating point),
    # longer drafts, both arms: every sequence decodes in-vocabulary tokens
    # with accepted runs within gamma, from its own random stream
    full.truncate(ctx - 1)
    res = _speculative(model, full, toks, Switch(arms, 8, 2), 24, 0.8, arms, seed=11)
    for r in res:
        assert len(r.tokens) == ctx + 24
        assert all(0 <= t < model.vocab_size for t in r.tokens[ctx:])
        assert all(0 <= x.accepted <= x.gamma and x.emitted == x.accepted + 1 for x in r.rounds)
        assert sum(x.emitted for x in r.rounds) >= 24
    assert {x.cfg for x in res[0].rounds} == set(arms)
    assert len({tuple(r.tokens[ctx:]) for r in res}) == b     # every sequence its own stream
    del full
    gc.collect()
    torch.cuda.empty_cache()


@pytest.mark.timeout(900)
def test_b1_ctx262k_lossless_and_sampled_rounds(dev, model):
    from draftkv import CompressionConfig
    b, ctx = 1, 262144
    full = _synthetic_cache(model, b, ctx, 128, seed=2)
    toks = [[int(x) for x in np.random.default_rng(5).integers(0, model.vocab_size, ctx)]]
    arms = [CompressionConfig(4, 0.25, group=32, scale_fp16=True),
            CompressionConfig(8, 1.0, group=64, scale_fp16=True)]
    n_new = 40
    res = _speculative(model, full, toks, Switch(arms, 16, 2), n_new, 0.0, arms)
    assert {x.cfg for x in res[0].rounds} == set(arms)
    spec = np.array([res[0].tokens[ctx:]])
    full.truncate(ctx - 1)
    base = _greedy_full_kv(model, full, toks, n_new)
    assert np.array_equal(spec, base)
    # temperature 1.0 rejection sampling over the 128256-token vocabulary
    full.truncate(ctx - 1)
    res = _speculative(model, full, toks, Switch(arms, 16, 2), 24, 1.0, arms, seed=3)
    r = res[0]
    assert len(r.tokens) == ctx + 24
    assert all(0 <= t < model.vocab_size for t in r.tokens[ctx:])
    assert all(0 <= x.accepted <= x.gamma and x.emitted == x.accepted + 1 for x in r.rounds)
    assert sum(x.emitted for x in r.rounds) >= 24
    del full
    gc.collect()
    torch.cuda.empty_cache()
