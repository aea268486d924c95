"""Pins the oracle's attention, models, sampling and engine loop against the
reference's own test expectations (tests/test_lossless.py, tests/test_llama.py,
tests/test_sampling.py) and against the mathematics (textbook softmax by
brute force, RoPE invariants, numpy's Generator.choice)."""

import math

import numpy as np
import pytest

from oracle.attention import attend
from oracle.caches import FullKVCache, PagedKVCache
from oracle.config import Cfg
from oracle.engine import Engine, fixed
from oracle.models import GPT2, demo_llama, demo_model, gpt2_random_weights, rotate_half
from oracle.sampling import accept, probs, sample_u


def test_attention_matches_scalar_softmax():
    rng = np.random.default_rng(0)
    T, H, KV, D, Tk = 3, 4, 2, 8, 7
    q = rng.standard_normal((T, H, D)).astype(np.float32)
    k = rng.standard_normal((Tk, KV, D)).astype(np.float32)
    v = rng.standard_normal((Tk, KV, D)).astype(np.float32)
    cpos, pos = np.arange(Tk), np.array([4, 5, 6])
    out, p, mp = attend(q, k, v, cpos, pos, n_rep=2)
    for t in range(T):
        for h in range(H):
            kv = h // 2
            s = [sum(float(q[t, h, d]) * float(k[j, kv, d]) for d in range(D)) / math.sqrt(D)
                 for j in range(Tk)]
            valid = [j for j in range(Tk) if cpos[j] <= pos[t]]
            mx = max(s[j] for j in valid)
            e = {j: math.exp(s[j] - mx) for j in valid}
            z = sum(e.values())
            for j in range(Tk):
                assert p[t, h, j] == pytest.approx(e.get(j, 0.0) / z, rel=1e-6, abs=1e-7)
            o = [sum(e[j] / z * float(v[j, kv, d]) for j in valid) for d in range(D)]
            assert np.allclose(out[t, h], o, rtol=1e-5, atol=1e-6)
    assert np.allclose(mp, p.reshape(T, KV, 2, Tk).sum(2))


def test_rope_norm_and_relative_position():            # reference test_llama.py:25-50
    m = demo_llama()
    cos, sin = m.rope(np.arange(8))
    x = np.random.default_rng(0).standard_normal((8, 2, m.d_head)).astype(np.float32)
    y = x * cos[:, None, :] + rotate_half(x) * sin[:, None, :]
    assert np.allclose(np.linalg.norm(x, axis=-1), np.linalg.norm(y, axis=-1), atol=1e-4)
    rng = np.random.default_rng(1)
    q, k = rng.standard_normal(m.d_head), rng.standard_normal(m.d_head)

    def score(i, j):
        c, s = m.rope(np.array([i, j]))
        return float((q * c[0] + rotate_half(q) * s[0]) @ (k * c[1] + rotate_half(k) * s[1]))

    for delta in (1, 3, 7):
        vals = [score(p, p + delta) for p in (0, 5, 11, 40)]
        assert np.allclose(vals, vals[0], atol=1e-3)


def test_choice_is_searchsorted_of_one_uniform():
    """numpy's own Generator.choice(p=...) is one random() draw searched in
    the normalised cumulative sum -- what sample_u restates."""
    for seed in range(50):
        p = np.random.default_rng(seed + 99).random(37)
        p[seed % 37] = 0.0
        p /= p.sum()
        a, b = np.random.default_rng(seed), np.random.default_rng(seed)
        assert a.choice(37, p=p) == sample_u(p, b.random())
        assert a.random() == b.random()                 # exactly one draw consumed
    one_hot = np.zeros(9)
    one_hot[4] = 1.0
    assert all(sample_u(one_hot, u) == 4 for u in (0.0, 0.3, 0.999999))


def test_accept_greedy_cases():
    V = 6
    tl = np.zeros((4, V), np.float32)
    tl[0, 2] = tl[1, 3] = tl[2, 1] = tl[3, 5] = 1.0
    assert accept(tl, [2, 3, 1], None, 0.0, [0.5]) == (3, 5, 1)       # all accepted: bonus
    assert accept(tl, [2, 0, 1], None, 0.0, []) == (1, 3, 0)          # first miss at 1


def test_accept_sampling_ratio_and_residual():
    V = 4
    tl = np.log(np.array([[0.1, 0.2, 0.3, 0.4], [0.25, 0.25, 0.25, 0.25]], np.float32))
    q = np.array([0.7, 0.1, 0.1, 0.1])
    # p[0]/q[0] = 0.1/0.7: u below it accepts, above rejects
    acc, nxt, used = accept(tl, [0], [q], 1.0, [0.1, 0.0])
    assert (acc, used) == (1, 2)
    acc, nxt, used = accept(tl, [0], [q], 1.0, [0.2, 0.0])
    assert acc == 0 and used == 2
    # residual clip(p - q) = [0, .1, .2, .3] normalised: u=0 -> first positive index
    assert nxt == 1
    assert accept(tl, [0], [q], 1.0, [0.2, 0.99])[1] == 3


@pytest.fixture(scope="module")
def tiny():
    m = demo_model()
    prompt = [int(x) for x in np.random.default_rng(0).integers(0, m.vocab_size, 192)]
    base = Engine(m, fixed(Cfg(16, 1.0), 1)).generate_baseline(prompt, 32, 0.0)
    return m, prompt, base


@pytest.mark.parametrize("cfg", [Cfg(16, 1.0), Cfg(8, 1.0), Cfg(4, 0.5), Cfg(2, 0.25)],
                         ids=lambda c: f"{c.bits}b{c.keep_frac}")
@pytest.mark.parametrize("gamma", [1, 3, 6])
def test_greedy_lossless(tiny, cfg, gamma):             # reference test_lossless.py:28-35
    m, prompt, base = tiny
    assert Engine(m, fixed(cfg, gamma)).generate(prompt, 32, 0.0).tokens == base


def test_compression_costs_acceptance(tiny):            # reference test_lossless.py:38-46
    m, prompt, _ = tiny
    mild = Engine(m, fixed(Cfg(16, 1.0), 6)).generate(prompt, 32, 0.0)
    harsh = Engine(m, fixed(Cfg(2, 0.25), 6)).generate(prompt, 32, 0.0)
    assert mild.acceptance_rate > harsh.acceptance_rate + 0.2


def test_paged_lossless(tiny):                          # reference test_paged.py:103-116
    m, prompt, base = tiny
    for bs in (4, 16):
        e = Engine(m, fixed(Cfg(4, 0.5), 5),
                   full_cache_factory=lambda bs=bs: PagedKVCache(m.n_layers, m.n_heads, m.d_head, bs, 2048))
        assert e.generate(prompt, 32, 0.0).tokens == base


@pytest.mark.parametrize("n_kv", [8, 4, 1])
def test_llama_gqa_lossless(n_kv):                      # reference test_llama.py:66-74
    m = demo_llama(n_heads=8, n_kv_heads=n_kv, seed=2)
    prompt = [int(x) for x in np.random.default_rng(0).integers(0, m.vocab_size, 96)]
    base = Engine(m, fixed(Cfg(16, 1.0), 1)).generate_baseline(prompt, 20, 0.0)
    for cfg in (Cfg(8, 1.0), Cfg(4, 0.5), Cfg(2, 0.25)):
        assert Engine(m, fixed(cfg, 4)).generate(prompt, 20, 0.0).tokens == base


def test_llama_bias_path_and_kv_heads():                # reference test_llama.py:54-63,90-94
    m = demo_llama(attn_bias=True)
    out = m.forward(np.arange(8) % m.vocab_size, FullKVCache(m.n_layers), 0)
    assert out.shape == (8, m.vocab_size) and np.isfinite(out).all()
    m = demo_llama(n_heads=8, n_kv_heads=2)
    c = FullKVCache(m.n_layers)
    m.forward(np.arange(32) % m.vocab_size, c, 0)
    assert c.read(0)[0].shape == (32, 2, m.d_head)


def test_gpt2_random_model_runs_lossless():
    cfg = dict(n_layer=2, n_embd=32, n_head=4, vocab_size=97, n_positions=256)
    m = GPT2(gpt2_random_weights(cfg, seed=0), cfg)
    prompt = list(np.random.default_rng(1).integers(0, 97, 40))
    base = Engine(m, fixed(Cfg(16, 1.0), 1)).generate_baseline(prompt, 12, 0.0)
    assert Engine(m, fixed(Cfg(8, 1.0), 4)).generate(prompt, 12, 0.0).tokens == base


def test_first_token_distribution_under_sampling():     # reference test_sampling.py:19-42
    m = demo_model()
    prompt = [int(x) for x in np.random.default_rng(0).integers(0, m.vocab_size, 48)]
    cache = FullKVCache(m.n_layers)
    m.forward(np.array(prompt[:-1]), cache, 0)
    p = probs(m.forward(np.array([prompt[-1]]), cache, len(prompt) - 1)[-1], 1.0)
    trials = 600
    e = Engine(m, fixed(Cfg(2, 0.25), 4), seed=1)
    counts = np.zeros(m.vocab_size)
    for _ in range(trials):
        counts[e.generate(prompt, 1, 1.0).tokens[len(prompt)]] += 1
    ctrl = np.bincount(np.random.default_rng(2).choice(m.vocab_size, size=trials, p=p),
                       minlength=m.vocab_size) / trials
    tv = lambda a: 0.5 * float(np.abs(a - p).sum())
    assert tv(counts / trials) < max(1.5 * tv(ctrl), 0.05)
