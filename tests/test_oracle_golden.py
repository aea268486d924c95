"""The oracle against vectors recorded from the reference implementation
(tests/golden/make_golden.py). Everything here is exact equality: the oracle
restates the reference's numpy operations, so it must reproduce them bit for
bit -- logits (float64 promotion included), steady-state eviction sets and
scores, accepted-run lengths and temperature-mode tokens."""

import os

import numpy as np
import pytest

from oracle.caches import CompressedKVCache, FullKVCache
from oracle.config import Cfg
from oracle.engine import Engine, fixed
from oracle.models import GPT2, demo_llama, demo_model
from oracle.quant import quantize

G = np.load(os.path.join(os.path.dirname(__file__), "golden", "reference_vectors.npz"))


@pytest.mark.parametrize("i", range(4))
def test_quantize(i):
    x, bits = G[f"quant{i}_x"], int(G[f"quant{i}_bits"])
    assert np.array_equal(quantize(x, bits), G[f"quant{i}_deq"])


def test_forward_logits_exact():
    m = demo_model()
    assert np.array_equal(m.forward(G["tiny_tokens"], FullKVCache(m.n_layers), 0), G["tiny_logits"])
    ml = demo_llama(n_heads=8, n_kv_heads=2, attn_bias=True, seed=3)
    assert np.array_equal(ml.forward(G["llama_tokens"], FullKVCache(ml.n_layers), 0), G["llama_logits"])
    w = {k[len("gpt2w_"):]: G[k] for k in G.files if k.startswith("gpt2w_")}
    g = GPT2(w, dict(n_layer=2, n_embd=32, n_head=4, vocab_size=97, n_positions=256))
    assert np.array_equal(g.forward(G["gpt2_tokens"], FullKVCache(2), 0), G["gpt2_logits"])


@pytest.mark.parametrize("j", range(3))
def test_greedy_runs(j):
    bits, keep, gamma = G[f"greedy{j}_cfg"]
    m = demo_model()
    r = Engine(m, fixed(Cfg(int(bits), float(keep)), int(gamma))).generate(list(G["run_prompt"]), 32, 0.0)
    assert r.tokens == G[f"greedy{j}_tokens"].tolist()
    assert [x.accepted for x in r.rounds] == G[f"greedy{j}_accepted"].tolist()


def test_mirror_after_drafting():
    m = demo_model()
    prompt = G["run_prompt"].tolist()
    full = FullKVCache(m.n_layers)
    m.forward(np.array(prompt[:-1]), full, 0)
    comp = CompressedKVCache(m.n_layers, Cfg(4, 0.25))
    comp.sync_from(full, 0)
    x, n, drafted = prompt[-1], len(prompt), []
    for i in range(8):
        x = int(np.argmax(m.forward(np.array([x]), comp, n - 1 + i)[-1]))
        drafted.append(x)
    assert drafted == G["mirror_drafts"].tolist()
    for L in range(m.n_layers):
        assert comp.pos[L].tolist() == G[f"mirror_pos{L}"].tolist()
        assert np.array_equal(comp.score[L], G[f"mirror_score{L}"])


@pytest.mark.parametrize("j", range(2))
def test_temperature_runs(j):
    bits, keep, gamma, seed = G[f"temp{j}_cfg"]
    m = demo_model()
    r = Engine(m, fixed(Cfg(int(bits), float(keep)), int(gamma)), seed=int(seed)).generate(
        list(G["temp_prompt"]), 24, 1.0)
    assert r.tokens == G[f"temp{j}_tokens"].tolist()
    assert [x.accepted for x in r.rounds] == G[f"temp{j}_accepted"].tolist()
