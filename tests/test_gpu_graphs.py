"""Draft steps replayed from recorded HIP graphs against the same steps run
eagerly.

Two decodes of the same batch with the same seeds, one with draft-step
graphs and one without. In every round the replayed steps' draft logits and
draft tokens must equal the eager ones bit for bit (the same kernels on the
same inputs), with the round's eager verify, accept, rollback and mirror
resync (and host synchronisations) running between replays; the decoded
tokens and accepted runs must match as well. The cases cover RoPE and
learned-position models, float32 and bf16 weights, eviction (keep < 1), arm
switches (a graph recorded per mirror layout), ragged batches whose
sequences finish in different rounds, and greedy and temperature sampling.
"""

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu


class Alternate:
    """Arms switched every ``period`` rounds, fixed gamma (controller protocol)."""

    def __init__(self, arms, gamma, period=2):
        self.arms, self.gamma, self.period, self.n = list(arms), gamma, period, 0

    def select(self, ctx, key=None):
        arm = self.arms[(self.n // self.period) % len(self.arms)]
        self.n += 1
        return arm, self.gamma

    def update(self, cfg, gamma, accepted, ctx, key=None):
        pass


def _model(name):
    from draftkv import gpt2, llama, model
    if name == "tiny":
        return model.demo_model()
    if name == "llama":
        return llama.demo_llama()
    if name == "llama_bf16":
        w, c = llama.demo_llama_weights(attn_sharpness=1.0, attn_gain=1.0)
        return llama.LlamaLike(w, c, dtype=torch.bfloat16)
    if name == "gpt2":
        import oracle.models as om
        cfg = dict(n_layer=2, n_head=4, n_embd=64, vocab_size=97, n_positions=512, n_inner=None,
                   layer_norm_epsilon=1e-5)
        return gpt2.GPT2(om.gpt2_random_weights(cfg, seed=0, std=0.2), cfg)
    raise KeyError(name)


def _decode(m, prompts, max_new, T, arms, gamma, graphs):
    from draftkv import DraftKVEngine
    from draftkv.engine import DecodeBatch
    eng = DraftKVEngine(m, Alternate(arms, gamma), seed=3)
    eng.draft_graphs = graphs
    toks = eng._check_prompts(prompts, m.vocab_size)
    full = eng._new_full(len(toks), max(len(t) for t in toks) + max_new + 16)
    eng._prefill(toks, full)
    batch = DecodeBatch(eng, toks, full, max_new, T)
    rounds = []
    while batch.step():
        d = batch.last_draft
        if d is None:
            rounds.append(None)
            continue
        rounds.append((d[0].cpu().numpy(), None if d[1] is None else d[1].cpu().numpy()))
    return batch.results(), rounds, batch


CASES = [("tiny", 0.0, 5), ("llama", 0.0, 4), ("llama", 0.8, 6), ("llama_bf16", 0.7, 4), ("gpt2", 0.9, 3)]


@pytest.mark.parametrize("name,T,gamma", CASES)
def test_graph_replays_equal_eager_steps(dev, name, T, gamma):
    from draftkv import CompressionConfig
    m = _model(name)
    rng = np.random.default_rng(11)
    prompts = [[int(x) for x in rng.integers(0, m.vocab_size, n)] for n in (70, 45, 96)]
    arms = [CompressionConfig(4, 0.5, group=32, scale_fp16=True), CompressionConfig(8, 1.0),
            CompressionConfig(2, 0.25)]
    res_g, rounds_g, bg = _decode(m, prompts, 40, T, arms, gamma, graphs=True)
    res_e, rounds_e, be = _decode(m, prompts, 40, T, arms, gamma, graphs=False)
    assert bg.use_graphs and not be.use_graphs
    replays = sum(g.replays for g in bg._graphs.values())
    assert len(bg._graphs) >= 2 and replays >= len(rounds_g), "the graph path did not run"
    assert len(rounds_g) == len(rounds_e)
    for i, (rg, re_) in enumerate(zip(rounds_g, rounds_e)):
        assert (rg is None) == (re_ is None)
        if rg is None:
            continue
        np.testing.assert_array_equal(rg[0], re_[0], err_msg=f"round {i}: draft tokens")
        if re_[1] is not None:
            assert np.array_equal(rg[1], re_[1]), f"round {i}: draft logits differ"
    for a, b in zip(res_g, res_e):
        assert a.tokens == b.tokens
        assert [x.accepted for x in a.rounds] == [x.accepted for x in b.rounds]
    # the live mirror rows agree too
    np.testing.assert_array_equal(bg.comp.rows(), be.comp.rows())


def test_graph_is_rerecorded_when_the_rope_table_grows(dev):
    """Decoding past 4096 positions regrows the RoPE table (a buffer the graph
    reads): the next round records a new graph, and decoding stays identical
    to eager."""
    from draftkv import CompressionConfig
    m = _model("llama")
    rng = np.random.default_rng(5)
    prompts = [[int(x) for x in rng.integers(0, m.vocab_size, 4000)]]
    arms = [CompressionConfig(8, 1.0)]
    res_g, rounds_g, bg = _decode(m, prompts, 200, 0.0, arms, 6, graphs=True)
    res_e, rounds_e, _ = _decode(m, prompts, 200, 0.0, arms, 6, graphs=False)
    assert res_g[0].tokens == res_e[0].tokens
    for rg, re_ in zip(rounds_g, rounds_e):
        if rg is not None:
            np.testing.assert_array_equal(rg[0], re_[0])
    assert len(bg._graphs) >= 2 and sum(g.replays for g in bg._graphs.values()) > 0


class Pattern:
    """One arm, gamma from a repeating pattern (0 = a plain full-KV step)."""

    def __init__(self, arm, gammas):
        self.arm, self.gammas, self.n = arm, list(gammas), 0

    def select(self, ctx, key=None):
        g = self.gammas[self.n % len(self.gammas)]
        self.n += 1
        return self.arm, g

    def update(self, cfg, gamma, accepted, ctx, key=None):
        pass


def _decode_pattern(m, prompts, max_new, T, arm, gammas, graphs):
    from draftkv import DraftKVEngine
    from draftkv.engine import DecodeBatch
    eng = DraftKVEngine(m, Pattern(arm, gammas), seed=4)
    eng.draft_graphs = graphs
    toks = eng._check_prompts(prompts, m.vocab_size)
    full = eng._new_full(len(toks), max(len(t) for t in toks) + max_new + 16)
    eng._prefill(toks, full)
    batch = DecodeBatch(eng, toks, full, max_new, T)
    while batch.step():
        pass
    return batch.results(), batch


@pytest.mark.parametrize("name,T", [("llama", 0.0), ("llama_bf16", 0.8), ("gpt2", 0.0), ("tiny", 0.9)])
def test_gamma0_graph_replays_equal_eager_rounds(dev, name, T):
    """Rounds that decline to draft (gamma 0) replayed from a recorded full-KV
    step graph: the tokens, accepted runs and mirror rows equal an eager
    decode's, over a ragged batch whose sequences finish in different rounds
    (inactive rows in the replayed step) with drafted rounds in between."""
    from draftkv import CompressionConfig
    from draftkv.graphs import FullStepGraph
    m = _model(name)
    rng = np.random.default_rng(12)
    prompts = [[int(x) for x in rng.integers(0, m.vocab_size, n)] for n in (60, 33, 81)]
    arm = CompressionConfig(4, 0.5, group=32, scale_fp16=True)
    gammas = [0, 0, 3, 0, 0, 0, 2]
    budgets = 37
    res_g, bg = _decode_pattern(m, prompts, budgets, T, arm, gammas, graphs=True)
    res_e, be = _decode_pattern(m, prompts, budgets, T, arm, gammas, graphs=False)
    full_graphs = [g for g in bg._graphs.values() if isinstance(g, FullStepGraph)]
    assert full_graphs and sum(g.replays for g in full_graphs) >= 10, "the gamma-0 graph did not run"
    for a, b in zip(res_g, res_e):
        assert a.tokens == b.tokens
        assert [x.accepted for x in a.rounds] == [x.accepted for x in b.rounds]
        assert [x.gamma for x in a.rounds] == [x.gamma for x in b.rounds]
    np.testing.assert_array_equal(bg.comp.rows(), be.comp.rows())
    np.testing.assert_array_equal(bg.full.lengths(), be.full.lengths())
