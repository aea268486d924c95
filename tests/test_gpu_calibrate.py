"""Cost-model calibration on a live decode (HIP events around the phases of
real rounds), and decode rounds with gamma 0 (the controller declining to
draft): greedy output stays identical to full-KV decoding either way."""

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu


def _setup(b=3, seed=5):
    from draftkv import CompressionConfig, CostModel, DraftKVEngine
    from draftkv.engine import DecodeBatch
    from draftkv.llama import demo_llama
    m = demo_llama()
    rng = np.random.default_rng(seed)
    prompts = [[int(x) for x in rng.integers(0, m.vocab_size, n)] for n in (90, 64, 120)[:b]]
    arms = [CompressionConfig(8, 1.0), CompressionConfig(4, 0.25, group=32, scale_fp16=True)]
    return m, prompts, arms, CostModel, DraftKVEngine, DecodeBatch


def test_calibration_fits_the_measured_phases(dev):
    from draftkv.calibrate import PhaseLog, calibrate, fit_from_log
    from draftkv.controller import FixedPolicy
    m, prompts, arms, CostModel, DraftKVEngine, DecodeBatch = _setup()
    eng = DraftKVEngine(m, FixedPolicy(arms[0], 2), seed=0)
    toks = eng._check_prompts(prompts, m.vocab_size)
    full = eng._new_full(len(toks), max(len(t) for t in toks) + 200)
    eng._prefill(toks, full)
    batch = DecodeBatch(eng, toks, full, 150, 0.0, reserve_cfgs=arms)
    batch.step()
    base = CostModel(n_layers=m.n_layers, n_kv_heads=m.n_kv_heads, d_head=m.d_head, batch=len(toks),
                     weight_bytes=1e6, bandwidth=8e12)
    saved = eng.controller
    fit = calibrate(batch, base, arms, gammas=(1, 3), reps=2)
    assert eng.controller is saved and batch.phases is None
    for f in ("bandwidth", "full_kv_bandwidth", "fixed_draft", "fixed_verify", "resync_per_token",
              "controller_overhead"):
        v = getattr(fit, f)
        assert np.isfinite(v) and v >= 0.0, f
    assert fit.bandwidth > 0 and fit.full_kv_bandwidth > 0
    # a fresh log of a few more rounds under one arm: every phase is recorded
    log = PhaseLog()
    batch.phases = log
    for _ in range(3):
        batch.step()
    batch.phases = None
    f2 = fit_from_log(base, int(max(len(t) for t in batch.toks)), log)
    assert sum(len(v) for v in log.draft.values()) == 3 and len(log.resync) == 3 and len(log.host) == 3
    assert all(t > 0 for v in log.draft.values() for t in v)
    assert f2.t_draft(arms[0], 100) > 0


class _Decline:
    """Drafts (gamma 3) on odd rounds, declines (gamma 0) on even ones."""

    def __init__(self, arm):
        self.arm, self.n, self.arms = arm, 0, [arm]

    def select(self, ctx, key=None):
        self.n += 1
        return self.arm, (3 if self.n % 2 else 0)

    def update(self, cfg, gamma, accepted, ctx, key=None):
        pass


def test_declined_rounds_keep_greedy_output_identical(dev):
    from draftkv import DraftKVEngine
    m, prompts, arms, *_ = _setup()
    base = DraftKVEngine(m, seed=0).generate_baseline(prompts[0], 30, 0.0)
    r = DraftKVEngine(m, _Decline(arms[1]), seed=0).generate(prompts[0], 30, 0.0)
    assert r.tokens == base
    assert any(x.gamma == 0 for x in r.rounds) and any(x.gamma > 0 for x in r.rounds)


class _AlwaysDecline(_Decline):
    def select(self, ctx, key=None):
        return self.arm, 0


def test_consecutive_declined_rounds_resolve_their_tokens(dev):
    # every round declines: each one's token stays on the device until the
    # batch resolves it; the streams equal plain full-KV decoding
    from draftkv import DraftKVEngine
    from draftkv.engine import DecodeBatch
    m, prompts, arms, *_ = _setup()
    base = [DraftKVEngine(m, seed=0).generate_baseline(p, 12, 0.0) for p in prompts]
    eng = DraftKVEngine(m, _AlwaysDecline(arms[0]), seed=0)
    toks = eng._check_prompts(prompts, m.vocab_size)
    full = eng._new_full(len(toks), max(len(t) for t in toks) + 32)
    eng._prefill(toks, full)
    batch = DecodeBatch(eng, toks, full, 12, 0.0)
    for _ in range(5):
        assert batch.step()
    batch.resolve_tokens()
    assert all(-1 not in t for t in batch.toks)
    assert [t[: len(p) + 5] for t, p in zip(batch.toks, prompts)] == [b[: len(p) + 5] for b, p in zip(base, prompts)]
    while batch.step():
        pass
    assert [r.tokens for r in batch.results()] == base
    assert all(x.gamma == 0 for r in batch.res for x in r.rounds)
