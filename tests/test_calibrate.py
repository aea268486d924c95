"""Cost-model calibration: the fit of CostModel's time parameters to
measured draft, verify and full-KV step times.

The fit is pinned by construction: times generated from a known CostModel
(the reference's formulas, throughput.py:110-155) must give back that
model's parameters, and the fitted model must reproduce the times it was
fitted to. The partial cases (one arm, no full-KV step, a full cache that
streams faster than the draft fit can resolve) keep the terms the data do
not determine.
"""

import dataclasses

import numpy as np
import pytest

from draftkv import CompressionConfig, CostModel
from draftkv.calibrate import FixedRounds, PhaseLog, fit_cost_model

ARMS = [CompressionConfig(8, 1.0, group=64, scale_fp16=True), CompressionConfig(4, 0.25, group=32, scale_fp16=True),
        CompressionConfig(2, 0.5, group=32)]


def _truth(**kw):
    base = dict(n_layers=32, n_kv_heads=8, d_head=128, weight_bytes=16.06e9, batch=32, bandwidth=4.4e12,
                full_kv_bandwidth=5.8e12, compute_per_token=35e-6, fixed_draft=420e-6, fixed_verify=420e-6,
                resync_per_token=3e-6, controller_overhead=150e-6)
    base.update(kw)
    return CostModel(**base)


def _times(m, ctx, arms, gammas):
    return ({a: m.t_draft(a, ctx) for a in arms}, {g: m.t_verify(ctx, g) for g in gammas}, m.t_baseline(ctx))


FIELDS = ("bandwidth", "full_kv_bandwidth", "compute_per_token", "fixed_draft", "fixed_verify")


@pytest.mark.parametrize("ctx", [4096, 32768, 262144])
@pytest.mark.parametrize("narms", [2, 3])
def test_fit_recovers_a_known_model(ctx, narms):
    truth = _truth(batch=1 if ctx == 262144 else 32)
    draft, verify, t_base = _times(truth, ctx, ARMS[:narms], (1, 4, 8))
    start = CostModel(n_layers=32, n_kv_heads=8, d_head=128, weight_bytes=truth.weight_bytes, batch=truth.batch,
                      bandwidth=8e12)
    fit = fit_cost_model(start, ctx, draft, verify, t_base, resync_per_token=3e-6, controller_overhead=150e-6)
    for f in FIELDS:
        assert getattr(fit, f) == pytest.approx(getattr(truth, f), rel=1e-6), f
    # the fitted model reproduces every time it was fitted to, and its ceiling
    for a in ARMS[:narms]:
        assert fit.t_draft(a, ctx) == pytest.approx(draft[a], rel=1e-9)
        assert fit.ceiling(a, ctx) == pytest.approx(truth.ceiling(a, ctx), rel=1e-6)
    for g, t in verify.items():
        assert fit.t_verify(ctx, g) == pytest.approx(t, rel=1e-9)
    assert fit.t_baseline(ctx) == pytest.approx(t_base, rel=1e-9)
    # shape, bytes and batch are the start model's
    for f in ("n_layers", "n_kv_heads", "d_head", "weight_bytes", "batch"):
        assert getattr(fit, f) == getattr(start, f)


def test_one_arm_keeps_the_bandwidth_and_absorbs_the_rest():
    truth = _truth()
    ctx = 32768
    draft, verify, t_base = _times(truth, ctx, ARMS[1:2], (2,))
    start = dataclasses.replace(truth, bandwidth=8e12, full_kv_bandwidth=None, fixed_draft=0.0, fixed_verify=0.0)
    start.__post_init__()
    fit = fit_cost_model(start, ctx, draft, verify, t_base)
    assert fit.bandwidth == 8e12
    assert fit.t_draft(ARMS[1], ctx) == pytest.approx(draft[ARMS[1]], rel=1e-9)
    assert fit.t_verify(ctx, 2) == pytest.approx(verify[2], rel=1e-9)
    assert fit.t_baseline(ctx) == pytest.approx(t_base, rel=1e-9)


def test_without_a_full_kv_step_the_full_cache_terms_stay():
    truth = _truth()
    ctx = 32768
    draft, verify, _ = _times(truth, ctx, ARMS[:2], (1, 4))
    start = _truth(full_kv_bandwidth=7e12, compute_per_token=1e-6, fixed_verify=9e-6)
    fit = fit_cost_model(start, ctx, draft, verify)
    assert fit.full_kv_bandwidth == 7e12 and fit.compute_per_token == 1e-6
    assert fit.bandwidth == pytest.approx(truth.bandwidth, rel=1e-6)


def test_fast_full_cache_goes_to_the_fixed_term():
    # a full-KV step so short that the full cache would need a negative time:
    # the fit keeps the start model's full-cache rate and the fixed term absorbs the rest
    truth = _truth()
    ctx = 4096
    draft, verify, _ = _times(truth, ctx, ARMS[:2], (1,))
    t_base = truth.weight_bytes / truth.bandwidth + 1e-6
    fit = fit_cost_model(truth, ctx, draft, {1: t_base + 2e-6}, t_base)
    assert fit.full_kv_bandwidth == truth.full_kv_bandwidth
    assert fit.fixed_verify >= 0.0 and np.isfinite(fit.t_baseline(ctx))


def test_fixed_rounds_controller():
    a, b = ARMS[:2]
    c = FixedRounds([(a, 0), (a, 1), (b, 4)])
    assert [c.select(100) for _ in range(5)] == [(a, 0), (a, 1), (b, 4), (b, 4), (b, 4)]
    assert c.arms == [a, b]
    c.update(a, 1, 1, 100)


def test_phase_log_starts_empty():
    log = PhaseLog()
    log.collect()
    assert log.draft == {} and log.verify == {} and log.resync == [] and log.host == []
