"""CostModel calibration from measured decode rounds.

The reference prices a round with ``CostModel`` (draftkv/throughput.py:69-81
holds its parameters, :110-155 the times they enter): a draft step streams
the weights and the drafter's cache, a verify pass the weights and the full
cache, and fixed per-step, per-token and per-round terms cover launches,
sampling, resync and the controller. Its defaults describe an H100-class
device; here the parameters are fitted to times measured on the device, and
the class itself is left untouched (a calibrated model is an ordinary
``CostModel`` with other numbers).

``PhaseLog`` collects, per decode round, the GPU time of its phases (HIP
events around the draft steps, the verify forward + accept, the rollback +
resync) and the host time of the round's bookkeeping; a round with gamma 0
is one full-KV decode step. ``fit_cost_model`` turns those samples into a
``CostModel`` whose predictions reproduce the measured medians:

* ``bandwidth`` -- slope of the draft-step time over the drafter's KV bytes
  (two or more arms with different bytes), so the weights and the compressed
  cache stream at the rate the device showed for them;
* ``compute_per_token`` -- slope of the verify time over gamma (each extra
  query row of a verify pass), taken against the full-KV step;
* ``fixed_draft`` -- what the draft step costs beyond the streamed bytes;
* ``full_kv_bandwidth`` -- the full-KV step's rate for the full cache, with
  ``fixed_verify`` set equal to ``fixed_draft`` (one forward's launches);
* ``resync_per_token`` -- rollback + resync time per emitted token;
* ``controller_overhead`` -- the host's per-round bookkeeping.
"""

from __future__ import annotations

import dataclasses
from typing import Dict, List, Optional, Sequence

import numpy as np

from .throughput import CostModel


class PhaseLog:
    """Per-round phase times of a ``DecodeBatch`` (enabled by setting
    ``batch.phases = PhaseLog()``). Events are read lazily, after the round's
    own host synchronisation, so timing adds no waits."""

    def __init__(self) -> None:
        self.draft: Dict[object, List[float]] = {}     # cfg -> seconds per draft step
        self.verify: Dict[int, List[float]] = {}       # gamma -> seconds per verify pass (0: full-KV step)
        self.resync: List[tuple] = []                  # (seconds, tokens emitted)
        self.host: List[float] = []                    # seconds of host bookkeeping per round
        self._open: List[tuple] = []

    # -- called by DecodeBatch
    def event(self):
        import torch
        e = torch.cuda.Event(enable_timing=True)
        e.record()
        return e

    def add(self, cfg, gamma: int, ev: dict, emitted: int, host_s: float) -> None:
        self._open.append((cfg, gamma, ev, emitted))
        self.host.append(host_s)

    def collect(self) -> None:
        """Resolve the recorded events (waits for the last of them)."""
        for cfg, gamma, ev, emitted in self._open:
            ev["end"].synchronize()
            if gamma > 0:
                self.draft.setdefault(cfg, []).append(ev["d0"].elapsed_time(ev["d1"]) * 1e-3 / gamma)
                self.verify.setdefault(gamma, []).append(ev["d1"].elapsed_time(ev["v1"]) * 1e-3)
            else:
                self.verify.setdefault(0, []).append(ev["d1"].elapsed_time(ev["v1"]) * 1e-3)
            self.resync.append((ev["s0"].elapsed_time(ev["end"]) * 1e-3, emitted))
        self._open.clear()


def _median(xs: Sequence[float]) -> float:
    return float(np.median(np.asarray(xs, np.float64)))


def fit_cost_model(base: CostModel, ctx: int, draft: Dict[object, float], verify: Dict[int, float],
                   t_baseline: Optional[float] = None, resync_per_token: Optional[float] = None,
                   controller_overhead: Optional[float] = None) -> CostModel:
    """Fit ``base``'s time parameters (its shape, weight bytes and batch are
    kept) to measured times at context ``ctx``: ``draft`` maps an arm to the
    seconds of one draft step, ``verify`` maps gamma >= 1 to the seconds of a
    verify pass, ``t_baseline`` is one full-KV decode step (``verify[0]`` if
    absent). Terms the data do not determine keep ``base``'s values."""
    W = base.weight_bytes
    t_base = t_baseline if t_baseline is not None else verify.get(0)
    # bandwidth: the draft-step time is linear in the drafter's KV bytes
    arms = list(draft)
    kv = np.array([base.draft_kv_bytes(c, ctx) for c in arms], np.float64)
    td = np.array([draft[c] for c in arms], np.float64)
    bw = base.bandwidth
    if len(arms) >= 2 and np.ptp(kv) > 0:
        slope, icpt = np.polyfit(kv, td, 1)
        if slope > 0:
            bw = 1.0 / slope
    # compute per query row: verify(g) - baseline = g * cpt
    cpt = base.compute_per_token
    gs = np.array([g for g in verify if g > 0], np.float64)
    if t_base is not None and len(gs):
        tv = np.array([verify[int(g)] for g in gs], np.float64) - t_base
        cpt = max(0.0, float(np.dot(gs, tv) / np.dot(gs, gs)))
    # fixed draft: the draft steps' intercept beyond the streamed bytes
    fd = base.fixed_draft
    if len(arms):
        fd = max(0.0, float(np.mean(td - (W + kv) / bw)) - cpt)
    # the full cache's rate from the full-KV step, with the same fixed launch cost
    fv, fbw = fd, base.full_kv_bandwidth
    if t_base is not None:
        rest = t_base - W / bw - cpt - fv
        if rest > 0:
            fbw = base.full_kv_bytes(ctx) / rest
        else:   # the full cache streams faster than the fit can resolve: keep the rate, absorb in fixed
            fv = max(0.0, t_base - W / bw - cpt - base.full_kv_bytes(ctx) / fbw)
    return dataclasses.replace(
        base, bandwidth=float(bw), full_kv_bandwidth=float(fbw), compute_per_token=float(cpt),
        fixed_draft=float(fd), fixed_verify=float(fv),
        resync_per_token=base.resync_per_token if resync_per_token is None else float(resync_per_token),
        controller_overhead=base.controller_overhead if controller_overhead is None else float(controller_overhead))


def fit_from_log(base: CostModel, ctx: int, log: PhaseLog) -> CostModel:
    """``fit_cost_model`` on the medians of a ``PhaseLog``."""
    log.collect()
    draft = {c: _median(v) for c, v in log.draft.items() if v}
    verify = {g: _median(v) for g, v in log.verify.items() if v}
    rs = None
    toks = sum(t for _, t in log.resync)
    if toks > 0:
        rs = sum(s for s, _ in log.resync) / toks
    co = _median(log.host) if log.host else None
    return fit_cost_model(base, ctx, draft, verify, resync_per_token=rs, controller_overhead=co)


class FixedRounds:
    """Controller for calibration rounds: the given (cfg, gamma) pairs in
    turn, then the last one; update is a no-op."""

    def __init__(self, plan: Sequence[tuple]) -> None:
        self.plan, self.i = list(plan), 0
        self.arms = list(dict.fromkeys(c for c, _ in self.plan))

    def select(self, ctx: int, key=None):
        p = self.plan[min(self.i, len(self.plan) - 1)]
        self.i += 1
        return p

    def update(self, cfg, gamma, accepted, ctx, key=None) -> None:
        pass


def calibrate(batch, base: CostModel, arms: Sequence, gammas: Sequence[int] = (1, 4), reps: int = 2) -> CostModel:
    """Run calibration rounds on a live ``DecodeBatch``: full-KV steps, then
    every (arm, gamma) ``reps`` times (each arm's first round absorbs its
    rebuild and is not used), and fit ``base`` to them at the batch's
    current context. The rounds decode real tokens; the engine's controller
    is restored afterwards."""
    eng = batch.engine
    plan = [(arms[0], 0)] * (reps + 1)
    for a in arms:
        plan.append((a, gammas[0]))          # warm: rebuild under the arm, record its graph
        for g in gammas:
            plan += [(a, g)] * reps
    saved = eng.controller
    eng.controller = FixedRounds(plan)
    log = PhaseLog()
    batch.phases = log
    try:
        skip = {0, reps + 1} | {reps + 1 + i * (1 + reps * len(gammas)) for i in range(len(arms))}
        kept = PhaseLog()
        for i in range(len(plan)):
            if not batch.step():
                break
            log.collect()
            if i in skip:
                log.draft.clear(), log.verify.clear(), log.resync.clear()
                log.host.clear()
                continue
            for c, v in log.draft.items():
                kept.draft.setdefault(c, []).extend(v)
            for g, v in log.verify.items():
                kept.verify.setdefault(g, []).extend(v)
            kept.resync += log.resync
            kept.host += log.host
            log.draft.clear(), log.verify.clear(), log.resync.clear()
            log.host.clear()
    finally:
        batch.phases = None
        eng.controller = saved
    ctx = int(max(len(t) for t in batch.toks))
    return fit_from_log(base, ctx, kept)
