"""Online choice of (compression arm, draft length).

Reference: draftkv/controller.py:29-335. Host-side scalar Python, kept with
the reference's interface (``select(ctx, key) -> (cfg, gamma)``,
``update(cfg, gamma, accepted, ctx, key)``) and decision rules, so the GPU
engine is driven exactly as the reference engine is.
"""

from __future__ import annotations

from dataclasses import dataclass
from typing import Optional, Protocol, Sequence

import numpy as np

from .config import CompressionConfig, default_arms
from .throughput import CostModel, best_gamma, best_gamma_profile


class Controller(Protocol):
    def select(self, ctx: int, key: Optional[str] = None) -> tuple: ...
    def update(self, cfg, gamma: int, accepted: int, ctx: int, key: Optional[str] = None) -> None: ...


@dataclass
class FixedPolicy:
    """A static arm and draft length."""

    cfg: object
    gamma: int

    def select(self, ctx: int, key=None):
        return self.cfg, self.gamma

    def update(self, cfg, gamma, accepted, ctx, key=None) -> None:
        return None


class _Beta:
    """Beta posterior over per-token acceptance, decaying toward the uniform prior."""

    __slots__ = ("a", "b")

    def __init__(self, a: float = 1.0, b: float = 1.0) -> None:
        self.a, self.b = a, b

    def observe(self, accepted: int, gamma: int, decay: float) -> None:
        self.a = 1.0 + (self.a - 1.0) * decay + accepted
        self.b = 1.0 + (self.b - 1.0) * decay + (1.0 if accepted < gamma else 0.0)

    @property
    def mean(self) -> float:
        return self.a / (self.a + self.b)

    def sample(self, rng: np.random.Generator) -> float:
        return float(rng.beta(self.a, self.b))


class ThompsonController:
    """Thompson sampling over arms; gamma solved in closed form from the
    sampled acceptance (controller.py:68-170)."""

    def __init__(self, cost: CostModel, arms: Optional[Sequence[CompressionConfig]] = None, gamma_max: int = 8,
                 decay: float = 0.995, min_speedup: float = 1.05, switch_amortize: int = 32,
                 commit_rounds: int = 1, seed: int = 0, prior: tuple = (2.0, 1.0)) -> None:
        self.cost = cost
        self.arms = list(arms or default_arms())
        self.gamma_max = gamma_max
        self.decay = decay
        self.min_speedup = min_speedup
        self.switch_amortize = max(1, switch_amortize)
        self.commit_rounds = max(1, commit_rounds)
        self.rng = np.random.default_rng(seed)
        self.prior = prior
        self.post: dict = {}
        self._held = None
        self._since_switch = 0
        self.switches = 0
        self.n_decisions = 0

    def _beta(self, cfg, key) -> _Beta:
        k = (key, cfg)
        if k not in self.post:
            self.post[k] = _Beta(*self.prior)
        return self.post[k]

    def select(self, ctx: int, key=None):
        self.n_decisions += 1
        self._since_switch += 1
        base = 1.0 / self.cost.t_baseline(ctx)
        if self._held is not None:
            a = self._beta(self._held, key).sample(self.rng)
            hg, ht = best_gamma(self.cost, self._held, a, ctx, self.gamma_max)
            if self._since_switch < self.commit_rounds:
                if hg > 0 and ht >= base * self.min_speedup:
                    return self._held, hg
                if hg == 0:
                    return self._held, 0
        penalty = self.cost.rebuild_cost(ctx) / self.switch_amortize
        best_cfg, best_g, best_t = self.arms[0], 0, base
        for cfg in self.arms:
            a = self._beta(cfg, key).sample(self.rng)
            g, t = best_gamma(self.cost, cfg, a, ctx, self.gamma_max, 0.0 if cfg == self._held else penalty)
            if g > 0 and t > best_t:
                best_cfg, best_g, best_t = cfg, g, t
        if best_g > 0 and best_cfg != self._held:
            self._held, self._since_switch = best_cfg, 0
            self.switches += 1
        if best_g > 0 and best_t < base * self.min_speedup:
            best_g = 0
        return best_cfg, best_g

    def update(self, cfg, gamma, accepted, ctx, key=None) -> None:
        if gamma > 0:
            self._beta(cfg, key).observe(accepted, gamma, self.decay)

    def alpha_estimates(self, key=None) -> dict:
        return {c: self._beta(c, key).mean for c in self.arms}

    def best_known(self, ctx: int, key=None):
        rows = []
        for cfg in self.arms:
            g, t = best_gamma(self.cost, cfg, self._beta(cfg, key).mean, ctx, self.gamma_max)
            rows.append((t, cfg, g))
        t, cfg, g = max(rows)
        return cfg, g, t


class FlatBandit:
    """Every (arm, gamma) pair as its own arm -- the baseline formulation."""

    def __init__(self, cost: CostModel, arms=None, gamma_max: int = 8, decay: float = 0.995, seed: int = 0):
        self.cost = cost
        self.cfgs = list(arms or default_arms())
        self.gamma_max = gamma_max
        self.decay = decay
        self.rng = np.random.default_rng(seed)
        self.post = {(c, g): _Beta(2.0, 1.0) for c in self.cfgs for g in range(1, gamma_max + 1)}

    def select(self, ctx: int, key=None):
        best, best_t = (self.cfgs[0], 1), -1.0
        for (cfg, g), post in self.post.items():
            t = self.cost.throughput(cfg, g, post.sample(self.rng), ctx)
            if t > best_t:
                best, best_t = (cfg, g), t
        return best

    def update(self, cfg, gamma, accepted, ctx, key=None) -> None:
        if gamma > 0:
            self.post[(cfg, gamma)].observe(accepted, gamma, self.decay)


class OraclePolicy:
    """Plays the exact argmax given every arm's true acceptance."""

    def __init__(self, cost: CostModel, alphas: dict, gamma_max: int = 8):
        self.cost, self.alphas, self.gamma_max = cost, alphas, gamma_max

    def select(self, ctx: int, key=None):
        rows = []
        for c, a in self.alphas.items():
            g, t = best_gamma(self.cost, c, a, ctx, self.gamma_max)
            rows.append((t, c, g))
        t, cfg, g = max(rows)
        return cfg, g

    def update(self, cfg, gamma, accepted, ctx, key=None) -> None:
        return None


class DepthThompsonController:
    """Thompson sampling with one Beta per (arm, draft depth) (controller.py:233-335)."""

    def __init__(self, cost: CostModel, arms=None, gamma_max: int = 12, decay: float = 0.995,
                 min_speedup: float = 1.05, switch_amortize: int = 32, seed: int = 0, prior=(2.0, 1.0),
                 min_obs: float = 1.0):
        self.cost = cost
        self.arms = list(arms or default_arms())
        self.gamma_max = gamma_max
        self.decay = decay
        self.min_speedup = min_speedup
        self.switch_amortize = max(1, switch_amortize)
        self.rng = np.random.default_rng(seed)
        self.prior = prior
        self.min_obs = min_obs
        self.post: dict = {}
        self.obs: dict = {}
        self._held = None
        self.switches = 0

    def _profile_post(self, cfg, key):
        k = (key, cfg)
        if k not in self.post:
            self.post[k] = [_Beta(*self.prior) for _ in range(self.gamma_max)]
            self.obs[k] = [0.0] * self.gamma_max
        return self.post[k]

    def _profile(self, cfg, key, draw: bool) -> list:
        post = self._profile_post(cfg, key)
        obs = self.obs[(key, cfg)]
        out, last = [], None
        for d in range(self.gamma_max):
            if obs[d] >= self.min_obs:
                last = post[d].sample(self.rng) if draw else post[d].mean
                out.append(last)
            elif last is not None:
                out.append(last)
            else:
                out.append(post[d].sample(self.rng) if draw else post[d].mean)
        return out

    def sample_profile(self, cfg, key=None) -> list:
        return self._profile(cfg, key, True)

    def mean_profile(self, cfg, key=None) -> list:
        return self._profile(cfg, key, False)

    def select(self, ctx: int, key=None):
        base = 1.0 / self.cost.t_baseline(ctx)
        penalty = self.cost.rebuild_cost(ctx) / self.switch_amortize
        best_cfg, best_g, best_t = self.arms[0], 0, base
        for cfg in self.arms:
            prof = self.sample_profile(cfg, key)
            g, t = best_gamma_profile(self.cost, cfg, prof, ctx, 0.0 if cfg == self._held else penalty)
            if g > 0 and t > best_t:
                best_cfg, best_g, best_t = cfg, g, t
        if best_g > 0 and best_cfg != self._held:
            self._held = best_cfg
            self.switches += 1
        if best_g > 0 and best_t < base * self.min_speedup:
            best_g = 0
        return best_cfg, best_g

    def update(self, cfg, gamma, accepted, ctx, key=None) -> None:
        if gamma <= 0:
            return
        post = self._profile_post(cfg, key)
        obs = self.obs[(key, cfg)]
        for d in range(min(accepted, self.gamma_max)):
            post[d].observe(1, 1, self.decay)
            obs[d] += 1
        if accepted < gamma and accepted < self.gamma_max:
            post[accepted].observe(0, 1, self.decay)
            obs[accepted] += 1
