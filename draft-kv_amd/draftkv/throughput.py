"""Tokens per verify pass and the memory-traffic cost model.

Reference: draftkv/throughput.py:24-155,188-268 (``expected_tokens``,
``CostModel``'s byte, time, throughput, speedup and ceiling terms,
``best_gamma``). The formulas are the reference's, so a CostModel built with
MI355X parameters -- ``bandwidth=8e12`` -- prices the same decisions; the
depth-profile and arm-switch terms, which only the reference's bandit
controllers use, are not part of the decode round and are left out.
"""

from __future__ import annotations

from dataclasses import dataclass
from typing import Optional

from .config import CompressionConfig


def _clip01(a: float) -> float:
    return min(1.0, max(0.0, float(a)))


def expected_tokens(alpha: float, gamma: int) -> float:
    """E = (1 - alpha^(gamma+1)) / (1 - alpha): accepted run plus the bonus token."""
    if gamma < 0:
        raise ValueError("gamma must be >= 0")
    a = _clip01(alpha)
    if a >= 1.0 - 1e-12:
        return float(gamma + 1)
    return (1.0 - a ** (gamma + 1)) / (1.0 - a)



@dataclass
class CostModel:
    """Decode wall-clock from bytes moved (defaults: Llama-3-8B shape, 2 TB/s)."""

    n_layers: int = 32
    n_kv_heads: int = 8
    d_head: int = 128
    weight_bytes: float = 16.0e9
    bandwidth: float = 2.0e12
    full_kv_bandwidth: Optional[float] = None
    batch: int = 1
    hbm_kv_budget: Optional[float] = None
    compute_per_token: float = 1.0e-6
    fixed_draft: float = 5.0e-6
    fixed_verify: float = 1.0e-5
    resync_per_token: float = 2.0e-6
    controller_overhead: float = 1.0e-6

    def __post_init__(self) -> None:
        if self.full_kv_bandwidth is None:
            self.full_kv_bandwidth = self.bandwidth

    # bytes
    def full_kv_bytes(self, ctx: int) -> float:
        return 2.0 * 2.0 * ctx * self.n_layers * self.n_kv_heads * self.d_head * self.batch

    def draft_kv_bytes(self, cfg, ctx: int) -> float:
        if hasattr(cfg, "per_layer_bytes"):
            return cfg.per_layer_bytes(ctx, self.n_kv_heads, self.d_head) * self.batch
        kept = min(ctx, max(cfg.sink + cfg.recent, int(round(cfg.keep_frac * ctx))))
        return 2.0 * kept * self.n_layers * self.n_kv_heads * cfg.bytes_per_entry(self.d_head) * self.batch

    # times
    def _kv_read_time(self, nbytes: float) -> float:
        if self.hbm_kv_budget is None:
            return nbytes / self.bandwidth
        on_chip = min(nbytes, self.hbm_kv_budget)
        spill = max(0.0, nbytes - self.hbm_kv_budget)
        return on_chip / self.bandwidth + spill / self.full_kv_bandwidth

    def draft_kv_resident_frac(self, cfg, ctx: int) -> float:
        n = self.draft_kv_bytes(cfg, ctx)
        if self.hbm_kv_budget is None or n <= 0:
            return 1.0
        return min(1.0, self.hbm_kv_budget / n)

    def _weights_time(self) -> float:
        return self.weight_bytes / self.bandwidth

    def t_draft(self, cfg, ctx: int) -> float:
        return (self._weights_time() + self._kv_read_time(self.draft_kv_bytes(cfg, ctx))
                + self.compute_per_token + self.fixed_draft)

    def t_verify(self, ctx: int, gamma: int) -> float:
        return (self._weights_time() + self.full_kv_bytes(ctx) / self.full_kv_bandwidth
                + (gamma + 1) * self.compute_per_token + self.fixed_verify)

    def t_baseline(self, ctx: int) -> float:
        return (self._weights_time() + self.full_kv_bytes(ctx) / self.full_kv_bandwidth
                + self.compute_per_token + self.fixed_verify)

    # objectives
    def round_cost(self, cfg, gamma: int, alpha: float, ctx: int, extra_cost: float = 0.0) -> float:
        return (gamma * self.t_draft(cfg, ctx) + self.t_verify(ctx, gamma)
                + expected_tokens(alpha, gamma) * self.resync_per_token + self.controller_overhead + extra_cost)

    def throughput(self, cfg, gamma: int, alpha: float, ctx: int, extra_cost: float = 0.0) -> float:
        if gamma == 0:
            return 1.0 / self.t_baseline(ctx)
        return expected_tokens(alpha, gamma) / self.round_cost(cfg, gamma, alpha, ctx, extra_cost)

    def speedup(self, cfg, gamma: int, alpha: float, ctx: int) -> float:
        return self.throughput(cfg, gamma, alpha, ctx) * self.t_baseline(ctx)

    def ceiling(self, cfg, ctx: int) -> float:
        """Speedup as alpha -> 1 and gamma -> infinity (throughput.py:214-225)."""
        base = self._weights_time() + self.full_kv_bytes(ctx) / self.full_kv_bandwidth
        draft = self._weights_time() + self._kv_read_time(self.draft_kv_bytes(cfg, ctx))
        return (base + self.compute_per_token + self.fixed_verify) / (
            draft + self.compute_per_token + self.fixed_draft + self.resync_per_token)



def best_gamma(cost: CostModel, cfg, alpha: float, ctx: int, gamma_max: int = 8,
               extra_cost: float = 0.0) -> tuple[int, float]:
    best, best_t = 0, cost.throughput(cfg, 0, alpha, ctx)
    for g in range(1, gamma_max + 1):
        t = cost.throughput(cfg, g, alpha, ctx, extra_cost)
        if t > best_t:
            best, best_t = g, t
    return best, best_t
