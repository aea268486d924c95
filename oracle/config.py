"""Compression arm and its byte accounting, restated.

Reference: draftkv/config.py:9-53 (``CompressionConfig``), :74-119
(``LayerPlan``). Extension: ``group`` (reference hard-wires 64 through
compress.py:124-125) and ``meta`` ("f32" = the reference's arithmetic, "f16" =
the storage its byte accounting at config.py:39-48 already assumes).
"""

from __future__ import annotations

from dataclasses import dataclass


@dataclass(frozen=True)
class Cfg:
    bits: int = 16
    keep_frac: float = 1.0
    sink: int = 4
    recent: int = 32
    group: int = 64
    meta: str = "f32"

    def __post_init__(self) -> None:        # config.py:29-33
        if self.bits not in (2, 3, 4, 8, 16):
            raise ValueError(f"unsupported bits={self.bits}")
        if not 0.0 < self.keep_frac <= 1.0:
            raise ValueError(f"keep_frac must be in (0, 1], got {self.keep_frac}")

    def bytes_per_entry(self, d_head: int, group: int = 64) -> float:   # config.py:39-48
        if self.bits == 16:
            return 2.0 * d_head
        return d_head * self.bits / 8.0 + 4.0 * max(1, -(-d_head // group))


def budget(cfg: Cfg, seen: int) -> int:
    """compress.py:154-157: Python ``round`` (half to even) of keep * max(seen, 1)."""
    keep = int(round(cfg.keep_frac * max(seen, 1)))
    return max(keep, cfg.sink + cfg.recent)


def closed_form_kept(n: int, cfg: Cfg, seen: int) -> list[int]:
    """Kept storage indices after one eviction over rows whose scores are all 0.

    With every score equal, compress.py:173-174's stable sort drops the oldest
    unprotected rows, so the survivors are the ``sink`` oldest plus the newest
    ``B - sink`` (B = budget). ``recent == 0`` protects every row
    (``order[-0:]`` is the whole array, compress.py:167), so nothing is dropped.
    """
    B = budget(cfg, seen)
    if n <= B or cfg.recent == 0:
        return list(range(n))
    sink = min(cfg.sink, n)
    return list(range(sink)) + list(range(n - (B - sink), n))
