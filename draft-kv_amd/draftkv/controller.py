"""What the engine asks of a controller, and the static policy it uses by default.

Reference interface: draftkv/controller.py:29-48. The engine calls
``select(ctx, key)`` once per round for ``(cfg, gamma)`` and
``update(cfg, gamma, accepted, ctx, key)`` once per sequence after the
round; any object with those two methods drives it (the reference's own
bandit controllers included -- they live with the reference's cost model and
are not part of the decode round this package accelerates). ``gamma == 0``
means a plain full-KV step.
"""

from __future__ import annotations

from typing import Optional, Protocol, runtime_checkable


@runtime_checkable
class Controller(Protocol):
    def select(self, ctx: int, key: Optional[str] = None) -> tuple: ...

    def update(self, cfg, gamma: int, accepted: int, ctx: int, key: Optional[str] = None) -> None: ...


class FixedPolicy:
    """Always the same compression arm and draft length; learns nothing."""

    __slots__ = ("cfg", "gamma")

    def __init__(self, cfg, gamma: int) -> None:
        if int(gamma) < 0:
            raise ValueError(f"gamma must be >= 0, got {gamma}")
        self.cfg = cfg
        self.gamma = int(gamma)

    @property
    def arms(self) -> list:
        return [self.cfg]

    def select(self, ctx: int, key: Optional[str] = None) -> tuple:
        return self.cfg, self.gamma

    def update(self, cfg, gamma: int, accepted: int, ctx: int, key: Optional[str] = None) -> None:
        pass

    def __repr__(self) -> str:
        return f"FixedPolicy({self.cfg!r}, {self.gamma})"
