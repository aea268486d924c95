"""Compression arms and the arm space (reference draftkv/config.py:9-119).

Kept field for field, with two storage extensions that default to the
reference's behaviour: ``group`` (channels per scale/lo pair; the reference's
``quantize`` hard-wires 64) and ``scale_fp16`` (store scale/lo as IEEE half,
which the reference's byte accounting already assumes; its arithmetic keeps
them in float32, the default here).
"""

from __future__ import annotations

from dataclasses import dataclass
from typing import Iterator, Optional, Sequence


@dataclass(frozen=True, order=True)
class CompressionConfig:
    """How the drafter's view of the KV cache is compressed.

    bits: 2, 3, 4, 8 or 16 (16 = no quantization); keep_frac in (0, 1];
    sink / recent: leading / trailing tokens always kept.
    """

    bits: int = 16
    keep_frac: float = 1.0
    sink: int = 4
    recent: int = 32
    group: int = 64
    scale_fp16: bool = False

    def __post_init__(self) -> None:
        if self.bits not in (2, 3, 4, 8, 16):
            raise ValueError(f"unsupported bits={self.bits}")
        if not 0.0 < self.keep_frac <= 1.0:
            raise ValueError(f"keep_frac must be in (0, 1], got {self.keep_frac}")
        if self.group <= 0:
            raise ValueError(f"group must be positive, got {self.group}")

    @property
    def lossless(self) -> bool:
        return self.bits == 16 and self.keep_frac >= 1.0

    def bytes_per_entry(self, d_head: int, group: Optional[int] = None) -> float:
        """Bytes of one (token, head) K or V vector as the mirror stores it:
        ``bits`` per element plus one scale and one zero per group of
        ``group`` (default: this arm's) channels, each 2 bytes with
        ``scale_fp16`` and 4 bytes (float32) without. With 64-channel groups
        and fp16 meta this is the reference formula (config.py:39-48)."""
        if self.bits == 16:
            return 2.0 * d_head
        g = self.group if group is None else group
        meta = 4.0 if self.scale_fp16 else 8.0
        return d_head * self.bits / 8.0 + meta * max(1, -(-d_head // g))

    def label(self) -> str:
        b = "fp16" if self.bits == 16 else f"{self.bits}b"
        return f"{b}/keep{self.keep_frac:g}"


def default_arms(bits: Sequence[int] = (2, 3, 4, 8, 16), keep_fracs: Sequence[float] = (0.25, 0.5, 1.0),
                 sink: int = 4, recent: int = 32) -> list[CompressionConfig]:
    """Every (bits, keep) pair once, sorted (config.py:56-67)."""
    arms = {(b, k): CompressionConfig(bits=b, keep_frac=k, sink=sink, recent=recent)
            for b in bits for k in keep_fracs}
    return sorted(arms.values())


def gamma_range(gamma_max: int = 8) -> Iterator[int]:
    return iter(range(1, gamma_max + 1))


@dataclass(frozen=True)
class LayerPlan:
    """A per-layer compression assignment (config.py:74-119)."""

    cfgs: tuple

    def __len__(self) -> int:
        return len(self.cfgs)

    def __getitem__(self, i: int) -> CompressionConfig:
        return self.cfgs[i]

    def __iter__(self):
        return iter(self.cfgs)

    def per_layer_bytes(self, ctx: int, n_kv_heads: int, d_head: int) -> float:
        """K+V bytes of the whole plan, priced layer by layer."""
        total = 0.0
        for c in self.cfgs:
            kept = min(ctx, max(c.sink + c.recent, int(round(c.keep_frac * ctx))))
            total += 2.0 * kept * n_kv_heads * c.bytes_per_entry(d_head)
        return total

    def label(self) -> str:
        names = sorted({c.label() for c in self.cfgs})
        if len(names) == 1:
            return f"plan[{names[0]}]"
        counts: dict[str, int] = {}
        for c in self.cfgs:
            counts[c.label()] = counts.get(c.label(), 0) + 1
        return "plan[" + ",".join(f"{k}x{v}" for k, v in sorted(counts.items())) + "]"

    @classmethod
    def uniform(cls, cfg: CompressionConfig, n_layers: int) -> "LayerPlan":
        return cls(tuple([cfg] * n_layers))
