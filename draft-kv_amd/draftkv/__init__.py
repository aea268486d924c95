"""DRAFTKV on MI355X: KV-cache compression as a pure speed knob.

Drop-in for the reference package (aabhimittal/Draft-KV, ``draftkv``): the
same public names and call signatures, with the decode round -- quantized
drafter mirror, paged full cache, drafter and verify attention, acceptance --
running in a gfx950 HIP library (``_lib/libdraftkv_hip.so``).
"""

from .compress import CompressedKVCache, FullKVCache, quantize
from .config import CompressionConfig, LayerPlan, default_arms
from .controller import Controller, FixedPolicy
from .engine import DraftKVEngine, GenerationResult, RoundLog
from .model import TinyTransformer
from .paged import BlockPool, BlockPoolExhausted, PagedKVCache, plan_blocks_needed
from .throughput import CostModel, best_gamma, expected_tokens

__all__ = [
    "BlockPool", "BlockPoolExhausted", "CompressedKVCache", "CompressionConfig", "Controller", "CostModel",
    "DraftKVEngine", "FixedPolicy", "FullKVCache", "GenerationResult", "LayerPlan", "PagedKVCache", "RoundLog",
    "TinyTransformer", "best_gamma", "default_arms", "expected_tokens", "plan_blocks_needed", "quantize",
]
__version__ = "0.1.0"
