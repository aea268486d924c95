"""DRAFTKV on MI355X: KV-cache compression as a pure speed knob.

Drop-in for the reference package (aabhimittal/Draft-KV, ``draftkv``): the
same public names and call signatures, with the decode round -- quantized
drafter mirror, paged full cache, drafter and verify attention, acceptance --
running in a gfx950 HIP library (``_lib/libdraftkv_hip.so``).
"""

from .compress import CompressedKVCache, FullKVCache, quantize
from .config import CompressionConfig, LayerPlan, default_arms
from .controller import DepthThompsonController, FixedPolicy, FlatBandit, OraclePolicy, ThompsonController
from .engine import DraftKVEngine, GenerationResult, RoundLog
from .model import TinyTransformer
from .paged import BlockPool, BlockPoolExhausted, PagedKVCache, plan_blocks_needed
from .throughput import CostModel, best_gamma, best_gamma_profile, expected_tokens, expected_tokens_profile

__all__ = [
    "BlockPool", "BlockPoolExhausted", "CompressedKVCache", "CompressionConfig", "CostModel",
    "DepthThompsonController", "DraftKVEngine", "FixedPolicy", "FlatBandit", "FullKVCache", "GenerationResult",
    "LayerPlan", "OraclePolicy", "PagedKVCache", "RoundLog", "ThompsonController", "TinyTransformer", "best_gamma",
    "best_gamma_profile", "default_arms", "expected_tokens", "expected_tokens_profile", "plan_blocks_needed",
    "quantize",
]
__version__ = "0.1.0"
