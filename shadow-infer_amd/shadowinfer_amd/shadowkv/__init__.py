"""Packed mixed-precision KV cache (PackedKVCache), its precision plan and the
fused packed-KV attention."""

from .packed_attention import packed_attention
from .packed_kv_cache import PackedKVCache
from .precision_plan import (
    CODE_PRECISIONS,
    EVICTED,
    PRECISION_CODES,
    PRECISION_ORDER,
    PrecisionPlan,
    codes_to_map,
    map_to_codes,
)

__all__ = [
    "CODE_PRECISIONS",
    "EVICTED",
    "PRECISION_CODES",
    "PRECISION_ORDER",
    "PackedKVCache",
    "PrecisionPlan",
    "codes_to_map",
    "map_to_codes",
    "packed_attention",
]
