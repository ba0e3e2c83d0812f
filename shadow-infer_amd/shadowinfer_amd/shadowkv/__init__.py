"""Packed mixed-precision KV cache (PackedKVCache), its precision plan, the
rate-distortion admission that chooses the precisions, and the fused
packed-KV attention."""

from .compress import compress_kv_with_plan
from .packed_attention import packed_attention
from .packed_kv_cache import PackedKVCache
from .paged_kv_store import PagedKVStore
from .rd_allocator import (
    admit_budget,
    admit_codes,
    entry_bytes,
    kv_sensitivity,
    predict_codes_bytes,
)
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
    "PagedKVStore",
    "PrecisionPlan",
    "admit_budget",
    "admit_codes",
    "codes_to_map",
    "compress_kv_with_plan",
    "entry_bytes",
    "kv_sensitivity",
    "map_to_codes",
    "packed_attention",
    "predict_codes_bytes",
]
