"""shadowinfer_amd: the quantized data plane of ShadowInfer (packed
mixed-precision KV cache and INT8 FFN linear) as gfx950 HIP kernels behind the
reference's Python API."""

__version__ = "0.1.0"

from .ffn_optimizer import INT8Linear, quantize_ffn_modules
from .kernels import get_kernel_status
from .shadowkv import PackedKVCache, PrecisionPlan, codes_to_map, map_to_codes, packed_attention
from .utils import Quantizer

__all__ = [
    "INT8Linear",
    "PackedKVCache",
    "PrecisionPlan",
    "Quantizer",
    "codes_to_map",
    "get_kernel_status",
    "map_to_codes",
    "packed_attention",
    "quantize_ffn_modules",
]
