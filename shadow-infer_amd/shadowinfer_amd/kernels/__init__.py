"""Kernel-backend registry of the gfx950 data plane.

Mirrors the reference's registry (shadowinfer/kernels/__init__.py:63-87,
382-420): a status dict telling which kernels are active, a memoized,
lock-guarded library load, and the internal int4 byte helpers used by the KV
cache. Every kernel here is HIP; the status reports ``"hip"`` for a kernel
whose library is loaded and ``"unavailable"`` otherwise (there is no CPU
fallback to report).
"""

from __future__ import annotations

import torch
from torch import Tensor

from .. import _native

__all__ = ["get_kernel_status", "_pack_int4", "_unpack_int4", "load_native"]

_KERNELS = (
    "plan_scan_kernel",
    "kv_pack_kernel",
    "kv_unpack_kernel",
    "kv_reuse_kernel",
    "kv_compact_kernel",
    "int8_kernel",
    "int4_kernel",
    "int8_gemm_kernel",
    "fused_attention_kernel",
    "kv_sensitivity_kernel",
    "admit_codes_kernel",
)


def load_native():
    """Load the HIP library (memoized). Raises RuntimeError if it cannot be loaded."""
    return _native.load()


def get_kernel_status() -> dict:
    """Which kernels are active (reference: kernels/__init__.py:78-87)."""
    try:
        lib = _native.load()
        loaded, version = True, int(lib.si_abi_version())
    except RuntimeError:
        loaded, version = False, None
    status = {
        "hip_available": torch.cuda.is_available(),
        "hip_extensions_loaded": loaded,
        "abi_version": version,
        "library": _native.LIB_PATH,
        "load_error": _native.load_error(),
        "cpu_fallback": False,
    }
    for name in _KERNELS:
        status[name] = "hip" if loaded else "unavailable"
    return status


def _pack_int4(int8_tensor: Tensor) -> Tensor:
    """int8-encoded int4 values -> bytes, first value in the high nibble
    (reference kernels/__init__.py:382-402; offset-binary, odd tail padded)."""
    _native.require_device(int8_tensor, "_pack_int4")
    flat = int8_tensor.reshape(-1).to(torch.int8).contiguous()
    n = flat.numel()
    out = torch.empty((n + 1) // 2, dtype=torch.uint8, device=flat.device)
    if n:
        _native.call("si_int4_pack_rows", flat.data_ptr(), 1, n, out.data_ptr(),
                     _native.stream(flat.device))
    return out


def _unpack_int4(packed: Tensor, num_elements: int) -> Tensor:
    """Inverse of :func:`_pack_int4` (reference kernels/__init__.py:405-420)."""
    _native.require_device(packed, "_unpack_int4")
    flat = packed.reshape(-1).contiguous()
    n = min(int(num_elements), 2 * flat.numel())
    out = torch.empty(n, dtype=torch.int8, device=flat.device)
    if n:
        _native.call("si_int4_unpack_rows", flat.data_ptr(), 1, flat.numel(), n, out.data_ptr(),
                     _native.stream(flat.device))
    return out
