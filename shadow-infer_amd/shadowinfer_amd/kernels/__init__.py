"""Kernel-backend registry of the gfx950 data plane.

Mirrors the reference's registry (shadowinfer/kernels/__init__.py:63-87,
382-420; kernels/dispatcher.py:46-49): a status dict telling which kernels are
active, a memoized, lock-guarded library load, and the internal int4 byte
helpers used by the KV cache.

``get_kernel_status()`` carries every key of the reference's status dict with
the same types: ``cuda_available`` / ``cuda_extensions_loaded`` (booleans: a
HIP device is visible / the HIP library is loaded), ``int8_kernel``,
``int4_kernel``, ``sparse_gemm_kernel``, ``fused_attention_kernel`` (strings),
``autotune_cache_entries`` (int) and ``force_cpu`` (bool, from
``SHADOWINFER_FORCE_CPU_KERNELS=1``). A kernel this library provides reports
``"hip"`` when the library is loaded and ``"unavailable"`` otherwise; the
reference's sparse FFN GEMM is not part of this data plane and always reports
``"unavailable"``, so callers that test for a native sparse GEMM take their
dense path. There is no CPU fallback: with ``force_cpu`` set every kernel call
raises RuntimeError. Tile choices come from closed-form models, so there is no
autotuning cache (``autotune_cache_entries`` is 0). The build's own keys
(``hip_*``, ``abi_version``, ``library``, ``load_error``, one entry per kernel
family) follow.
"""

from __future__ import annotations

import torch
from torch import Tensor

from .. import _native

__all__ = ["get_kernel_status", "_pack_int4", "_unpack_int4", "load_native", "force_cpu"]

# kernel families of this library (the build's own status keys)
_KERNELS = (
    "plan_scan_kernel",
    "kv_pack_kernel",
    "kv_unpack_kernel",
    "kv_reuse_kernel",
    "kv_compact_kernel",
    "int8_gemm_kernel",
    "kv_sensitivity_kernel",
    "admit_codes_kernel",
    "paged_kv_kernel",
    "step_row_kernel",
)

# keys of the reference's status dict (kernels/__init__.py:63-70) and whether
# this library provides that kernel
_REFERENCE_KERNELS = {
    "int8_kernel": True,
    "int4_kernel": True,
    "sparse_gemm_kernel": False,
    "fused_attention_kernel": True,
}


def force_cpu() -> bool:
    """``SHADOWINFER_FORCE_CPU_KERNELS=1`` (reference kernels/dispatcher.py:46-49)."""
    return _native.force_cpu()


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
    available = bool(torch.cuda.is_available())
    status = {
        "cuda_available": available,
        "cuda_extensions_loaded": loaded,
    }
    for name, provided in _REFERENCE_KERNELS.items():
        status[name] = "hip" if (loaded and provided) else "unavailable"
    status["autotune_cache_entries"] = 0
    status["force_cpu"] = force_cpu()
    status.update({
        "hip_available": available,
        "hip_extensions_loaded": loaded,
        "abi_version": version,
        "library": _native.LIB_PATH,
        "load_error": _native.load_error(),
        "cpu_fallback": False,
    })
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
