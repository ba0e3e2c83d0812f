"""ctypes binding of libshadowinfer_hip.so (the C ABI in include/shadowinfer_hip.h).

The library is loaded lazily, once, under a lock (the pattern of the
reference's extension loader, shadowinfer/kernels/__init__.py:94-158). There
is no fallback: if the library is missing or a call fails, a RuntimeError
says why.

``torch`` is imported before the library is opened so that the HIP runtime
torch already loaded (soname libamdhip64.so.7) is the one the library binds
to; device pointers and streams are then shared with torch.
"""

from __future__ import annotations

import ctypes
import os
import threading
from typing import Optional

import torch

LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "_lib",
                        "libshadowinfer_hip.so")

DT_F32, DT_F16, DT_BF16 = 0, 1, 2
_TORCH_TO_DT = {torch.float32: DT_F32, torch.float16: DT_F16, torch.bfloat16: DT_BF16}
_DT_TO_TORCH = {v: k for k, v in _TORCH_TO_DT.items()}

_lock = threading.Lock()
_lib: Optional[ctypes.CDLL] = None
_load_attempted = False
_load_error: Optional[str] = None

_vp = ctypes.c_void_p
_i64 = ctypes.c_int64
_i32 = ctypes.c_int
_sz = ctypes.c_size_t
_PTR16 = ctypes.c_void_p * 16
_PTR4 = ctypes.c_void_p * 4

_SIGNATURES = {
    "si_abi_version": (_i32, []),
    "si_last_error": (ctypes.c_char_p, []),
    "si_check_bf16_convert": (_i32, [_vp, _vp]),
    "si_tune_gemm_plan": (None, [_i32, _i32]),
    "si_tune_attn_offset64": (None, [_i32]),
    "si_plan_workspace_bytes": (_sz, [_i64]),
    "si_plan_scan": (_i32, [_vp, _vp, _i64, _vp, _vp, _vp, _vp, _sz, _vp]),
    "si_plan_scatter": (_i32, [_vp, _vp, _i64, _i64, _vp, _vp, _vp]),
    "si_plan_scan_lists": (_i32, [_vp, _vp, _i64, _i64, _vp, _vp, _vp, _vp, _vp, _vp, _sz, _vp]),
    "si_kv_pack": (_i32, [_vp, _vp, _i32, _i64, _i64, _i64, _i64, _i64, _vp, _vp, _vp, _vp]),
    "si_kv_pack_flat": (_i32, [_vp, _vp, _i32, _i64, _i64, _i64, _i64, _i64, _vp, _vp, _vp, _vp,
                               _vp, _vp]),
    "si_kv_pack_rope_flat": (_i32, [_vp, _vp, _vp, _i32, _i64, _i64, _i64, _i64, _i64, _vp,
                                    _vp, _vp, _vp, _vp, _vp]),
    "si_kv_pack_copy": (_i32, [_vp, _vp, _i32, _i64, _i64, _i64, _i64, _i64, _vp, _vp, _vp, _vp,
                               _vp, _vp, _vp, _vp, _vp]),
    "si_page_write": (_i32, [_vp, _vp, _i32, _i64, _i64, _i64, _i64, _i64, _i64, _i32, _i64, _vp,
                             _i64, _i64, _vp]),
    "si_page_write_pages": (_i32, [_vp, _vp, _i32, _i64, _i64, _i64, _i64, _i64, _i64, _i32, _i64,
                                   _vp, _i64, _vp]),
    "si_page_gather": (_i32, [_vp, _i64, _i64, _i64, _i64, _i64, _i64, _vp, _vp, _vp]),
    "si_kv_unpack_flat": (_i32, [_vp, _vp, _vp, _vp, _vp, _i32, _i64, _i64, _i64, _i64, _i64, _vp,
                                 _vp, _vp]),
    "si_kv_unpack": (_i32, [_vp, _vp, _vp, _i32, _i64, _i64, _i64, _i64, _i64, _vp, _vp, _vp]),
    "si_kv_reuse": (_i32, [_vp, _vp, _vp, _i64, _vp, _vp, _vp, _i64, _vp, _i64, _i64, _i64,
                           _i64, _i32, _vp, _vp]),
    "si_kv_compact": (_i32, [_vp, _vp, _vp, _vp, _vp, _vp, _i64, _i64, _i64, _i64, _i32, _vp]),
    "si_kv_reuse_flat": (_i32, [_vp, _vp, _vp, _i64, _vp, _vp, _vp, _i64, _vp, _i64, _i64, _i64,
                                _i64, _i32, _vp, _vp]),
    "si_kv_evict_chunks": (_i64, [_vp]),
    "si_kv_evict_chunk_words": (_i64, []),
    "si_kv_evict_count": (_i32, [_vp, _vp, _vp, _vp, _i64, _i64, _vp, _vp, _vp, _vp, _vp]),
    "si_kv_evict_flat": (_i32, [_vp, _vp, _vp, _vp, _i64, _i64, _vp, _vp, _vp, _vp, _vp, _i64,
                                _i64, _i64, _i32, _vp]),
    "si_kv_compact_flat": (_i32, [_vp, _vp, _vp, _vp, _vp, _i64, _i64, _i64, _i64, _i64, _i32,
                                  _vp]),
    "si_attn_workspace_bytes": (_sz, [_i64, _i64]),
    "si_attn_packed_fwd": (_i32, [_vp, _i32, _i64, _i64, _i64, _i64, _vp, _vp, _vp, _i32, _i64,
                                  _i64, ctypes.c_float, _vp, _i32, _vp, _sz, _vp]),
    "si_attn_packed_fwd_tokens": (_i32, [_vp, _i32, _i64, _i64, _i64, _i64, _vp, _vp, _vp, _i32,
                                         _i64, _i64, ctypes.c_float, _vp, _i32, _vp, _sz, _vp]),
    "si_attn_build_lists": (_i32, [_vp, _vp, _i64, _i64, _vp, _sz, _vp]),
    "si_attn_packed_fwd_built": (_i32, [_vp, _i32, _i64, _i64, _i64, _i64, _vp, _sz, _vp, _i32,
                                        _i64, _i64, ctypes.c_float, _vp, _i32, _i32, _vp]),
    "si_quant_rows_i8": (_i32, [_vp, _i32, _i64, _i64, _vp, _vp, _vp]),
    "si_quant_rows_i4": (_i32, [_vp, _i32, _i64, _i64, _i64, _vp, _vp, _vp]),
    "si_int4_pack_rows": (_i32, [_vp, _i64, _i64, _vp, _vp]),
    "si_int4_unpack_rows": (_i32, [_vp, _i64, _i64, _i64, _vp, _vp]),
    "si_dequant_rows": (_i32, [_vp, _vp, _i32, _i64, _i64, _i64, _vp, _vp]),
    "si_weight_quant_i8": (_i32, [_vp, _i64, _i64, _vp, _vp, _vp]),
    "si_act_quant_i8": (_i32, [_vp, _i32, _i64, _i64, _vp, _vp, _vp]),
    "si_gemm_workspace_bytes": (_sz, [_i64, _i64, _i64]),
    "si_gemm_i8i8_i32": (_i32, [_vp, _vp, _i64, _i64, _i64, _vp, _vp, _sz, _vp]),
    "si_gemm_i8_dequant": (_i32, [_vp, _vp, _vp, _vp, _vp, _i64, _i64, _i64, _vp, _i32, _vp,
                                  _sz, _vp]),
    "si_gemm_i8_dequant_add": (_i32, [_vp, _vp, _vp, _vp, _vp, _vp, _i64, _i64, _i64, _vp, _i32,
                                      _vp, _sz, _vp]),
    "si_kv_sensitivity": (_i32, [_vp, _vp, _i32, _i64, _i64, _i64, _i64, _vp, _vp]),
    "si_admit_workspace_bytes": (_sz, [_i64]),
    "si_admit_codes": (_i32, [_vp, _vp, _i64, _i64, _vp, _vp, _vp, _i64, _i64, _i32, _i32, _vp,
                              _vp, _vp, _sz, _vp]),
    "si_rmsnorm_rows": (_i32, [_vp, _i32, _i64, _i64, _vp, ctypes.c_float, _vp, _vp, _vp, _vp]),
    "si_add_rmsnorm_rows": (_i32, [_vp, _vp, _i32, _i64, _i64, _vp, ctypes.c_float, _vp, _vp, _vp,
                                   _vp, _vp]),
    "si_rope_split": (_i32, [_vp, _i32, _i64, _i64, _i64, _i64, _vp, _vp, _vp, _vp, _vp, _vp]),
    "si_swiglu_quant": (_i32, [_vp, _i32, _i64, _i64, _vp, _vp, _vp, _vp]),
    "si_row_argmax_conf": (_i32, [_vp, _i32, _i64, _i64, _vp, _vp, _vp]),
    "si_reuse_drift_workspace_bytes": (_sz, [_i64]),
    "si_reuse_drift": (_i32, [_vp, _vp, _i32, _i64, _vp, _vp, _sz, _vp]),
    "si_reuse_apply": (_i32, [_vp, _vp, _vp, _i32, _i64, _vp, _vp]),
    "si_int8_linear_workspace_bytes": (_sz, [_i64, _i64, _i64]),
    "si_int8_linear_forward": (_i32, [_vp, _i32, _i64, _i64, _i64, _vp, _vp, _vp, _vp, _vp,
                                      _sz, _vp]),
    "si_int8_linear_forward_add": (_i32, [_vp, _i32, _i64, _i64, _i64, _vp, _vp, _vp, _vp, _vp,
                                          _vp, _sz, _vp]),
    "si_int8_linear_forward_noalloc": (_i32, [_vp, _i32, _i64, _i64, _i64, _vp, _vp, _vp, _vp,
                                              _vp]),
}

EXPORTED_SYMBOLS = tuple(_SIGNATURES)


def _declare(lib: ctypes.CDLL) -> None:
    for name, (res, args) in _SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args


def load() -> ctypes.CDLL:
    """Return the loaded library, loading it on first use (memoized, locked)."""
    global _lib, _load_attempted, _load_error
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is None:
            if _load_attempted and _load_error is not None:
                raise RuntimeError(_load_error)
            _load_attempted = True
            if not os.path.exists(LIB_PATH):
                _load_error = (f"HIP library not built: {LIB_PATH} is missing "
                               "(run shadow-infer_amd/build.py)")
                raise RuntimeError(_load_error)
            try:
                lib = ctypes.CDLL(LIB_PATH)
                _declare(lib)
            except (OSError, AttributeError) as exc:
                _load_error = f"cannot load {LIB_PATH}: {exc}"
                raise RuntimeError(_load_error) from exc
            _lib = lib
    return _lib


def loaded() -> bool:
    return _lib is not None


def load_error() -> Optional[str]:
    return _load_error


def force_cpu() -> bool:
    """The reference's switch to its CPU kernels (kernels/dispatcher.py:46-49)."""
    return os.environ.get("SHADOWINFER_FORCE_CPU_KERNELS", "0") == "1"


def _refuse_forced_cpu(what: str) -> None:
    if force_cpu():
        raise RuntimeError(
            f"{what}: SHADOWINFER_FORCE_CPU_KERNELS=1 asks for CPU kernels, and this data "
            "plane has none (every kernel is HIP); unset it to run on the GPU")


def call(name: str, *args) -> None:
    """Invoke ``name`` and raise RuntimeError with the library's message on failure."""
    _refuse_forced_cpu(name)
    lib = load()
    rc = getattr(lib, name)(*args)
    if rc != 0:
        msg = lib.si_last_error().decode(errors="replace")
        if rc == 1:
            raise ValueError(f"{name}: {msg}")
        raise RuntimeError(f"{name}: {msg} (status {rc})")


def size_query(name: str, *args) -> int:
    return int(getattr(load(), name)(*args))


def ptr(t: Optional[torch.Tensor]) -> Optional[int]:
    return None if t is None else t.data_ptr()


def stream(device: torch.device) -> int:
    return torch.cuda.current_stream(device).cuda_stream


def dtype_code(dtype: torch.dtype) -> int:
    try:
        return _TORCH_TO_DT[dtype]
    except KeyError:
        raise TypeError(f"unsupported dtype {dtype}; expected float32, float16 or bfloat16")


def torch_dtype(code: int) -> torch.dtype:
    return _DT_TO_TORCH[code]


def require_device(t: torch.Tensor, what: str) -> None:
    """The data plane runs only as HIP kernels: CPU tensors are an error."""
    _refuse_forced_cpu(what)
    if t.device.type != "cuda":
        raise RuntimeError(
            f"{what}: tensors must live on a HIP device (got {t.device}); "
            "this data plane has no CPU implementation")
    load()


def table16(ptrs) -> "ctypes.Array":
    arr = _PTR16()
    for i, p in enumerate(ptrs):
        arr[i] = p
    return arr


def table4(ptrs) -> "ctypes.Array":
    arr = _PTR4()
    for i, p in enumerate(ptrs):
        arr[i] = p
    return arr
