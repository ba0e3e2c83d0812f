"""Thin tensor wrappers over the denoising-step row kernels and the INT8 GEMM
entry points (outputs allocated here, kernels on the current stream).

Every function requires HIP tensors and raises if the library is missing.
"""

from __future__ import annotations

from typing import Optional, Tuple

import torch

from .. import _native
from .._checks import check_rope_args as _check_rope_args


def _ptr(t: Optional[torch.Tensor]) -> Optional[int]:
    return None if t is None else t.data_ptr()


def rmsnorm(x: torch.Tensor, weight: torch.Tensor, eps: float, want_y: bool = True,
            want_q: bool = False, residual: Optional[torch.Tensor] = None
            ) -> Tuple[Optional[torch.Tensor], Optional[torch.Tensor], Optional[torch.Tensor],
                       Optional[torch.Tensor]]:
    """RMSNorm over the last dim of ``x`` as the reference's op chain in the
    row dtype (models/diffusion_llama.py:311-321), optionally preceded by the
    residual add ``x = x + residual`` (diffusion_llama.py:421-422) and fused
    with INT8Linear's activation quantization of the result
    (int8_linear.py:96-98). Returns ``(y, q, scale, x_sum)`` with None for what
    was not asked (``x_sum`` is the rounded ``x + residual``)."""
    _native.require_device(x, "rmsnorm")
    K = x.shape[-1]
    xf = x.reshape(-1, K).contiguous()
    M = xf.shape[0]
    if weight.shape != (K,) or weight.dtype != x.dtype:
        raise ValueError(f"weight must be [{K}] in {x.dtype}")
    y = torch.empty_like(xf) if want_y else None
    q = torch.empty(M, K, dtype=torch.int8, device=x.device) if want_q else None
    s = torch.empty(M, dtype=torch.float32, device=x.device) if want_q else None
    if residual is None:
        xo = None
        _native.call("si_rmsnorm_rows", xf.data_ptr(), _native.dtype_code(x.dtype), M, K,
                     weight.contiguous().data_ptr(), float(eps), _ptr(y), _ptr(q), _ptr(s),
                     _native.stream(x.device))
    else:
        if residual.shape != x.shape or residual.dtype != x.dtype:
            raise ValueError("residual must match x in shape and dtype")
        rf = residual.reshape(-1, K).contiguous()
        xo = torch.empty_like(xf)
        _native.call("si_add_rmsnorm_rows", xf.data_ptr(), rf.data_ptr(),
                     _native.dtype_code(x.dtype), M, K, weight.contiguous().data_ptr(), float(eps),
                     xo.data_ptr(), _ptr(y), _ptr(q), _ptr(s), _native.stream(x.device))
    return ((None if y is None else y.view(x.shape)), q, s,
            (None if xo is None else xo.view(x.shape)))


def rope_split(qkv: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor, batch: int, seq: int,
               heads: int, head_dim: int, kv: bool = True
               ) -> Tuple[torch.Tensor, Optional[torch.Tensor], Optional[torch.Tensor]]:
    """``qkv [B*S, 3*H*D]`` -> rotated q, rotated k and v, each ``[B, H, S, D]``
    (models/diffusion_llama.py:362-373); ``cos``/``sin`` ``[S, D]`` in qkv's dtype.
    ``kv=False`` writes q only (k and v are returned as None)."""
    _check_rope_args(qkv, cos, sin, batch, seq, heads, head_dim, "rope_split")
    # contiguous copies stay bound until the launch is queued
    src, cos_c, sin_c = qkv.contiguous(), cos.contiguous(), sin.contiguous()
    q = torch.empty(batch, heads, seq, head_dim, dtype=qkv.dtype, device=qkv.device)
    k = torch.empty_like(q) if kv else None
    v = torch.empty_like(q) if kv else None
    _native.call("si_rope_split", src.data_ptr(), _native.dtype_code(qkv.dtype), batch, seq,
                 heads, head_dim, cos_c.data_ptr(), sin_c.data_ptr(),
                 q.data_ptr(), _native.ptr(k), _native.ptr(v), _native.stream(qkv.device))
    return q, k, v


def rope_pack_supported(dtype: torch.dtype, head_dim: int, group_size: int) -> bool:
    """Whether ``PackedKVCache.pack_projection`` (si_kv_pack_rope_flat) takes
    these shapes: bf16/fp16 rows, D = 64 or 128, int4 groups of 8 * 2^k dividing D."""
    g = group_size if head_dim % group_size == 0 else head_dim
    return (dtype in (torch.bfloat16, torch.float16) and head_dim in (64, 128)
            and g % 8 == 0 and (g // 8) & (g // 8 - 1) == 0)


def swiglu_quant(gate_up: torch.Tensor, want_h: bool = False
                 ) -> Tuple[Optional[torch.Tensor], torch.Tensor, torch.Tensor]:
    """``gate_up [M, 2F]`` -> (h = silu(gate) * up ``[M, F]`` or None, int8 q
    ``[M, F]``, fp32 scale ``[M]``): models/diffusion_llama.py:332-333 and the
    down projection's INT8Linear prologue."""
    _native.require_device(gate_up, "swiglu_quant")
    src = gate_up.contiguous()
    M, F2 = src.shape
    F = F2 // 2
    if F2 != 2 * F:
        raise ValueError("gate_up must have an even number of columns")
    h = torch.empty(M, F, dtype=src.dtype, device=src.device) if want_h else None
    q = torch.empty(M, F, dtype=torch.int8, device=src.device)
    s = torch.empty(M, dtype=torch.float32, device=src.device)
    _native.call("si_swiglu_quant", src.data_ptr(), _native.dtype_code(src.dtype), M, F, _ptr(h),
                 q.data_ptr(), s.data_ptr(), _native.stream(src.device))
    return h, q, s


def int8_gemm_dequant(q: torch.Tensor, sx: torch.Tensor, qweight_nk: torch.Tensor,
                      sw: torch.Tensor, out_dtype: torch.dtype,
                      bias: Optional[torch.Tensor] = None,
                      residual: Optional[torch.Tensor] = None) -> torch.Tensor:
    """INT8Linear.forward after its prologue (int8_linear.py:102-115):
    ``T(float(q @ qweight_nk^T) * (sx[m] * sw[n]) [+ bias])``; with
    ``residual`` (``[M, N]`` in ``out_dtype``) the decoder layer's residual add
    follows in the same pass: ``T(residual + T(...))``
    (models/diffusion_llama.py:421-423)."""
    _native.require_device(q, "int8_gemm_dequant")
    M, K = q.shape
    N = qweight_nk.shape[0]
    if qweight_nk.shape != (N, K):
        raise ValueError(f"qweight_nk must be [N, {K}], got {tuple(qweight_nk.shape)}")
    out = torch.empty(M, N, dtype=out_dtype, device=q.device)
    ws_bytes = _native.size_query("si_gemm_workspace_bytes", M, N, K)
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device=q.device) if ws_bytes else None
    if residual is None:
        _native.call("si_gemm_i8_dequant", q.data_ptr(), sx.data_ptr(), qweight_nk.data_ptr(),
                     sw.data_ptr(), _ptr(bias), M, N, K, out.data_ptr(),
                     _native.dtype_code(out_dtype), _ptr(ws), ws_bytes, _native.stream(q.device))
        return out
    if residual.shape != (M, N) or residual.dtype != out_dtype or not residual.is_contiguous():
        raise ValueError(f"residual must be a contiguous [{M}, {N}] {out_dtype} tensor, got "
                         f"{tuple(residual.shape)} {residual.dtype}")
    _native.call("si_gemm_i8_dequant_add", q.data_ptr(), sx.data_ptr(), qweight_nk.data_ptr(),
                 sw.data_ptr(), _ptr(bias), residual.data_ptr(), M, N, K, out.data_ptr(),
                 _native.dtype_code(out_dtype), _ptr(ws), ws_bytes, _native.stream(q.device))
    return out


def weight_quant_i8(w: torch.Tensor) -> Tuple[torch.Tensor, torch.Tensor]:
    """INT8Linear.from_linear's quantization (int8_linear.py:70-74) of an fp32
    ``[N, K]`` weight: (int8 ``[N, K]``, fp32 per-row scale ``[N]``)."""
    _native.require_device(w, "weight_quant_i8")
    wf = w.to(torch.float32).contiguous()
    N, K = wf.shape
    q = torch.empty(N, K, dtype=torch.int8, device=w.device)
    s = torch.empty(N, dtype=torch.float32, device=w.device)
    _native.call("si_weight_quant_i8", wf.data_ptr(), N, K, q.data_ptr(), s.data_ptr(),
                 _native.stream(w.device))
    return q, s
