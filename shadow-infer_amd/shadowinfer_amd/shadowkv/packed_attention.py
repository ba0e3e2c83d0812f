"""Fused dequantize + bidirectional attention over a PackedKVCache.

Replaces the reference's ``k, v = packed.unpack()`` followed by dense
``softmax(q k^T / sqrt(D)) v`` without a mask
(shadowinfer/models/simple_diffusion_llm.py:165-169) with one HIP kernel that
dequantizes packed K/V tiles straight into LDS. Evicted token-heads behave as
in the unpacked tensors: zero keys and values that still take part in the
softmax.
"""

from __future__ import annotations

import math
from typing import Optional

import torch

from .. import _native
from .packed_kv_cache import PackedKVCache


def packed_attention(q: torch.Tensor, cache: PackedKVCache, sm_scale: Optional[float] = None,
                     out_dtype: torch.dtype = torch.float32,
                     token_major: bool = False) -> torch.Tensor:
    """``q`` ``[B, H, S_q, D]`` (bf16 or fp16) against the cache's K/V
    ``[B, H, S_kv, D]``; returns ``[B, H, S_q, D]`` in ``out_dtype`` (fp32 by
    default, the dtype of attention over the fp32 tensors unpack() returns).
    ``token_major=True`` returns ``[B, S_q, H, D]`` instead, written directly
    by the kernel: the ``attn.transpose(1, 2)`` layout an output projection
    reads (models/diffusion_llama.py:390-391)."""
    if q.dim() != 4:
        raise ValueError(f"q must be [batch, heads, seq, dim], got {tuple(q.shape)}")
    B, H, Sq, D = q.shape
    if (B, H, D) != (cache.batch_size, cache.num_heads, cache.head_dim):
        raise ValueError(
            f"q shape {tuple(q.shape)} does not match the cache "
            f"(batch={cache.batch_size}, heads={cache.num_heads}, head_dim={cache.head_dim})")
    if q.dtype not in (torch.bfloat16, torch.float16):
        raise TypeError(f"q must be bfloat16 or float16, got {q.dtype}")
    _native.require_device(q, "packed_attention")
    code, _, table, sdt, group = cache.device_state()
    if code.device != q.device:
        raise ValueError("q and the packed cache live on different devices")
    if sm_scale is None:
        sm_scale = 1.0 / math.sqrt(D)
    qc = q.contiguous()
    shape = (B, Sq, H, D) if token_major else (B, H, Sq, D)
    out = torch.empty(shape, dtype=out_dtype, device=qc.device)
    lists = cache.attention_lists()
    _native.call("si_attn_packed_fwd_built", qc.data_ptr(), _native.dtype_code(q.dtype), B, H,
                 Sq, D, lists.data_ptr(), lists.numel(), table, sdt, cache.seq_len, group,
                 float(sm_scale), out.data_ptr(), _native.dtype_code(out_dtype),
                 1 if token_major else 0, _native.stream(q.device))
    return out
