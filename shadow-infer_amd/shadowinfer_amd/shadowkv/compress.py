"""Plan-driven KV compression fused with the pack
(ShadowKVAgent._compress_kv_with_plan, shadowinfer/shadowkv/shadowkv_agent.py:1698-1809,
followed by PackedKVCache.pack with the same plan).

The reference first builds a dense working copy of K/V (per entry: the fp32
values, the fp16 round trip, or the int8/int4 integer codes cast back to the
input dtype; reuse entries copied from the previous step) and hands the
quantized groups to ``PackedKVCache.pack``. Here one HIP pass
(``si_kv_pack_copy``) reads K/V once and writes both the packed buckets and
the working copy.
"""

from __future__ import annotations

from typing import Any, Dict, Optional, Tuple

import torch

from .packed_kv_cache import PackedKVCache
from .precision_plan import PRECISION_ORDER


def compress_kv_with_plan(
    k_tensor: torch.Tensor,
    v_tensor: torch.Tensor,
    k_prev: Optional[torch.Tensor],
    v_prev: Optional[torch.Tensor],
    plan: Any,
    int4_group_size: int = 16,
    build_scale_map: bool = False,
) -> Dict[str, Any]:
    """Returns ``{"k", "v", "scale_k_map", "scale_v_map", "packed_kv",
    "memory_bytes", "memory_mb"}``: the working copy and scale maps of the
    reference's ``_compress_kv_with_plan`` plus the ``PackedKVCache`` its
    ``group_payload`` would have produced. Errors follow the reference
    (shadowkv_agent.py:1716-1745): plan/tensor shape mismatch, reuse without
    ``v_prev``, previous tensors of another shape and a plan on another device
    type raise ``ValueError``."""
    if k_tensor.dim() != 4:
        raise ValueError(f"k_tensor must be [batch, heads, seq, dim], got {tuple(k_tensor.shape)}")
    B, H, S, D = k_tensor.shape
    if plan.seq_len != S or plan.num_heads != H or v_tensor.shape != k_tensor.shape:
        raise ValueError(
            "PrecisionPlan shape mismatch: plan "
            f"(seq_len={plan.seq_len}, num_heads={plan.num_heads}) vs "
            f"tensor (seq_len={S}, num_heads={H})")
    reuse_active = k_prev is not None and plan.reuse_flat.numel() > 0
    if reuse_active and v_prev is None:
        raise ValueError("v_prev is required when reuse entries are active")
    if reuse_active and (k_prev.shape != k_tensor.shape or v_prev.shape != v_tensor.shape):
        raise ValueError("previous KV tensors must match the current KV shape")
    if plan.codes.device.type != k_tensor.device.type:
        raise ValueError(
            f"PrecisionPlan device ({plan.codes.device}) does not match "
            f"KV device ({k_tensor.device})")
    dev = k_tensor.device
    out_k = torch.empty(k_tensor.shape, dtype=k_tensor.dtype, device=dev)
    out_v = torch.empty(v_tensor.shape, dtype=v_tensor.dtype, device=dev)
    kp = vp = reuse = None
    if reuse_active:
        if k_prev.dtype != k_tensor.dtype or v_prev.dtype != v_tensor.dtype:
            raise ValueError("previous KV tensors must have the current KV dtype")
        kp = k_prev.detach().to(dev).contiguous()
        vp = v_prev.detach().to(dev).contiguous()
        flat = plan.reuse_flat.to(dev)
        reuse = torch.zeros(S * H, dtype=torch.uint8, device=dev)
        reuse[(flat % S) * H + flat // S] = 1  # h*S + t -> entry t*H + h
    cache = PackedKVCache(B, H, S, D, device=dev)
    cache._do_pack(k_tensor, v_tensor, None, group_size=int4_group_size, plan=plan,
                   work_copy=(out_k, out_v, kp, vp, reuse))

    scale_k_map = scale_v_map = None
    if build_scale_map:
        scale_k_map, scale_v_map = _scale_maps(cache, plan, reuse_active)
    return {"k": out_k, "v": out_v, "scale_k_map": scale_k_map, "scale_v_map": scale_v_map,
            "packed_kv": cache, "memory_bytes": cache.memory_bytes(),
            "memory_mb": cache.memory_mb()}


def _scale_maps(cache: PackedKVCache, plan: Any, reuse_active: bool) -> Tuple[dict, dict]:
    """Per entry: None for fp32/fp16, else the entry's scale slice
    ``[1, B, 1]`` (int8) or ``[1, B, G, 1]`` (int4), views of the buckets
    (shadowkv_agent.py:1783-1788); reuse entries are left out."""
    reuse = plan.reuse_set() if reuse_active else set()
    data = cache.packed_data
    B = cache.batch_size
    smk: Dict[Tuple[int, int], Optional[torch.Tensor]] = {}
    smv: Dict[Tuple[int, int], Optional[torch.Tensor]] = {}
    for precision in PRECISION_ORDER:
        entries = plan.groups.get(precision, [])
        if not entries:
            continue
        sk = data[precision]["scale_k"]
        sv = data[precision]["scale_v"]
        if sk is not None and precision == "int4":
            sk = sk.view(len(entries), B, sk.shape[1], 1)
            sv = sv.view(len(entries), B, sv.shape[1], 1)
        for index, entry in enumerate(entries):
            if entry in reuse:
                continue
            smk[entry] = None if sk is None else sk[index:index + 1]
            smv[entry] = None if sv is None else sv[index:index + 1]
    return smk, smv
