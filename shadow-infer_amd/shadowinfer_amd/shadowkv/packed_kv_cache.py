"""PackedKVCache with the reference API
(shadowinfer/shadowkv/packed_kv_cache.py:22-885) on gfx950 HIP kernels.

State of a packed cache on the device:

* ``code``  int8 [S*H]: precision of each token-head (token-major entry id
  ``e = t*H + h``), 4 when absent (evicted or never packed).
* ``slot``  int32 [S*H]: the entry's row in its precision bucket.
* one bucket per present precision, in the reference's exact tensor layouts:
  fp32/fp16 ``k, v [n, B, D]``; int8 ``k, v [n, B, D]`` + ``scale [n, B, 1]``;
  int4 ``k, v [n * ceil(B*D/2)]`` uint8 + ``scale [n*B, G, 1]``.

Within a bucket entries are token-major, as in the reference. Eviction is a
stable compaction, so that order holds after evict; reuse copies rows in
place. The reference's ``packed_data`` dict (with Python ``indices`` lists and
``byte_offsets``) is available as a read-only view built on first access.

Every operation runs on the HIP device of the K/V tensors; CPU tensors raise
RuntimeError (this build has no CPU implementation of the data plane).
"""

from __future__ import annotations

import ctypes
from typing import Any, Dict, List, Optional, Set, Tuple, Union

import numpy as np
import torch

from .. import _native
from .._checks import check_rope_args as _check_rope_args
from ._masks import token_head_mask
from .precision_plan import EVICTED, PRECISION_ORDER, DeviceGrouping, PrecisionPlan

_PREC_INDEX = {name: i for i, name in enumerate(PRECISION_ORDER)}


class PackedKVCache:
    """Byte-level packed KV cache storage with per-token-head precision."""

    PRECISION_BITS = {"fp32": 32, "fp16": 16, "int8": 8, "int4": 4}

    def __init__(self, batch_size: int, num_heads: int, seq_len: int, head_dim: int,
                 device: Any = "cpu"):
        self.batch_size = batch_size
        self.num_heads = num_heads
        self.seq_len = seq_len
        self.head_dim = head_dim
        self.device = device
        self._buckets: Dict[str, Dict[str, Any]] = {}
        self._grouping: Optional[DeviceGrouping] = None
        self._group_size: Optional[int] = None  # effective int4 group
        self._scale_dtype: Optional[torch.dtype] = None
        self._view: Optional[Dict[str, Dict[str, Any]]] = None

    # ------------------------------------------------------------------ pack
    @classmethod
    def pack(cls, k_tensor: torch.Tensor, v_tensor: torch.Tensor,
             precision_map: Optional[Dict[int, Dict[int, str]]], group_size: int = 16,
             plan: Any = None, precomputed: Optional[Dict[str, Any]] = None) -> Dict[str, Any]:
        """packed_kv_cache.py:43-82: returns ``{packed_kv, memory_bytes, memory_mb}``."""
        if k_tensor.dim() != 4:
            raise ValueError(f"k_tensor must be [batch, heads, seq, dim], got {tuple(k_tensor.shape)}")
        batch_size, num_heads, seq_len, head_dim = k_tensor.shape
        cache = cls(batch_size, num_heads, seq_len, head_dim, device=k_tensor.device)
        cache._do_pack(k_tensor, v_tensor, precision_map, group_size=group_size, plan=plan,
                       precomputed=precomputed)
        return {"packed_kv": cache, "memory_bytes": cache.memory_bytes(),
                "memory_mb": cache.memory_mb()}

    @classmethod
    def pack_projection(cls, qkv: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor,
                        batch_size: int, seq_len: int, num_heads: int, head_dim: int,
                        group_size: int, plan: Any) -> "PackedKVCache":
        """The cache ``pack(k, v, None, group_size, plan)`` returns for the
        post-RoPE K and V of an attention layer (models/diffusion_llama.py:362-373),
        read straight from the q|k|v projection ``qkv [B*S, 3*H*D]`` with the
        rotate-half tables ``cos``/``sin`` ``[S, D]`` (si_kv_pack_rope_flat): the
        dense K/V are never written. bf16/fp16, D = 64 or 128."""
        B, S, H, D = batch_size, seq_len, num_heads, head_dim
        # qkv [B*S, 3*H*D] on a GPU, cos/sin [S, D] in its dtype and on its device
        _check_rope_args(qkv, cos, sin, B, S, H, D, "PackedKVCache.pack_projection")
        if plan.seq_len != S or plan.num_heads != H:
            raise ValueError(
                "PrecisionPlan shape mismatch: plan "
                f"(seq_len={plan.seq_len}, num_heads={plan.num_heads}) vs "
                f"tensor (seq_len={S}, num_heads={H})")
        dev = qkv.device
        cache = cls(B, H, S, D, device=dev)
        grouping = plan.device_grouping()
        if grouping.code.device != dev:
            grouping = DeviceGrouping(grouping.code.to(dev), grouping.slot.to(dev),
                                      list(grouping.counts))
        g = group_size if D % group_size == 0 else D
        cache._grouping = grouping
        cache._group_size = g
        cache._scale_dtype = qkv.dtype
        cache._buckets = cache._alloc_buckets(grouping.counts, dev, qkv.dtype)
        cache._view = None
        flat = grouping.flat_lists(S, H)
        counts = (ctypes.c_int64 * 5)(*[int(c) for c in grouping.counts])
        # contiguous copies stay bound until the launch is queued
        src, cos_c, sin_c = qkv.contiguous(), cos.contiguous(), sin.contiguous()
        _native.call("si_kv_pack_rope_flat", src.data_ptr(), cos_c.data_ptr(), sin_c.data_ptr(),
                     _native.dtype_code(qkv.dtype), B, H, S, D, g, grouping.code.data_ptr(),
                     grouping.slot.data_ptr(), _native.table4([f.data_ptr() for f in flat]),
                     counts, cache._bucket_table(), _native.stream(dev))
        return cache

    def _do_pack(self, k_tensor: torch.Tensor, v_tensor: torch.Tensor,
                 precision_map: Optional[Dict[int, Dict[int, str]]], group_size: int = 16,
                 plan: Any = None, precomputed: Optional[Dict[str, Any]] = None,
                 work_copy: Optional[Tuple[Any, ...]] = None) -> None:
        """``work_copy`` = (out_k, out_v, k_prev, v_prev, reuse_u8) makes the same
        pass write the dense working copy of the plan-driven compression
        (``si_kv_pack_copy``)."""
        B, H, S, D = k_tensor.shape
        if plan is not None:
            # packed_kv_cache.py:238-251
            if plan.seq_len != S or plan.num_heads != H:
                raise ValueError(
                    "PrecisionPlan shape mismatch: plan "
                    f"(seq_len={plan.seq_len}, num_heads={plan.num_heads}) vs "
                    f"tensor (seq_len={S}, num_heads={H})")
            if v_tensor.shape != k_tensor.shape:
                raise ValueError("k_tensor and v_tensor must have identical shapes")
            if plan.codes.device.type != k_tensor.device.type:
                raise ValueError(
                    f"PrecisionPlan device ({plan.codes.device}) does not match "
                    f"KV device ({k_tensor.device})")
        elif v_tensor.shape != k_tensor.shape:
            raise ValueError("k_tensor and v_tensor must have identical shapes")
        _native.require_device(k_tensor, "PackedKVCache.pack")
        if v_tensor.device != k_tensor.device:
            raise ValueError("k_tensor and v_tensor must be on the same device")
        if k_tensor.dtype != v_tensor.dtype:
            raise ValueError("k_tensor and v_tensor must have the same dtype")
        dt = _native.dtype_code(k_tensor.dtype)
        dev = k_tensor.device
        k = k_tensor.detach().contiguous()
        v = v_tensor.detach().contiguous()

        if plan is not None:
            grouping = plan.device_grouping()
            if grouping.code.device != dev:
                grouping = DeviceGrouping(grouping.code.to(dev), grouping.slot.to(dev),
                                          list(grouping.counts))
        else:
            codes = _pack_codes_from_map(precision_map or {}, S, H)
            grouping = DeviceGrouping.scan(torch.from_numpy(codes).to(dev))

        g = group_size if D % group_size == 0 else D
        self._grouping = grouping
        self._group_size = g
        self._scale_dtype = k.dtype
        self._buckets = self._alloc_buckets(grouping.counts, dev, k.dtype)
        self._view = None
        if work_copy is None:
            flat = grouping.flat_lists(S, H)
            counts = (ctypes.c_int64 * 5)(*[int(c) for c in grouping.counts])
            _native.call("si_kv_pack_flat", k.data_ptr(), v.data_ptr(), dt, B, H, S, D, g,
                         grouping.code.data_ptr(), grouping.slot.data_ptr(),
                         _native.table4([f.data_ptr() for f in flat]), counts,
                         self._bucket_table(), _native.stream(dev))
        else:
            out_k, out_v, k_prev, v_prev, reuse = work_copy
            _native.call("si_kv_pack_copy", k.data_ptr(), v.data_ptr(), dt, B, H, S, D, g,
                         grouping.code.data_ptr(), grouping.slot.data_ptr(), self._bucket_table(),
                         _native.ptr(k_prev), _native.ptr(v_prev), _native.ptr(reuse),
                         out_k.data_ptr(), out_v.data_ptr(), _native.stream(dev))
        if precomputed:
            self._apply_precomputed(precomputed, grouping.counts)

    def _alloc_buckets(self, counts: List[int], dev: torch.device,
                       scale_dtype: torch.dtype) -> Dict[str, Dict[str, Any]]:
        B, D = self.batch_size, self.head_dim
        g = self._group_size or D
        G = D // g
        out: Dict[str, Dict[str, Any]] = {}
        for p, name in enumerate(PRECISION_ORDER):
            n = int(counts[p])
            if n == 0:
                continue
            if name in ("fp32", "fp16"):
                dtype = torch.float32 if name == "fp32" else torch.float16
                out[name] = {"k": torch.empty((n, B, D), dtype=dtype, device=dev),
                             "v": torch.empty((n, B, D), dtype=dtype, device=dev),
                             "scale_k": None, "scale_v": None}
            elif name == "int8":
                out[name] = {"k": torch.empty((n, B, D), dtype=torch.int8, device=dev),
                             "v": torch.empty((n, B, D), dtype=torch.int8, device=dev),
                             "scale_k": torch.empty((n, B, 1), dtype=scale_dtype, device=dev),
                             "scale_v": torch.empty((n, B, 1), dtype=scale_dtype, device=dev)}
            else:
                rb = (B * D + 1) // 2
                out[name] = {"k": torch.empty(n * rb, dtype=torch.uint8, device=dev),
                             "v": torch.empty(n * rb, dtype=torch.uint8, device=dev),
                             "scale_k": torch.empty((n * B, G, 1), dtype=scale_dtype, device=dev),
                             "scale_v": torch.empty((n * B, G, 1), dtype=scale_dtype, device=dev)}
        return out

    def _bucket_table(self, buckets: Optional[Dict[str, Dict[str, Any]]] = None):
        buckets = self._buckets if buckets is None else buckets
        ptrs: List[Optional[int]] = [None] * 16
        for name, data in buckets.items():
            p = _PREC_INDEX[name]
            for j, key in enumerate(("k", "v", "scale_k", "scale_v")):
                t = data.get(key)
                ptrs[4 * p + j] = None if t is None else t.data_ptr()
        return _native.table16(ptrs)

    def _apply_precomputed(self, precomputed: Dict[str, Any], counts: List[int]) -> None:
        """Use tensors handed over by the compression stage
        (packed_kv_cache.py:263-330) in place of the freshly packed ones."""
        from ..kernels import _pack_int4  # noqa: F401  (device helpers)
        from ..utils.quantization import Quantizer
        B, D = self.batch_size, self.head_dim
        g = self._group_size
        G = D // g
        for name, pre in precomputed.items():
            if name not in self._buckets or pre is None:
                continue
            n = int(counts[_PREC_INDEX[name]])
            data = self._buckets[name]
            if name in ("fp32", "fp16", "int8"):
                for key, src in (("k", "qk"), ("v", "qv"), ("scale_k", "scale_k"),
                                 ("scale_v", "scale_v")):
                    if data.get(key) is not None and pre.get(src) is not None:
                        data[key] = pre[src]
                continue
            if pre.get("qk") is not None and pre.get("scale_k") is not None:
                qk = pre["qk"].reshape(n, B, G, g)
                qv = pre["qv"].reshape(n, B, G, g)
                sk = pre["scale_k"].reshape(n, B, G, 1)
                sv = pre["scale_v"].reshape(n, B, G, 1)
            elif pre.get("k_group") is not None:
                qk, sk = Quantizer.quantize_int4(pre["k_group"], group_size=g)
                qv, sv = Quantizer.quantize_int4(pre["v_group"], group_size=g)
            else:
                continue
            data["k"] = _pack_rows(qk.reshape(n, -1))
            data["v"] = _pack_rows(qv.reshape(n, -1))
            data["scale_k"] = sk.reshape(-1, G, 1)
            data["scale_v"] = sv.reshape(-1, G, 1)

    # ---------------------------------------------------------------- unpack
    def unpack(self) -> Tuple[torch.Tensor, torch.Tensor]:
        """packed_kv_cache.py:535-577: fp32 ``[B, H, S, D]``, absent entries 0."""
        shape = (self.batch_size, self.num_heads, self.seq_len, self.head_dim)
        if self._grouping is None:
            k_out = torch.zeros(shape, dtype=torch.float32, device=self.device)
            return k_out, torch.zeros_like(k_out)
        dev = self._grouping.code.device
        k_out = torch.empty(shape, dtype=torch.float32, device=dev)
        v_out = torch.empty(shape, dtype=torch.float32, device=dev)
        if k_out.numel():
            gr = self._grouping
            flat = gr.flat_lists(self.seq_len, self.num_heads)
            counts = (ctypes.c_int64 * 5)(*[int(c) for c in gr.counts])
            _native.call("si_kv_unpack_flat", gr.code.data_ptr(), gr.slot.data_ptr(),
                         _native.table4([f.data_ptr() for f in flat]), counts,
                         self._bucket_table(), _native.dtype_code(self._scale_dtype), *shape,
                         self._group_size, k_out.data_ptr(), v_out.data_ptr(),
                         _native.stream(dev))
        return k_out, v_out

    def unpack_reference(self) -> Tuple[torch.Tensor, torch.Tensor]:
        """Bucket-by-bucket unpack (packed_kv_cache.py:579-634) through the
        standalone Quantizer kernels and index scatter; an independent path
        to cross-check :meth:`unpack`."""
        from ..utils.quantization import Quantizer
        B, H, S, D = self.batch_size, self.num_heads, self.seq_len, self.head_dim
        dev = self._grouping.code.device if self._grouping is not None else self.device
        k_out = torch.zeros((B, H, S, D), dtype=torch.float32, device=dev)
        v_out = torch.zeros_like(k_out)
        if self._grouping is None:
            return k_out, v_out
        for name, data in self._buckets.items():
            entries = self._bucket_entries(name)
            n = entries.numel()
            t = torch.div(entries, H, rounding_mode="floor")
            h = torch.remainder(entries, H)
            for key, out in (("k", k_out), ("v", v_out)):
                if name in ("fp32", "fp16"):
                    vals = data[key].float()
                elif name == "int8":
                    vals = Quantizer.dequantize_int8(data[key], data["scale_" + key])
                else:
                    g = self._group_size
                    codes = Quantizer.unpack_int4(data[key], data[key].numel() * 2)
                    codes = codes.reshape(n, -1)[:, : B * D].reshape(n, B, D // g, g)
                    vals = Quantizer.dequantize_int4(
                        codes.contiguous(), data["scale_" + key].reshape(n, B, D // g, 1))
                    vals = vals.reshape(n, B, D)
                out[:, h, t, :] = vals.reshape(n, B, D).permute(1, 0, 2)
        return k_out, v_out

    # --------------------------------------------------------------- accounting
    def memory_bytes(self) -> int:
        """packed_kv_cache.py:658-660, 856-863."""
        return self._compute_data_bytes()

    def memory_mb(self) -> float:
        return self.memory_bytes() / (1024.0 * 1024.0)

    def _compute_data_bytes(self) -> int:
        total = 0
        for data in self._buckets.values():
            for key in ("k", "v", "scale_k", "scale_v"):
                t = data.get(key)
                if t is not None:
                    total += t.numel() * t.element_size()
        return total

    def data_plane_bytes(self) -> int:
        return self._compute_data_bytes()

    def num_entries(self) -> int:
        if self._grouping is None:
            return 0
        return int(sum(self._grouping.counts[:4]))

    def resident_bytes(self) -> int:
        """packed_kv_cache.py:869-878: data bytes + 48 per present entry."""
        if not self._buckets:
            return 0
        return self._compute_data_bytes() + 48 * self.num_entries()

    # ----------------------------------------------------------------- evict
    def evict(self, token_head_set: Union[Set[Tuple[int, int]], torch.Tensor]) -> int:
        """Stable in-bucket compaction (packed_kv_cache.py:666-740); returns the
        number of entries removed. Absent entries are never resurrected.
        Besides the reference's set of ``(t, h)`` pairs, a bool/uint8 ``[S, H]``
        tensor marking the entries to evict is accepted (no host loop)."""
        if torch.is_tensor(token_head_set):
            if tuple(token_head_set.shape) not in ((self.seq_len, self.num_heads),
                                                   (self.seq_len * self.num_heads,)):
                raise ValueError(
                    f"evict mask tensor must be [S, H], got {tuple(token_head_set.shape)}")
            if not self._buckets:
                return 0
            mask = token_head_set.reshape(-1).to(device=self._grouping.code.device,
                                                 dtype=torch.uint8).contiguous()
        else:
            if not token_head_set or not self._buckets:
                return 0
            mask = self._entry_mask(token_head_set, is_dict=False)
            if mask is None:
                return 0
        old = self._grouping
        dev = old.code.device
        S, H = self.seq_len, self.num_heads
        mask = mask.to(dev)
        code, slot, (chunk_counts, chunk_bits), counts = old.evict_count(mask, S, H)
        removed = int(sum(old.counts[:4]) - sum(counts[:4]))
        if removed == 0:
            return 0
        new_buckets: Dict[str, Dict[str, Any]] = {}
        changed: Dict[str, Dict[str, Any]] = {}
        fresh = self._alloc_buckets(counts, dev, self._scale_dtype)
        for name in PRECISION_ORDER:
            p = _PREC_INDEX[name]
            if counts[p] == 0:
                continue
            if counts[p] == old.counts[p]:
                new_buckets[name] = self._buckets[name]  # untouched (reference keeps it)
            else:
                new_buckets[name] = fresh[name]
                changed[name] = fresh[name]
        flat = [torch.empty(c, dtype=torch.long, device=dev) for c in counts[:4]]
        _native.call("si_kv_evict_flat", _native.table4([f.data_ptr() for f in old.flat_lists(S, H)]),
                     (ctypes.c_int64 * 4)(*old.counts[:4]), chunk_counts.data_ptr(),
                     chunk_bits.data_ptr(), S, H, self._bucket_table(), _native.table4([f.data_ptr() for f in flat]),
                     (ctypes.c_int64 * 4)(*counts[:4]), self._bucket_table(changed), slot.data_ptr(),
                     self.batch_size, self.head_dim, self._group_size,
                     _native.dtype_code(self._scale_dtype), _native.stream(dev))
        self._buckets = new_buckets
        self._grouping = DeviceGrouping(code, slot, counts, flat)
        self._view = None
        return removed

    def _entry_mask(self, items, is_dict: bool) -> Optional[torch.Tensor]:
        """uint8 [S*H] host mask of the in-range (t, h) pairs of the
        reference's set (or, with ``is_dict``, of the dict's truthy keys),
        built in one pass; None when no pair is in range."""
        mask = token_head_mask(items, self.seq_len, self.num_heads, is_dict=is_dict)
        return None if mask is None else torch.from_numpy(mask)

    def _precision_for(self, token_idx: int, head_idx: int) -> str:
        """packed_kv_cache.py:742-751: precision of an entry, EVICTED if absent."""
        if self._grouping is None or not (0 <= token_idx < self.seq_len
                                          and 0 <= head_idx < self.num_heads):
            return EVICTED
        c = int(self._grouping.code[token_idx * self.num_heads + head_idx].item())
        return PRECISION_ORDER[c] if 0 <= c < 4 else EVICTED

    # ----------------------------------------------------------------- reuse
    def apply_reuse_mask(self, kv_previous_packed: "PackedKVCache",
                         reuse_mask: Union[Dict[Tuple[int, int], bool], torch.Tensor],
                         return_stats: bool = False) -> Optional[Dict[str, int]]:
        """packed_kv_cache.py:753-854. ``reuse_mask`` is the reference's dict
        ``(t, h) -> bool``; a bool/uint8 tensor ``[S, H]`` is accepted too."""
        prev = kv_previous_packed
        if (self.batch_size != prev.batch_size or self.num_heads != prev.num_heads
                or self.head_dim != prev.head_dim):
            raise ValueError(
                "packed cache shape mismatch for reuse: "
                f"current=({self.batch_size},{self.num_heads},{self.head_dim}) "
                f"previous=({prev.batch_size},{prev.num_heads},{prev.head_dim})")
        if "int4" in self._buckets and "int4" in prev._buckets and \
                self._group_size != prev._group_size:
            raise ValueError(
                "INT4 group_size mismatch for reuse: "
                f"current={self._group_size} previous={prev._group_size}")
        stats = {"applied": 0, "skipped_precision": 0}
        empty_mask = (reuse_mask is None or (isinstance(reuse_mask, dict) and not reuse_mask)
                      or (torch.is_tensor(reuse_mask) and reuse_mask.numel() == 0))
        if empty_mask or not prev._buckets or not self._buckets:
            return stats if return_stats else None
        quantized = [n for n in ("int8", "int4") if n in self._buckets and n in prev._buckets]
        if quantized and self._scale_dtype != prev._scale_dtype:
            raise RuntimeError(
                f"scale dtype mismatch for reuse: current={self._scale_dtype} "
                f"previous={prev._scale_dtype}")
        dev = self._grouping.code.device
        if prev._grouping.code.device != dev:
            raise ValueError("previous packed cache lives on another device")
        if torch.is_tensor(reuse_mask):
            if tuple(reuse_mask.shape) not in ((self.seq_len, self.num_heads),
                                               (self.seq_len * self.num_heads,)):
                raise ValueError(f"reuse mask tensor must be [S, H], got {tuple(reuse_mask.shape)}")
            mask = reuse_mask.reshape(-1).to(device=dev, dtype=torch.uint8).contiguous()
        else:
            host = self._entry_mask(reuse_mask, is_dict=True)
            if host is None:
                return stats if return_stats else None
            mask = host.to(dev)
        stats_dev = torch.zeros(2, dtype=torch.int64, device=dev) if return_stats else None
        grouping = self._grouping
        flat = grouping.flat_lists(self.seq_len, self.num_heads)
        _native.call("si_kv_reuse_flat", _native.table4([f.data_ptr() for f in flat]),
                     (ctypes.c_int64 * 5)(*grouping.counts), self._bucket_table(), self.seq_len,
                     prev._grouping.code.data_ptr(), prev._grouping.slot.data_ptr(),
                     prev._bucket_table(), prev.seq_len, mask.data_ptr(), self.num_heads,
                     self.batch_size, self.head_dim, self._group_size,
                     _native.dtype_code(self._scale_dtype), _native.ptr(stats_dev),
                     _native.stream(dev))
        self._view = None
        if not return_stats:
            return None
        applied, skipped = (int(x) for x in stats_dev.tolist())
        return {"applied": applied, "skipped_precision": skipped}

    # ------------------------------------------------------------ dict view
    def _bucket_entries(self, name: str) -> torch.Tensor:
        """Token-major entry ids (int64, on the device) of one bucket, in slot order."""
        code = self._grouping.code
        return (code == _PREC_INDEX[name]).nonzero().reshape(-1)

    @property
    def packed_data(self) -> Dict[str, Dict[str, Any]]:
        """The reference's per-precision dict (packed_kv_cache.py:143-218):
        ``k, v, scale_k, scale_v`` are the live bucket tensors; ``indices``
        (and for int4 ``byte_offsets``, ``group_size``, ``num_groups``) are
        built on first access. Read-only: mutate through the methods."""
        if self._view is None:
            view: Dict[str, Dict[str, Any]] = {}
            H = self.num_heads
            for name in PRECISION_ORDER:
                if name not in self._buckets:
                    continue
                data = self._buckets[name]
                e = self._bucket_entries(name).to("cpu")
                indices = list(zip(torch.div(e, H, rounding_mode="floor").tolist(),
                                   torch.remainder(e, H).tolist()))
                entry = dict(data)
                entry["indices"] = indices
                if name == "int4":
                    n = len(indices)
                    rb = data["k"].numel() // max(n, 1)
                    entry["byte_offsets"] = [(i * rb, (i + 1) * rb, i * rb, (i + 1) * rb)
                                             for i in range(n)]
                    entry["group_size"] = self._group_size
                    entry["num_groups"] = self.head_dim // self._group_size
                view[name] = entry
            self._view = view
        return self._view

    def device_state(self):
        """(code, slot, bucket pointer table, scale dtype code, int4 group) for
        kernels that read the packed cache directly (fused attention)."""
        if self._grouping is None:
            raise ValueError("cache holds no packed data")
        return (self._grouping.code, self._grouping.slot, self._bucket_table(),
                _native.dtype_code(self._scale_dtype), self._group_size)

    def attention_lists(self) -> torch.Tensor:
        """The fused attention's per-head slot lists for this cache's grouping
        (built once per plan and shared by every cache packed with it)."""
        if self._grouping is None:
            raise ValueError("cache holds no packed data")
        return self._grouping.attn_lists(self.seq_len, self.num_heads)

    def __repr__(self) -> str:
        return (f"PackedKVCache(batch={self.batch_size}, heads={self.num_heads}, "
                f"seq_len={self.seq_len}, head_dim={self.head_dim}, "
                f"memory_mb={self.memory_mb():.2f})")


def _pack_codes_from_map(precision_map: Dict[int, Dict[int, str]], S: int, H: int) -> np.ndarray:
    """Grouping rules of _do_pack (packed_kv_cache.py:119-127): missing -> fp16,
    ``evicted`` -> absent, names outside fp32/fp16/int8/int4 -> fp16."""
    codes = np.full(S * H, 1, dtype=np.int8)
    for t, row in precision_map.items():
        if not (isinstance(t, (int, np.integer)) and 0 <= t < S):
            continue
        for h, name in row.items():
            if not (isinstance(h, (int, np.integer)) and 0 <= h < H):
                continue
            p = name.lower()
            codes[t * H + h] = 4 if p == EVICTED else _PREC_INDEX.get(p, 1)
    return codes


def _pack_rows(q: torch.Tensor) -> torch.Tensor:
    """Rows of int4 codes -> rows of bytes (si_int4_pack_rows), flattened."""
    q = q.to(torch.int8).contiguous()
    n, L = q.shape
    out = torch.empty(n * ((L + 1) // 2), dtype=torch.uint8, device=q.device)
    if n and L:
        _native.call("si_int4_pack_rows", q.data_ptr(), n, L, out.data_ptr(),
                     _native.stream(q.device))
    return out
