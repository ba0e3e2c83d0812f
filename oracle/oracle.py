"""Oracle for the quantized KV / INT8 FFN data plane.

TEST INFRASTRUCTURE ONLY: this module is the checker. Only ``tests/``,
``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of ``bench.py`` may
import it. The product package never imports, calls or links anything here.

Layout of the oracle:

* ``si_oracle.c`` holds the bit-level arithmetic (dtype rounding, int8/int4
  quantization, int4 nibble packing, int8 GEMM and its epilogue, dense
  attention in double precision). Each routine cites the reference line it
  restates.
* This file holds the structure the reference builds around that arithmetic
  (precision grouping, bucket order, eviction compaction, reuse copies, byte
  accounting) in numpy, and loads the C part through ctypes.

Array conventions: fp32 values are ``np.float32``; fp16 and bf16 values are
``np.uint16`` bit patterns tagged with a dtype code (``F32``/``F16``/``BF16``).
Bucket arrays have the exact shapes of the reference's ``packed_data`` tensors.
"""

from __future__ import annotations

import ctypes
import hashlib
import os
import struct
import subprocess
from typing import Dict, Iterable, List, Optional, Tuple

import numpy as np

F32, F16, BF16 = 0, 1, 2
PRECISIONS = ("fp32", "fp16", "int8", "int4")
CODES = {"fp32": 0, "fp16": 1, "int8": 2, "int4": 3, "evicted": 4}

_HERE = os.path.dirname(os.path.abspath(__file__))
_SRC = os.path.join(_HERE, "si_oracle.c")
_LIB_PATH = os.path.join(_HERE, "_build", "libsi_oracle.so")
_lib = None


def build(force: bool = False) -> str:
    """Compile ``si_oracle.c`` with gcc into ``oracle/_build/libsi_oracle.so``."""
    if force or not os.path.exists(_LIB_PATH) or (
        os.path.getmtime(_LIB_PATH) < os.path.getmtime(_SRC)
    ):
        os.makedirs(os.path.dirname(_LIB_PATH), exist_ok=True)
        tmp = _LIB_PATH + ".tmp%d" % os.getpid()
        subprocess.check_call(
            ["gcc", "-O2", "-fPIC", "-shared", "-ffp-contract=off", "-fno-fast-math",
             "-std=c11", _SRC, "-o", tmp, "-lm"]
        )
        os.replace(tmp, _LIB_PATH)
    return _LIB_PATH


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        _lib = ctypes.CDLL(build())
        vp, i64, i32 = ctypes.c_void_p, ctypes.c_int64, ctypes.c_int
        sig = {
            "or_quant_rows_i8": [vp, i32, i64, i64, vp, vp],
            "or_quant_rows_i4": [vp, i32, i64, i64, i64, vp, vp],
            "or_pack_int4_rows": [vp, i64, i64, vp],
            "or_unpack_int4_rows": [vp, i64, i64, i64, vp],
            "or_dequant_rows": [vp, vp, i32, i64, i64, i64, vp],
            "or_convert": [vp, i32, i64, vp, i32],
            "or_weight_quant_i8": [vp, i64, i64, vp, vp],
            "or_act_quant_i8": [vp, i32, i64, i64, vp, vp],
            "or_gemm_i8": [vp, vp, i64, i64, i64, vp],
            "or_int8_epilogue": [vp, vp, vp, vp, i64, i64, vp, i32],
            "or_attention": [vp, vp, vp, i64, i64, i64, i64, ctypes.c_double, vp, vp],
            "or_kv_sensitivity": [vp, vp, i32, i64, i64, i64, i64, vp],
        }
        for name, args in sig.items():
            fn = getattr(_lib, name)
            fn.argtypes = args
            fn.restype = None
        for name, ret, args in (
            ("or_f32_to_bf16", ctypes.c_uint16, [ctypes.c_float]),
            ("or_bf16_to_f32", ctypes.c_float, [ctypes.c_uint16]),
            ("or_f32_to_f16", ctypes.c_uint16, [ctypes.c_float]),
            ("or_f16_to_f32", ctypes.c_float, [ctypes.c_uint16]),
        ):
            fn = getattr(_lib, name)
            fn.argtypes = args
            fn.restype = ret
    return _lib


def _p(a: np.ndarray):
    assert a.flags["C_CONTIGUOUS"]
    return a.ctypes.data_as(ctypes.c_void_p)


def _np_dtype(dt: int):
    return np.float32 if dt == F32 else np.uint16


# --------------------------------------------------------------------------
# dtype helpers
# --------------------------------------------------------------------------

def to_f32(x: np.ndarray, dt: int) -> np.ndarray:
    """Widen fp32/fp16/bf16 bit patterns to fp32 (exact)."""
    x = np.ascontiguousarray(x)
    if dt == F32:
        return x.astype(np.float32, copy=True)
    out = np.empty(x.shape, np.float32)
    lib().or_convert(_p(x), dt, x.size, _p(out), F32)
    return out


def from_f32(x: np.ndarray, dt: int) -> np.ndarray:
    """Round fp32 values to dtype ``dt`` (RNE); fp16/bf16 come back as uint16 bits."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    if dt == F32:
        return x.copy()
    out = np.empty(x.shape, np.uint16)
    lib().or_convert(_p(x), F32, x.size, _p(out), dt)
    return out


def convert(x: np.ndarray, src: int, dst: int) -> np.ndarray:
    """``Tensor.to(dst)`` from ``src``: widen to fp32 exactly, round once to ``dst``."""
    return from_f32(to_f32(x, src), dst)


# --------------------------------------------------------------------------
# Quantizer (shadowinfer/utils/quantization.py)
# --------------------------------------------------------------------------

def quant_rows_i8(x: np.ndarray, dt: int) -> Tuple[np.ndarray, np.ndarray]:
    """quantize_int8 over the last dim (quantization.py:120-142).

    Returns ``(q [..., D] int8, scale [..., 1] in dtype dt)``.
    """
    x = np.ascontiguousarray(x)
    D = x.shape[-1]
    rows = x.size // D if D else 0
    q = np.empty(x.shape, np.int8)
    scale = np.empty(x.shape[:-1] + (1,), _np_dtype(dt))
    if rows:
        lib().or_quant_rows_i8(_p(x), dt, rows, D, _p(q), _p(scale))
    return q, scale


def quant_rows_i4(x: np.ndarray, dt: int, group_size: int) -> Tuple[np.ndarray, np.ndarray]:
    """quantize_int4 (quantization.py:144-178).

    Returns ``(q [..., G, g] int8, scale [..., G, 1] in dtype dt)``.
    """
    x = np.ascontiguousarray(x)
    D = x.shape[-1]
    if D % group_size:
        raise ValueError("last dim must be divisible by group_size")
    G = D // group_size
    rows = x.size // D if D else 0
    q = np.empty(x.shape[:-1] + (G, group_size), np.int8)
    scale = np.empty(x.shape[:-1] + (G, 1), _np_dtype(dt))
    if rows:
        lib().or_quant_rows_i4(_p(x), dt, rows, D, group_size, _p(q), _p(scale))
    return q, scale


def pack_int4_rows(q: np.ndarray) -> np.ndarray:
    """_pack_int4_rows (packed_kv_cache.py:367-388): ``[n, ...] -> [n, ceil(L/2)]``."""
    n = q.shape[0]
    rows = np.ascontiguousarray(q.reshape(n, -1)) if n else q.reshape(0, 0)
    L = rows.shape[1]
    out = np.empty((n, (L + 1) // 2), np.uint8)
    if n and L:
        lib().or_pack_int4_rows(_p(rows), n, L, _p(out))
    return out


def pack_int4_flat(q: np.ndarray) -> np.ndarray:
    """Quantizer.pack_int4 / kernels._pack_int4 on a flat tensor (quantization.py:248-277)."""
    flat = np.ascontiguousarray(q.reshape(1, -1))
    if flat.size == 0:
        return np.empty(0, np.uint8)
    return pack_int4_rows(flat).reshape(-1)


def unpack_int4_rows(packed: np.ndarray, L: int) -> np.ndarray:
    """Inverse of :func:`pack_int4_rows`: ``[n, rb] -> [n, L]`` int8 codes."""
    packed = np.ascontiguousarray(packed)
    n, rb = packed.shape
    out = np.empty((n, L), np.int8)
    if n and L:
        lib().or_unpack_int4_rows(_p(packed), n, rb, L, _p(out))
    return out


def dequant_rows(q: np.ndarray, scale: np.ndarray, scale_dt: int, group: int) -> np.ndarray:
    """float(q) * float(scale) with one scale per ``group`` trailing values."""
    q = np.ascontiguousarray(q)
    scale = np.ascontiguousarray(scale)
    D = q.shape[-1]
    rows = q.size // D if D else 0
    out = np.empty(q.shape, np.float32)
    if rows:
        lib().or_dequant_rows(_p(q), _p(scale), scale_dt, rows, D, group, _p(out))
    return out


# --------------------------------------------------------------------------
# PrecisionPlan (shadowinfer/shadowkv/precision_plan.py)
# --------------------------------------------------------------------------

def map_to_codes(precision_map: Dict[int, Dict[int, str]], seq_len: int, num_heads: int,
                 strict: bool = True) -> np.ndarray:
    """precision_plan.py:30-55: missing -> fp16; unknown -> ValueError or fp16."""
    codes = np.empty((seq_len, num_heads), np.int8)
    for t in range(seq_len):
        row = precision_map.get(t, {})
        for h in range(num_heads):
            raw = row.get(h, "fp16")
            name = raw.lower() if isinstance(raw, str) else raw
            if name not in CODES:
                if strict:
                    raise ValueError(f"Unsupported precision: {raw}")
                name = "fp16"
            codes[t, h] = CODES[name]
    return codes


def pack_map_to_codes(precision_map: Dict[int, Dict[int, str]], seq_len: int,
                      num_heads: int) -> np.ndarray:
    """Grouping of PackedKVCache._do_pack (packed_kv_cache.py:119-127):
    ``evicted`` -> 4, names outside fp32/fp16/int8/int4 -> fp16."""
    codes = np.empty((seq_len, num_heads), np.int8)
    for t in range(seq_len):
        row = precision_map.get(t, {})
        for h in range(num_heads):
            name = row.get(h, "fp16").lower()
            if name == "evicted":
                codes[t, h] = 4
            else:
                codes[t, h] = CODES.get(name, 1) if name in PRECISIONS else 1
    return codes


def plan_from_codes(codes: np.ndarray, reuse_mask: Optional[dict] = None) -> dict:
    """PrecisionPlan.from_codes (precision_plan.py:113-177) + _fingerprint (179-190)."""
    codes = np.ascontiguousarray(codes, dtype=np.int8)
    S, H = codes.shape
    flat = codes.reshape(-1).astype(np.int64)
    groups: Dict[str, List[Tuple[int, int]]] = {p: [] for p in PRECISIONS}
    flat_indices: Dict[str, np.ndarray] = {}
    evicted: List[Tuple[int, int]] = []
    for code, name in ((0, "fp32"), (1, "fp16"), (2, "int8"), (3, "int4"), (4, "evicted")):
        sel = np.nonzero(flat == code)[0]
        t = sel // H
        h = sel % H
        entries = list(zip(t.tolist(), h.tolist()))
        if name == "evicted":
            evicted = entries
        else:
            groups[name] = entries
            flat_indices[name] = (h * S + t).astype(np.int64)
    reuse_entries: List[Tuple[int, int]] = []
    if reuse_mask:
        reuse_entries = sorted(
            (int(t), int(h)) for (t, h), flag in reuse_mask.items()
            if flag and 0 <= t < S and 0 <= h < H
        )
    reuse_flat = np.array([h * S + t for t, h in reuse_entries], np.int64)
    digest = hashlib.sha256()
    digest.update(struct.pack("<QQ", S, H))
    digest.update(codes.tobytes())
    digest.update(reuse_flat.astype("<i8").tobytes())
    return {
        "seq_len": S, "num_heads": H, "codes": codes, "groups": groups,
        "flat_indices": flat_indices, "evicted_entries": evicted,
        "reuse_entries": reuse_entries, "reuse_flat": reuse_flat,
        "fingerprint": digest.hexdigest(),
    }


# --------------------------------------------------------------------------
# PackedKVCache (shadowinfer/shadowkv/packed_kv_cache.py)
# --------------------------------------------------------------------------

class OracleCache:
    """Numpy mirror of a PackedKVCache: ``packed_data`` holds arrays in the
    reference's tensor shapes; ``scale_dt`` is the dtype of the stored scales."""

    def __init__(self, B: int, H: int, S: int, D: int, scale_dt: int):
        self.batch_size, self.num_heads, self.seq_len, self.head_dim = B, H, S, D
        self.scale_dt = scale_dt
        self.packed_data: Dict[str, dict] = {}

    def memory_bytes(self) -> int:
        """_compute_data_bytes (packed_kv_cache.py:856-863)."""
        total = 0
        for data in self.packed_data.values():
            for key in ("k", "v", "scale_k", "scale_v"):
                arr = data.get(key)
                if arr is not None:
                    total += arr.nbytes
        return total

    def resident_bytes(self) -> int:
        """packed_kv_cache.py:869-878: data bytes + 48 per entry."""
        if not self.packed_data:
            return 0
        n = sum(len(d["indices"]) for d in self.packed_data.values())
        return self.memory_bytes() + 48 * n


def kv_pack(k: np.ndarray, v: np.ndarray, dt: int, codes: np.ndarray,
            group_size: int = 16) -> OracleCache:
    """_do_pack_with_plan (packed_kv_cache.py:222-365) with plan = from_codes(codes).

    ``k``/``v`` are ``[B,H,S,D]`` in dtype ``dt`` (float32 or uint16 bits).
    """
    B, H, S, D = k.shape
    plan = plan_from_codes(codes)
    cache = OracleCache(B, H, S, D, dt)
    k_flat = k.reshape(B, H * S, D)
    v_flat = v.reshape(B, H * S, D)
    for prec in PRECISIONS:
        entries = plan["groups"][prec]
        if not entries:
            continue
        flat = plan["flat_indices"][prec]
        ks = np.ascontiguousarray(k_flat[:, flat, :].transpose(1, 0, 2))
        vs = np.ascontiguousarray(v_flat[:, flat, :].transpose(1, 0, 2))
        if prec in ("fp32", "fp16"):
            dst = F32 if prec == "fp32" else F16
            cache.packed_data[prec] = {
                "k": convert(ks, dt, dst), "v": convert(vs, dt, dst),
                "scale_k": None, "scale_v": None, "indices": list(entries),
            }
        elif prec == "int8":
            qk, sk = quant_rows_i8(ks, dt)
            qv, sv = quant_rows_i8(vs, dt)
            cache.packed_data[prec] = {
                "k": qk, "v": qv, "scale_k": sk, "scale_v": sv, "indices": list(entries),
            }
        else:
            g = group_size if D % group_size == 0 else D
            G = D // g
            qk, sk = quant_rows_i4(ks, dt, g)
            qv, sv = quant_rows_i4(vs, dt, g)
            krows = pack_int4_rows(qk)
            vrows = pack_int4_rows(qv)
            rb = krows.shape[1]
            n = len(entries)
            cache.packed_data[prec] = {
                "k": krows.reshape(-1), "v": vrows.reshape(-1),
                "scale_k": sk.reshape(-1, G, 1), "scale_v": sv.reshape(-1, G, 1),
                "indices": list(entries),
                "byte_offsets": [(i * rb, (i + 1) * rb, i * rb, (i + 1) * rb) for i in range(n)],
                "group_size": g, "num_groups": G,
            }
    return cache


def _bucket_values(cache: OracleCache, prec: str, data: dict, key: str) -> np.ndarray:
    """Dequantized ``[n, B, D]`` fp32 values of one bucket tensor."""
    B, D = cache.batch_size, cache.head_dim
    n = len(data["indices"])
    if prec == "fp32":
        return data[key].astype(np.float32)
    if prec == "fp16":
        return to_f32(data[key], F16)
    scale = data["scale_" + key]
    if prec == "int8":
        return dequant_rows(data[key], scale, cache.scale_dt, D)
    # int4: _dequantize_int4_bucket (packed_kv_cache.py:636-656)
    rows = data[key].reshape(n, -1)
    codes = unpack_int4_rows(rows, B * D).reshape(n, B, D)
    return dequant_rows(codes, scale.reshape(n, B, -1), cache.scale_dt,
                        data["group_size"]).reshape(n, B, D)


def kv_unpack(cache: OracleCache) -> Tuple[np.ndarray, np.ndarray]:
    """unpack (packed_kv_cache.py:535-577): zero fp32 [B,H,S,D], scatter buckets."""
    B, H, S, D = cache.batch_size, cache.num_heads, cache.seq_len, cache.head_dim
    k_out = np.zeros((B, H, S, D), np.float32)
    v_out = np.zeros((B, H, S, D), np.float32)
    for prec, data in cache.packed_data.items():
        idx = data["indices"]
        if not idx:
            continue
        t = np.array([e[0] for e in idx], np.int64)
        h = np.array([e[1] for e in idx], np.int64)
        k_out[:, h, t, :] = _bucket_values(cache, prec, data, "k").transpose(1, 0, 2)
        v_out[:, h, t, :] = _bucket_values(cache, prec, data, "v").transpose(1, 0, 2)
    return k_out, v_out


def kv_evict(cache: OracleCache, token_head_set: Iterable[Tuple[int, int]]) -> int:
    """evict (packed_kv_cache.py:666-740): stable in-bucket compaction."""
    evict_set = set(token_head_set)
    if not evict_set or not cache.packed_data:
        return 0
    B = cache.batch_size
    removed = 0
    for prec in list(cache.packed_data.keys()):
        data = cache.packed_data[prec]
        idx = data["indices"]
        keep_pos = [i for i, e in enumerate(idx) if e not in evict_set]
        removed += len(idx) - len(keep_pos)
        if len(keep_pos) == len(idx):
            continue
        if not keep_pos:
            del cache.packed_data[prec]
            continue
        keep = np.array(keep_pos, np.int64)
        n = len(idx)
        if prec in ("fp32", "fp16", "int8"):
            for key in ("k", "v", "scale_k", "scale_v"):
                if data.get(key) is not None:
                    data[key] = np.ascontiguousarray(data[key][keep])
        else:
            G = data["num_groups"]
            rb = data["k"].size // n
            for key in ("k", "v"):
                data[key] = np.ascontiguousarray(data[key].reshape(n, rb)[keep].reshape(-1))
            for key in ("scale_k", "scale_v"):
                data[key] = np.ascontiguousarray(
                    data[key].reshape(n, B, G, 1)[keep].reshape(-1, G, 1))
            data["byte_offsets"] = [(i * rb, (i + 1) * rb, i * rb, (i + 1) * rb)
                                    for i in range(len(keep_pos))]
        data["indices"] = [idx[i] for i in keep_pos]
    return removed


def kv_apply_reuse_mask(cache: OracleCache, prev: OracleCache, reuse_mask: dict) -> dict:
    """apply_reuse_mask (packed_kv_cache.py:753-854), returning the stats dict."""
    if (cache.batch_size, cache.num_heads, cache.head_dim) != (
            prev.batch_size, prev.num_heads, prev.head_dim):
        raise ValueError("packed cache shape mismatch for reuse")
    cur4 = cache.packed_data.get("int4")
    prev4 = prev.packed_data.get("int4")
    if cur4 is not None and prev4 is not None and cur4["group_size"] != prev4["group_size"]:
        raise ValueError("INT4 group_size mismatch for reuse")
    stats = {"applied": 0, "skipped_precision": 0}
    if not reuse_mask or not prev.packed_data:
        return stats
    prev_prec: Dict[Tuple[int, int], str] = {}
    prev_pos: Dict[Tuple[int, int], int] = {}
    for prec, pdata in prev.packed_data.items():
        for pos, e in enumerate(pdata["indices"]):
            prev_prec[e] = prec
            prev_pos[e] = pos
    B = cache.batch_size
    for prec, data in cache.packed_data.items():
        pdata = prev.packed_data.get(prec)
        tgt, src = [], []
        for pos, e in enumerate(data["indices"]):
            if not reuse_mask.get(e, False):
                continue
            if prev_prec.get(e) == prec and e in prev_pos:
                tgt.append(pos)
                src.append(prev_pos[e])
            elif e in prev_prec:
                stats["skipped_precision"] += 1
        if not tgt:
            continue
        tgt_a = np.array(tgt, np.int64)
        src_a = np.array(src, np.int64)
        if prec in ("fp32", "fp16", "int8"):
            for key in ("k", "v", "scale_k", "scale_v"):
                if data.get(key) is not None:
                    data[key][tgt_a] = pdata[key][src_a]
        else:
            n, pn = len(data["indices"]), len(pdata["indices"])
            rb = data["k"].size // n
            G = data["num_groups"]
            for key in ("k", "v"):
                data[key].reshape(n, rb)[tgt_a] = pdata[key].reshape(pn, rb)[src_a]
            for key in ("scale_k", "scale_v"):
                data[key].reshape(n, B, G, 1)[tgt_a] = pdata[key].reshape(pn, B, G, 1)[src_a]
        stats["applied"] += len(tgt)
    return stats


# --------------------------------------------------------------------------
# INT8Linear (shadowinfer/ffn_optimizer/int8_linear.py)
# --------------------------------------------------------------------------

def int8_weight_quant(w: np.ndarray) -> Tuple[np.ndarray, np.ndarray]:
    """from_linear (int8_linear.py:65-82): w fp32 [N,K] -> (qweight [K,N], scale [N])."""
    w = np.ascontiguousarray(w, dtype=np.float32)
    N, K = w.shape
    qT = np.empty((K, N), np.int8)
    s = np.empty(N, np.float32)
    lib().or_weight_quant_i8(_p(w), N, K, _p(qT), _p(s))
    return qT, s


def int8_act_quant(x: np.ndarray, dt: int) -> Tuple[np.ndarray, np.ndarray]:
    """forward prologue (int8_linear.py:96-98): x [M,K] -> (q int8 [M,K], s fp32 [M])."""
    x = np.ascontiguousarray(x)
    M, K = x.shape
    q = np.empty((M, K), np.int8)
    s = np.empty(M, np.float32)
    if M:
        lib().or_act_quant_i8(_p(x), dt, M, K, _p(q), _p(s))
    return q, s


def gemm_i8(a: np.ndarray, b: np.ndarray) -> np.ndarray:
    """torch._int_mm: int8 [M,K] x int8 [K,N] -> int32 [M,N]."""
    a = np.ascontiguousarray(a, dtype=np.int8)
    b = np.ascontiguousarray(b, dtype=np.int8)
    M, K = a.shape
    N = b.shape[1]
    c = np.empty((M, N), np.int32)
    lib().or_gemm_i8(_p(a), _p(b), M, N, K, _p(c))
    return c


def int8_epilogue(acc: np.ndarray, sx: np.ndarray, sw: np.ndarray,
                  bias: Optional[np.ndarray], out_dt: int) -> np.ndarray:
    """int8_linear.py:112-115."""
    acc = np.ascontiguousarray(acc, dtype=np.int32)
    M, N = acc.shape
    out = np.empty((M, N), _np_dtype(out_dt))
    b = None if bias is None else np.ascontiguousarray(bias, dtype=np.float32)
    lib().or_int8_epilogue(_p(acc), _p(np.ascontiguousarray(sx, np.float32)),
                           _p(np.ascontiguousarray(sw, np.float32)),
                           None if b is None else _p(b), M, N, _p(out), out_dt)
    return out


def int8_linear_forward(x: np.ndarray, dt: int, qweight: np.ndarray, sw: np.ndarray,
                        bias: Optional[np.ndarray] = None):
    """INT8Linear.forward (int8_linear.py:88-115) on a 2-D input.

    Returns ``(out in dtype dt, acc int32, q_x, s_x)``.
    """
    q, s = int8_act_quant(x, dt)
    acc = gemm_i8(q, qweight)
    return int8_epilogue(acc, s, sw, bias, dt), acc, q, s


# --------------------------------------------------------------------------
# Attention over unpacked K/V
# --------------------------------------------------------------------------

def attention(q: np.ndarray, k: np.ndarray, v: np.ndarray,
              sm_scale: Optional[float] = None) -> np.ndarray:
    """softmax(q k^T * scale) v in double precision, no mask; inputs fp32
    ``[..., S, D]`` with matching leading dims. Returns fp32."""
    q = np.ascontiguousarray(q, np.float32)
    k = np.ascontiguousarray(k, np.float32)
    v = np.ascontiguousarray(v, np.float32)
    Sq, D = q.shape[-2:]
    Skv = k.shape[-2]
    BH = q.size // (Sq * D)
    if sm_scale is None:
        sm_scale = 1.0 / float(np.sqrt(D))
    out = np.empty(q.shape, np.float32)
    work = np.empty(Skv, np.float64)
    lib().or_attention(_p(q), _p(k), _p(v), BH, Sq, Skv, D, sm_scale, _p(out), _p(work))
    return out


# --------------------------------------------------------------------------
# Rate-distortion admission (shadowinfer/shadowkv/rd_allocator.py)
# --------------------------------------------------------------------------

CODE_NAMES = {0: "fp32", 1: "fp16", 2: "int8", 3: "int4", 4: "evicted"}
LADDER = {"fp32": "fp16", "fp16": "int8", "int8": "int4"}


def entry_bytes(precision: str, batch: int, head_dim: int, group_size: int = 16) -> float:
    """Stored bytes of one token-head, K + V with scales (rd_allocator.py:26-44)."""
    p = precision.lower()
    if p == "evicted":
        return 0.0
    if p == "int4":
        group = group_size if group_size > 0 and head_dim % group_size == 0 else head_dim
        per_tensor = batch * head_dim / 2.0 + batch * (head_dim // group) * 4
    elif p == "int8":
        per_tensor = batch * head_dim + batch * 4
    elif p == "fp32":
        per_tensor = batch * head_dim * 4
    else:
        per_tensor = batch * head_dim * 2
    return per_tensor * 2.0


def code_costs(batch: int, head_dim: int, group_size: int = 16) -> np.ndarray:
    """int64 bytes per code 0..4 (rd_allocator.py:180-188, 222-229)."""
    return np.array([int(entry_bytes(CODE_NAMES[c], batch, head_dim, group_size)) for c in range(5)],
                    np.int64)


def kv_sensitivity(k: np.ndarray, v: np.ndarray, dt: int) -> np.ndarray:
    """kv_sensitivity (rd_allocator.py:47-61): k, v [B, H, S, D] in dtype ``dt``
    (fp32 values or fp16/bf16 bits); returns [S, H] in ``dt``."""
    k = np.ascontiguousarray(k)
    v = np.ascontiguousarray(v)
    if k.shape != v.shape:
        raise ValueError("k and v must have identical shapes")
    B, H, S, D = k.shape
    out = np.empty((S, H), _np_dtype(dt))
    lib().or_kv_sensitivity(_p(k), _p(v), dt, B, H, S, D, _p(out))
    return out


def _score(importance, sensitivity, rd_allocation, S, H):
    imp = np.asarray(importance, np.float32)[:S, :H]
    sens = np.asarray(sensitivity, np.float32)[:S, :H]
    if sens.shape != imp.shape:
        sens = np.ones_like(imp)
    return (imp * sens).astype(np.float32) if rd_allocation else imp


def admit_codes(codes: np.ndarray, importance, sensitivity, budget_bytes, batch: int,
                head_dim: int, sink_tokens: int = 0, rd_allocation: bool = True,
                allow_eviction: bool = False, protected_mask=None,
                group_size: int = 16) -> Tuple[np.ndarray, int, int]:
    """Closed-form greedy ladder of admit_codes (rd_allocator.py:190-318):
    stable ascending argsort of the score, prefix sums of the per-candidate
    savings, searchsorted for the boundary, partial downgrade of the boundary
    entry, then the optional eviction prefix."""
    codes = np.asarray(codes)
    if codes.ndim != 2:
        raise ValueError("codes must be 2-D [seq, heads]")
    out = codes.astype(np.int8).copy()
    S, H = out.shape
    flat = out.reshape(-1)
    costs = code_costs(batch, head_dim, group_size)
    predicted = int(costs[flat.astype(np.int64)].sum())
    if budget_bytes is None or budget_bytes < 0:
        return out, predicted, 0
    score = _score(importance, sensitivity, rd_allocation, S, H)
    eligible = np.ones((S, H), bool)
    if sink_tokens > 0:
        eligible[: min(int(sink_tokens), S)] = False
    if protected_mask is not None:
        eligible &= ~np.asarray(protected_mask, bool)[:S, :H]
    order = np.argsort(score.reshape(-1), kind="stable")
    cand = order[eligible.reshape(-1)[order]]
    if cand.size == 0:
        return out, predicted, 0
    deltas = np.array([costs[c] - costs[c + 1] for c in (0, 1, 2)], np.int64)

    if predicted > budget_bytes:
        excess = predicted - budget_bytes
        base = flat[cand].astype(np.int64)
        step1 = np.where(base < 3, deltas[np.minimum(base, 2)], 0)
        next1 = np.where(base < 3, base + 1, base)
        step2 = np.where(next1 < 3, deltas[np.minimum(next1, 2)], 0)
        next2 = np.where(next1 < 3, next1 + 1, next1)
        step3 = np.where(next2 < 3, deltas[np.minimum(next2, 2)], 0)
        cum = np.cumsum(step1 + step2 + step3)
        boundary = min(int(np.searchsorted(cum, excess, side="left")), cand.size)
        new = base.copy()
        new[:boundary] = np.where(base[:boundary] != 4, 3, base[:boundary])
        if boundary < cand.size:
            remaining = excess - (int(cum[boundary - 1]) if boundary > 0 else 0)
            if base[boundary] != 4:
                if remaining <= step1[boundary]:
                    new[boundary] = next1[boundary]
                elif remaining <= step1[boundary] + step2[boundary]:
                    new[boundary] = next2[boundary]
                else:
                    new[boundary] = 3
        flat[cand] = new.astype(np.int8)
        predicted = int(costs[flat.astype(np.int64)].sum())

    evicted = 0
    if allow_eviction and predicted > budget_bytes:
        excess = predicted - budget_bytes
        cum = np.cumsum(costs[flat[cand].astype(np.int64)])
        boundary = int(np.searchsorted(cum, excess, side="left"))
        if boundary >= cand.size:
            boundary = cand.size - 1
        target = cand[: boundary + 1]
        evicted = int((flat[target] != 4).sum())
        flat[target] = 4
        predicted = int(costs[flat.astype(np.int64)].sum())
    return out, predicted, evicted


def admit_budget_greedy(importance, sensitivity, precision_map: Dict[int, Dict[int, str]],
                        budget_bytes, batch: int, head_dim: int, sink_tokens: int = 0,
                        rd_allocation: bool = True, allow_eviction: bool = False,
                        protected=None, group_size: int = 16):
    """The per-candidate greedy loop of admit_budget (rd_allocator.py:66-170),
    one ladder step at a time: an independent formulation of the same
    admission, used to pin admit_codes."""
    result = {int(t): dict(m) for t, m in precision_map.items()}

    def total():
        return int(sum(entry_bytes(p, batch, head_dim, group_size)
                       for m in result.values() for p in m.values()))

    if budget_bytes is None or budget_bytes < 0:
        return result, total(), 0
    imp = np.asarray(importance, np.float32)
    S = min(imp.shape[0], max(result.keys(), default=0) + 1)
    H = min(imp.shape[1] if imp.ndim > 1 else 1, max((len(m) for m in result.values()), default=0))
    if S <= 0 or H <= 0:
        return result, total(), 0
    score = _score(importance, sensitivity, rd_allocation, S, H)
    protected = frozenset(protected or ())
    cands = sorted(((float(score[t, h]), t, h) for t in range(S) for h in range(H)
                    if t >= sink_tokens and (t, h) not in protected), key=lambda c: c[0])
    predicted = total()
    i = 0
    while predicted > budget_bytes and i < len(cands):
        _, t, h = cands[i]
        m = result.setdefault(t, {})
        cur = m.get(h, "fp16")
        nxt = LADDER.get(cur)
        if nxt is None:
            i += 1
            continue
        predicted -= int(entry_bytes(cur, batch, head_dim, group_size)
                         - entry_bytes(nxt, batch, head_dim, group_size))
        m[h] = nxt
        if nxt == "int4":
            i += 1
    evicted = 0
    if allow_eviction and predicted > budget_bytes:
        i = 0
        while predicted > budget_bytes and i < len(cands):
            _, t, h = cands[i]
            m = result.setdefault(t, {})
            cur = m.get(h, "fp16")
            if cur != "evicted":
                predicted -= int(entry_bytes(cur, batch, head_dim, group_size))
                m[h] = "evicted"
                evicted += 1
            i += 1
    return result, int(predicted), evicted


# --------------------------------------------------------------------------
# Working copy of the plan-driven compression
# (shadowinfer/shadowkv/shadowkv_agent.py:1698-1809)
# --------------------------------------------------------------------------

def compress_working_copy(k: np.ndarray, v: np.ndarray, dt: int, codes: np.ndarray,
                          group_size: int = 16, k_prev: Optional[np.ndarray] = None,
                          v_prev: Optional[np.ndarray] = None,
                          reuse_entries: Iterable[Tuple[int, int]] = ()):
    """The dense ``k``/``v`` of _compress_kv_with_plan: zeros, then per
    precision group the fp32 values, the fp16 round trip or the int8/int4
    integer codes cast to the input dtype (index_copy_ of ``qk.to(dtype)``,
    shadowkv_agent.py:1762-1776), then the reuse entries copied from the
    previous K/V (:1790-1797). Inputs and outputs in dtype ``dt``."""
    B, H, S, D = k.shape
    plan = plan_from_codes(codes)
    outs = []
    for x, prev in ((k, k_prev), (v, v_prev)):
        xf = x.reshape(B, H * S, D)
        out = np.zeros((B, H * S, D), _np_dtype(dt))
        for prec in PRECISIONS:
            flat = plan["flat_indices"][prec]
            if len(flat) == 0:
                continue
            grp = np.ascontiguousarray(xf[:, flat, :].transpose(1, 0, 2))  # [n, B, D]
            if prec == "fp32":
                val = grp
            elif prec == "fp16":
                val = convert(grp, dt, F16)
                val = convert(val, F16, dt)
            else:
                if prec == "int8":
                    q, _ = quant_rows_i8(grp, dt)
                else:
                    g = group_size if D % group_size == 0 else D
                    q, _ = quant_rows_i4(grp, dt, g)
                    q = q.reshape(grp.shape)
                val = from_f32(q.astype(np.float32), dt)
            out[:, flat, :] = np.asarray(val).transpose(1, 0, 2)
        entries = list(reuse_entries)
        if prev is not None and entries:
            pf = prev.reshape(B, H * S, D)
            rflat = np.array([h * S + t for t, h in entries], np.int64)
            out[:, rflat, :] = pf[:, rflat, :]
        outs.append(out.reshape(B, H, S, D))
    return outs[0], outs[1]
