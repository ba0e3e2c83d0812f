"""Precision/reuse plan with the reference API
(shadowinfer/shadowkv/precision_plan.py:18-194).

On a HIP device the grouping is computed by ``si_plan_scan``: every token-head
gets its bucket position (slot) from prefix sums over the int8 ``[S, H]`` code
matrix in token-major order, which is the order ``from_codes`` produces with
``nonzero`` in the reference. ``flat_indices`` (``h*S + t`` per bucket) are
scattered on the device too. The Python lists of the reference (``groups``,
``evicted_entries``) and the SHA-256 ``fingerprint`` are materialized lazily,
on first access, because the pack/unpack path never needs them.

A plan whose ``device`` is the CPU holds the same metadata computed on the
host, as the reference does for CPU tensors; such a plan cannot drive a device
pack (``PackedKVCache.pack`` raises ValueError, as the reference does).
"""

from __future__ import annotations

import ctypes

import hashlib
import struct
from itertools import chain
from typing import Any, Dict, List, Optional, Tuple

import numpy as np
import torch

from .. import _native

PRECISION_ORDER: Tuple[str, ...] = ("fp32", "fp16", "int8", "int4")
EVICTED = "evicted"
PRECISION_CODES: Dict[str, int] = {"fp32": 0, "fp16": 1, "int8": 2, "int4": 3, EVICTED: 4}
CODE_PRECISIONS: Dict[int, str] = {code: name for name, code in PRECISION_CODES.items()}


_FP16 = PRECISION_CODES["fp16"]
_NAME_OF_CODE = np.array([CODE_PRECISIONS[c] for c in range(5)], dtype=object)


def _index_in(key: Any, n: int) -> Optional[int]:
    """The integer in [0, n) that ``key`` equals as a dict key (3, 3.0,
    True, numpy integers), or None."""
    try:
        i = int(key)
    except (TypeError, ValueError, OverflowError):
        return None
    return i if 0 <= i < n and i == key else None


def _code_of(raw: Any, strict: bool) -> int:
    name = raw.lower() if isinstance(raw, str) else raw
    code = PRECISION_CODES.get(name) if isinstance(name, str) else None
    if code is None:
        if strict:
            raise ValueError(f"Unsupported precision: {raw}")
        return _FP16
    return code


def map_to_codes(precision_map: Dict[int, Dict[int, str]], seq_len: int, num_heads: int,
                 strict: bool = True, device: Any = "cpu") -> torch.Tensor:
    """``int8 [seq_len, num_heads]`` codes of a ``token -> head -> name`` map
    (precision_plan.py:30-55): entries the map does not name are fp16, names
    are case-insensitive, an unknown name raises ValueError when ``strict`` and
    is fp16 otherwise; keys outside the grid are ignored.

    Only the entries the map holds are visited (a sparse map costs its size,
    not seq_len * num_heads); the rest of the matrix is filled at once."""
    codes = np.full((seq_len, num_heads), _FP16, dtype=np.int8)
    rows = sorted(((t, row) for t, row in ((_index_in(k, seq_len), r)
                                          for k, r in precision_map.items()) if t is not None),
                  key=lambda tr: tr[0])
    for t, row in rows:
        named = [(h, raw) for h, raw in ((_index_in(k, num_heads), r) for k, r in row.items())
                 if h is not None]
        named.sort(key=lambda hr: hr[0])   # unknown names raise in (token, head) order
        if named:
            heads, raws = zip(*named)
            codes[t, list(heads)] = [_code_of(r, strict) for r in raws]
    return torch.from_numpy(codes).to(device)


def codes_to_map(codes: torch.Tensor) -> Dict[int, Dict[int, str]]:
    """``token -> head -> name`` map of an ``[S, H]`` code matrix
    (precision_plan.py:58-69); a code outside 0..4 raises ValueError."""
    values = codes.detach().to("cpu").to(torch.int64).numpy()
    bad = (values < 0) | (values > 4)
    if bad.any():
        raise ValueError(f"Unsupported precision code: {int(values[bad][0])}")
    names = _NAME_OF_CODE[values]
    return {t: dict(enumerate(row)) for t, row in enumerate(names.tolist())}


def _reuse_entries(reuse_mask: Optional[Dict[Tuple[int, int], bool]], seq_len: int,
                   num_heads: int) -> List[Tuple[int, int]]:
    """Sorted ``(int(t), int(h))`` of the truthy keys inside the grid
    (precision_plan.py:154-163; repeats kept, fractions truncated by int()).
    Numeric keys go through numpy in one pass; other keys take the
    element-wise rule (which raises where the reference's unpacking does)."""
    if not reuse_mask:
        return []
    n = len(reuse_mask)
    try:
        tk = np.fromiter(chain.from_iterable(reuse_mask.keys()), dtype=np.float64,
                         count=2 * n).reshape(n, 2)
        flag = np.fromiter(reuse_mask.values(), dtype=bool, count=n)
    except (TypeError, ValueError):
        out = sorted((int(t), int(h)) for (t, h), f in reuse_mask.items()
                     if f and 0 <= t < seq_len and 0 <= h < num_heads)
        return out
    t, h = tk[:, 0], tk[:, 1]
    keep = flag & (t >= 0) & (t < seq_len) & (h >= 0) & (h < num_heads)
    flat = np.sort(t[keep].astype(np.int64) * num_heads + h[keep].astype(np.int64))
    return list(zip((flat // num_heads).tolist(), (flat % num_heads).tolist()))


class DeviceGrouping:
    """Device-side result of the plan scan shared by plans and packed caches.

    ``code``: int8 [S*H] sanitized codes (absent/unknown -> 4);
    ``slot``: int32 [S*H] bucket positions (-1 if absent);
    ``counts``: entries per code 0..4 (host ints);
    ``flat``: per precision, int64 ``h*S + t`` of the bucket's entries in
    slot order (the plan's ``flat_indices``), built on first use;
    ``attn``: the fused attention's per-head slot lists, built on first use.
    The tensors are never modified in place (eviction makes a new grouping),
    so what is derived from them stays valid.
    """

    __slots__ = ("code", "slot", "counts", "flat", "attn")

    def __init__(self, code: torch.Tensor, slot: torch.Tensor, counts: List[int],
                 flat: Optional[List[torch.Tensor]] = None):
        self.code = code
        self.slot = slot
        self.counts = counts
        self.flat = flat
        self.attn: Optional[torch.Tensor] = None

    def attn_lists(self, S: int, H: int) -> torch.Tensor:
        """Per-head slot lists of the fused attention (si_attn_build_lists)."""
        if self.attn is None:
            dev = self.code.device
            n = _native.size_query("si_attn_workspace_bytes", H, S)
            lists = torch.empty(max(n, 16), dtype=torch.uint8, device=dev)
            _native.call("si_attn_build_lists", self.code.data_ptr(), self.slot.data_ptr(), H, S,
                         lists.data_ptr(), n, _native.stream(dev))
            self.attn = lists
        return self.attn

    def flat_lists(self, S: int, H: int) -> List[torch.Tensor]:
        """Per-precision ``h*S + t`` lists in slot order (si_plan_scatter)."""
        if self.flat is None:
            dev = self.code.device
            flat = [torch.empty(self.counts[p], dtype=torch.long, device=dev) for p in range(4)]
            _native.call("si_plan_scatter", self.code.data_ptr(), self.slot.data_ptr(), S, H,
                         _native.table4([f.data_ptr() for f in flat]), _native.table4([None] * 4),
                         _native.stream(dev))
            self.flat = flat
        return self.flat

    @staticmethod
    def scan(codes_flat: torch.Tensor, evict_mask: Optional[torch.Tensor] = None) -> "DeviceGrouping":
        """Run si_plan_scan on int8 codes (token-major) on a HIP device."""
        _native.require_device(codes_flat, "plan scan")
        dev = codes_flat.device
        n = codes_flat.numel()
        ws_bytes = _native.size_query("si_plan_workspace_bytes", n)
        ws = torch.empty(ws_bytes, dtype=torch.uint8, device=dev)
        code = torch.empty(n, dtype=torch.int8, device=dev)
        slot = torch.empty(n, dtype=torch.int32, device=dev)
        counts = torch.empty(5, dtype=torch.int64, device=dev)
        _native.call("si_plan_scan", codes_flat.data_ptr(),
                     _native.ptr(evict_mask), n, code.data_ptr(), slot.data_ptr(),
                     counts.data_ptr(), ws.data_ptr(), ws_bytes, _native.stream(dev))
        return DeviceGrouping(code, slot, [int(c) for c in counts.tolist()])

    def evict_count(self, evict_mask: torch.Tensor, S: int, H: int):
        """First pass of an evict (si_kv_evict_count) over this grouping's
        lists: returns the new codes, the new slot array (-1 already written
        for every entry that is not kept), the per-chunk survivor counts and
        bits on the device, and the new bucket sizes (host ints, code 4 last),
        read from those counts."""
        dev = self.code.device
        n = S * H
        flat = self.flat_lists(S, H)
        lib = _native.load()
        old = (ctypes.c_int64 * 4)(*self.counts[:4])
        chunks = int(lib.si_kv_evict_chunks(old))
        words = int(lib.si_kv_evict_chunk_words())
        code = torch.empty(n, dtype=torch.int8, device=dev)
        slot = torch.empty(n, dtype=torch.int32, device=dev)
        cc = torch.empty(max(chunks, 1), dtype=torch.int32, device=dev)
        bits = torch.empty(max(chunks * words, 1), dtype=torch.int64, device=dev)
        _native.call("si_kv_evict_count", self.code.data_ptr(),
                     _native.table4([f.data_ptr() for f in flat]), old, evict_mask.data_ptr(), S, H,
                     code.data_ptr(), slot.data_ptr(), cc.data_ptr(), bits.data_ptr(),
                     _native.stream(dev))
        per = cc[:chunks].cpu().numpy().astype(np.int64)
        rows = 64 * words
        ends = np.cumsum([-(-c // rows) for c in self.counts[:4]])
        starts = np.concatenate(([0], ends[:-1]))
        new_counts = [int(per[a:b].sum()) for a, b in zip(starts, ends)]
        new_counts.append(n - sum(new_counts))
        return code, slot, (cc, bits), new_counts


class PrecisionPlan:
    """Immutable grouping/index plan shared by compress and pack
    (precision_plan.py:72-84). Fields: seq_len, num_heads, codes, groups,
    flat_indices, reuse_entries, reuse_flat, fingerprint, evicted_entries."""

    __slots__ = ("seq_len", "num_heads", "codes", "flat_indices", "reuse_entries", "reuse_flat",
                 "_groups", "_evicted", "_fingerprint", "_grouping", "_entries", "_frozen")

    def __init__(self, seq_len: int, num_heads: int, codes: torch.Tensor,
                 flat_indices: Dict[str, torch.Tensor], reuse_entries: List[Tuple[int, int]],
                 reuse_flat: torch.Tensor, grouping: Optional[DeviceGrouping] = None,
                 entries: Optional[Dict[str, torch.Tensor]] = None,
                 groups: Optional[Dict[str, List[Tuple[int, int]]]] = None,
                 evicted_entries: Optional[List[Tuple[int, int]]] = None,
                 fingerprint: Optional[str] = None):
        object.__setattr__(self, "_frozen", False)
        self.seq_len = seq_len
        self.num_heads = num_heads
        self.codes = codes
        self.flat_indices = flat_indices
        self.reuse_entries = reuse_entries
        self.reuse_flat = reuse_flat
        self._grouping = grouping
        self._entries = entries
        self._groups = groups
        self._evicted = evicted_entries
        self._fingerprint = fingerprint
        object.__setattr__(self, "_frozen", True)

    def __setattr__(self, name, value):
        if getattr(self, "_frozen", False) and not name.startswith("_"):
            raise AttributeError(f"PrecisionPlan is immutable (cannot set {name!r})")
        object.__setattr__(self, name, value)

    # ------------------------------------------------------------------ build
    @classmethod
    def build(cls, precision_map: Dict[int, Dict[int, str]], seq_len: int, num_heads: int,
              reuse_mask: Optional[Dict[Tuple[int, int], bool]] = None, device: Any = "cpu",
              strict: bool = True) -> "PrecisionPlan":
        """precision_plan.py:86-111."""
        codes = map_to_codes(precision_map, seq_len, num_heads, strict=strict, device=device)
        return cls.from_codes(codes, reuse_mask=reuse_mask, device=device)

    @classmethod
    def from_codes(cls, codes: torch.Tensor,
                   reuse_mask: Optional[Dict[Tuple[int, int], bool]] = None,
                   device: Any = None) -> "PrecisionPlan":
        """precision_plan.py:113-177 (device grouping by prefix sums)."""
        if codes.dim() != 2:
            raise ValueError(f"codes must be 2-D [seq, heads], got shape {tuple(codes.shape)}")
        seq_len, num_heads = int(codes.shape[0]), int(codes.shape[1])
        if seq_len <= 0 or num_heads <= 0:
            raise ValueError(f"seq_len and num_heads must be positive, got {seq_len}, {num_heads}")
        if device is None:
            device = codes.device
        device = torch.device(device)
        codes = codes.detach().to(device=device, dtype=torch.int8).contiguous()

        reuse_entries = _reuse_entries(reuse_mask, seq_len, num_heads)
        pairs = np.array(reuse_entries, dtype=np.int64).reshape(-1, 2)
        reuse_flat = torch.from_numpy(pairs[:, 1] * seq_len + pairs[:, 0]).to(device)

        if device.type == "cpu":
            return cls._from_codes_host(codes, reuse_entries, reuse_flat)

        grouping = DeviceGrouping.scan(codes.reshape(-1))
        flat_indices: Dict[str, torch.Tensor] = {}
        entries: Dict[str, torch.Tensor] = {}
        for p, name in enumerate(PRECISION_ORDER):
            flat_indices[name] = torch.empty(grouping.counts[p], dtype=torch.long, device=device)
            entries[name] = torch.empty(grouping.counts[p], dtype=torch.int32, device=device)
        _native.call("si_plan_scatter", grouping.code.data_ptr(), grouping.slot.data_ptr(),
                     seq_len, num_heads,
                     _native.table4([flat_indices[n].data_ptr() for n in PRECISION_ORDER]),
                     _native.table4([entries[n].data_ptr() for n in PRECISION_ORDER]),
                     _native.stream(device))
        grouping.flat = [flat_indices[n] for n in PRECISION_ORDER]
        return cls(seq_len, num_heads, codes, flat_indices, reuse_entries, reuse_flat,
                   grouping=grouping, entries=entries)

    @classmethod
    def _from_codes_host(cls, codes: torch.Tensor, reuse_entries, reuse_flat) -> "PrecisionPlan":
        """Host metadata of a CPU plan (the grouping of precision_plan.py:132-151):
        one stable argsort of the flat codes puts each code's entries together
        in token-major order; codes outside 0..4 belong to no group."""
        S, H = int(codes.shape[0]), int(codes.shape[1])
        flat = codes.reshape(-1).numpy().astype(np.int64)
        order = np.argsort(flat, kind="stable")
        counts = np.bincount(flat[(flat >= 0) & (flat <= 4)], minlength=5)
        first = int(np.count_nonzero(flat < 0))
        bounds = first + np.concatenate(([0], np.cumsum(counts)))
        groups: Dict[str, List[Tuple[int, int]]] = {}
        flat_indices: Dict[str, torch.Tensor] = {}
        evicted: List[Tuple[int, int]] = []
        for code in range(5):
            e = order[bounds[code]: bounds[code + 1]]
            t, h = e // H, e % H
            pairs = list(zip(t.tolist(), h.tolist()))
            if code == PRECISION_CODES[EVICTED]:
                evicted = pairs
            else:
                name = CODE_PRECISIONS[code]
                groups[name] = pairs
                flat_indices[name] = torch.from_numpy(h * S + t)
        return cls(S, H, codes, flat_indices, reuse_entries, reuse_flat,
                   groups=groups, evicted_entries=evicted)

    # ------------------------------------------------------------- lazy views
    @property
    def device(self) -> torch.device:
        return self.codes.device

    @property
    def counts(self) -> List[int]:
        """Entries per code 0..4."""
        if self._grouping is not None:
            return list(self._grouping.counts)
        c = [len(self.groups[p]) for p in PRECISION_ORDER]
        return c + [self.seq_len * self.num_heads - sum(c)]

    @property
    def groups(self) -> Dict[str, List[Tuple[int, int]]]:
        if self._groups is None:
            H = self.num_heads
            groups: Dict[str, List[Tuple[int, int]]] = {}
            for name in PRECISION_ORDER:
                e = self._entries[name].to("cpu", torch.int64)
                groups[name] = list(zip(torch.div(e, H, rounding_mode="floor").tolist(),
                                        torch.remainder(e, H).tolist()))
            object.__setattr__(self, "_groups", groups)
        return self._groups

    @property
    def evicted_entries(self) -> List[Tuple[int, int]]:
        if self._evicted is None:
            sel = (self.codes.reshape(-1).to("cpu", torch.int64) == 4).nonzero().reshape(-1)
            H = self.num_heads
            object.__setattr__(self, "_evicted", list(zip(
                torch.div(sel, H, rounding_mode="floor").tolist(),
                torch.remainder(sel, H).tolist())))
        return self._evicted

    @property
    def fingerprint(self) -> str:
        """SHA-256 of ``<QQ`` (S, H) + code bytes + reuse_flat int64 bytes
        (precision_plan.py:179-190)."""
        if self._fingerprint is None:
            digest = hashlib.sha256()
            digest.update(struct.pack("<QQ", self.seq_len, self.num_heads))
            digest.update(self.codes.detach().to("cpu").contiguous().numpy().tobytes())
            digest.update(self.reuse_flat.detach().to("cpu").contiguous().numpy().tobytes())
            object.__setattr__(self, "_fingerprint", digest.hexdigest())
        return self._fingerprint

    def reuse_set(self) -> set:
        """precision_plan.py:192-194."""
        return set(self.reuse_entries)

    def device_grouping(self) -> DeviceGrouping:
        """The device scan (code / slot / counts) driving a pack."""
        if self._grouping is None:
            raise ValueError("plan was built on the CPU; build it on the KV device")
        return self._grouping

    def __repr__(self) -> str:
        return (f"PrecisionPlan(seq_len={self.seq_len}, num_heads={self.num_heads}, "
                f"device={self.device}, counts={self.counts})")
