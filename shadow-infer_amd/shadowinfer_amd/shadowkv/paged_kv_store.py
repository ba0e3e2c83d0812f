"""Paged incremental KV residency with the reference API
(shadowinfer/shadowkv/paged_kv_store.py:24-717), on the packed row format.

Layout. A page holds one precision for a run of tokens of every (batch,
head): capacity buffers ``[B, H, page_size, ...]`` allocated once (whole runs
of pages in one allocation), with ``page.k`` / ``.v`` / ``.scale_*`` the views
of the filled rows (the reference's tensor shapes). Appends write rows in place
through the pack kernels' row quantizers (``si_page_write`` /
``si_page_write_pages``), so a row is bit-identical to the same row in a
``PackedKVCache``; sealed pages are never touched. Every page records the dtype
its scales and "fp32" payloads are stored in: appending another input dtype
to an open page widens the page to ``torch.promote_types`` of the two (the
reference's ``torch.cat`` does the same), and ``gather`` decodes each page in
its own dtype in one launch (``si_page_gather`` over a device page table
cached until the pages change).

Bookkeeping. Pages live in a slot pool (``pages``, with ``None`` for free
slots, reused last-freed first) ordered by ``_order``; the counters and the
byte accounting are the reference's. Eviction state is a dense boolean
``[tokens, heads]`` ledger rather than a set of pairs: ``evict_tokens``
turns its argument into a mask in one pass (``_masks.token_head_mask``),
computes each touched page's newly evicted pairs, drops tokens whose every
head is newly evicted (the page splits into runs of survivors, found with
numpy), and zeroes the payload rows of partially evicted heads with one
masked device fill per run and tensor.
"""

from __future__ import annotations

from typing import Any, Dict, List, Optional, Set, Tuple

import numpy as np
import torch

from .. import _native
from ._masks import token_head_mask

_PRECISIONS = ("fp32", "fp16", "int8", "int4")
_PREC_CODE = {"fp32": 0, "fp16": 1, "int8": 2, "int4": 3}
_TENSORS = ("k", "v", "scale_k", "scale_v")


class _Page:
    """One page: precision, storage dtype, token interval and capacity buffers."""

    __slots__ = ("precision", "dtype", "start_token", "num_tokens", "sealed", "buf")

    def __init__(self, precision: str, dtype: torch.dtype, buf: Dict[str, Optional[torch.Tensor]],
                 start_token: int, num_tokens: int, sealed: bool) -> None:
        self.precision = precision
        self.dtype = dtype
        self.buf = buf
        self.start_token = start_token
        self.num_tokens = num_tokens
        self.sealed = sealed

    def _view(self, name: str) -> Optional[torch.Tensor]:
        t = self.buf[name]
        return None if t is None else t[:, :, : self.num_tokens]

    k = property(lambda self: self._view("k"))
    v = property(lambda self: self._view("v"))
    scale_k = property(lambda self: self._view("scale_k"))
    scale_v = property(lambda self: self._view("scale_v"))

    @property
    def end_token(self) -> int:
        return self.start_token + self.num_tokens

    @property
    def capacity(self) -> int:
        return int(self.buf["k"].shape[2])


class PagedKVStore:
    """Page-table-indirected KV storage with incremental appends; one store
    covers one layer (paged_kv_store.py:63-717)."""

    def __init__(self, batch_size: int, num_heads: int, head_dim: int, page_size: int = 32,
                 device: Any = "cpu", int4_group_size: int = 16) -> None:
        if page_size < 1:
            raise ValueError(f"page_size must be >= 1, got {page_size}")
        if int4_group_size < 1:
            raise ValueError(f"int4_group_size must be >= 1, got {int4_group_size}")
        self.batch_size = int(batch_size)
        self.num_heads = int(num_heads)
        self.head_dim = int(head_dim)
        self.page_size = int(page_size)
        self.device = device
        self.int4_group_size = int(int4_group_size)
        self.clear()

    def clear(self) -> None:
        """Drop every page and counter (paged_kv_store.py:700-710)."""
        self.pages: List[Optional[_Page]] = []
        self._order: List[int] = []
        self._free: List[int] = []
        self._max_seq = 0
        self._stats = {"appended": 0, "page_evictions": 0, "rewritten_tokens": 0,
                       "rewritten_pages": 0}
        self._evicted = np.zeros((0, self.num_heads), dtype=bool)
        self._table: Optional[torch.Tensor] = None

    # ----------------------------------------------------------- properties
    max_seq = property(lambda self: self._max_seq)
    page_count = property(lambda self: len(self._order))
    appended_tokens = property(lambda self: self._stats["appended"])
    page_evictions = property(lambda self: self._stats["page_evictions"])
    rewritten_tokens = property(lambda self: self._stats["rewritten_tokens"])
    rewritten_pages = property(lambda self: self._stats["rewritten_pages"])

    @property
    def open_pages(self) -> int:
        return sum(not p.sealed for p in self._live())

    @property
    def _int4_effective_group(self) -> int:
        g = self.int4_group_size
        return g if self.head_dim % g == 0 else self.head_dim

    def _live(self) -> List[_Page]:
        return [self.pages[s] for s in self._order if self.pages[s] is not None]

    # ----------------------------------------------------------- validation
    def validate_against(self, batch: int, heads: int, head_dim: int) -> None:
        """Raise ValueError when the store's shape is not the model's
        (paged_kv_store.py:148-155)."""
        if (batch, heads, head_dim) != (self.batch_size, self.num_heads, self.head_dim):
            raise ValueError(
                "PagedKVStore shape mismatch: store="
                f"({self.batch_size},{self.num_heads},{self.head_dim}) vs "
                f"model=({batch},{heads},{head_dim})")

    def _check_rows(self, k_new: torch.Tensor, v_new: torch.Tensor, precision: str,
                    what: str) -> int:
        """The argument checks of append / rewrite_tokens (paged_kv_store.py:157-186,
        449-484); returns the token count."""
        if precision not in _PRECISIONS:
            raise ValueError(f"Unsupported page precision: {precision}")
        if k_new.dim() != 4 or v_new.dim() != 4:
            raise ValueError(
                "k_new/v_new must be 4-D [batch, heads, tokens, head_dim], got "
                f"k.dim={k_new.dim()}, v.dim={v_new.dim()}")
        if k_new.shape != v_new.shape:
            raise ValueError(
                f"k_new/v_new shapes disagree: {tuple(k_new.shape)} vs {tuple(v_new.shape)}")
        B, H, _, D = k_new.shape
        if (B, H, D) != (self.batch_size, self.num_heads, self.head_dim):
            raise ValueError(
                f"PagedKVStore {what} shape mismatch: expected "
                f"({self.batch_size},{self.num_heads},T,{self.head_dim}), got "
                f"{tuple(k_new.shape)}")
        return int(k_new.shape[2])

    @staticmethod
    def _device_rows(k_new: torch.Tensor, v_new: torch.Tensor):
        _native.require_device(k_new, "PagedKVStore")
        if v_new.device != k_new.device or v_new.dtype != k_new.dtype:
            raise ValueError("k_new and v_new must share device and dtype")
        _native.dtype_code(k_new.dtype)
        return k_new.detach().contiguous(), v_new.detach().contiguous()

    # ------------------------------------------------------------- buffers
    def _buffers(self, precision: str, dtype: torch.dtype, dev,
                 pages: Optional[int] = None) -> Dict[str, Optional[torch.Tensor]]:
        """Capacity buffers of one page, or of ``pages`` pages in one
        allocation (page i is ``buf[name][i]``)."""
        B, H, P, D = self.batch_size, self.num_heads, self.page_size, self.head_dim
        lead = () if pages is None else (pages,)
        G = D // self._int4_effective_group
        payload, row, scale = {"fp32": (dtype, D, None), "fp16": (torch.float16, D, None),
                               "int8": (torch.int8, D, (1,)),
                               "int4": (torch.uint8, (D + 1) // 2, (G, 1))}[precision]
        buf: Dict[str, Optional[torch.Tensor]] = {}
        for name in ("k", "v"):
            buf[name] = torch.empty(*lead, B, H, P, row, dtype=payload, device=dev)
        for name in ("scale_k", "scale_v"):
            buf[name] = (None if scale is None
                         else torch.empty(*lead, B, H, P, *scale, dtype=dtype, device=dev))
        return buf

    @staticmethod
    def _ptrs(buf) -> "Any":
        return _native.table4([None if buf[n] is None else buf[n].data_ptr() for n in _TENSORS])

    def _write_rows(self, page: _Page, k: torch.Tensor, v: torch.Tensor, t0: int, n: int,
                    row0: int) -> None:
        """Page rows [row0, row0 + n) <- tokens [t0, t0 + n) of k/v, quantized
        in k's dtype and stored in the page's (a torch copy converts them when
        the two differ, as the reference's copy_ / cat does)."""
        B, H, T, D = k.shape
        g = self._int4_effective_group
        if k.dtype == page.dtype:
            _native.call("si_page_write", k.data_ptr(), v.data_ptr(), _native.dtype_code(k.dtype),
                         B, H, T, D, t0, n, _PREC_CODE[page.precision], g, self._ptrs(page.buf),
                         page.capacity, row0, _native.stream(k.device))
            return
        tmp = self._buffers(page.precision, k.dtype, k.device)
        for lo in range(0, n, self.page_size):
            m = min(self.page_size, n - lo)
            _native.call("si_page_write", k.data_ptr(), v.data_ptr(), _native.dtype_code(k.dtype),
                         B, H, T, D, t0 + lo, m, _PREC_CODE[page.precision], g, self._ptrs(tmp),
                         self.page_size, 0, _native.stream(k.device))
            for name in _TENSORS:
                if page.buf[name] is not None:
                    page.buf[name][:, :, row0 + lo: row0 + lo + m].copy_(tmp[name][:, :, :m])

    def _widen(self, page: _Page, dtype: torch.dtype) -> None:
        """Store the page in ``dtype`` from now on (its filled rows converted)."""
        buf = self._buffers(page.precision, dtype, page.buf["k"].device)
        for name in _TENSORS:
            if buf[name] is not None:
                buf[name][:, :, : page.num_tokens].copy_(page.buf[name][:, :, : page.num_tokens])
        page.buf, page.dtype = buf, dtype

    def _take_slot(self) -> int:
        if self._free:
            return self._free.pop()
        self.pages.append(None)
        return len(self.pages) - 1

    def _grow_ledger(self, tokens: int) -> None:
        if tokens > self._evicted.shape[0]:
            grown = np.zeros((max(tokens, 2 * self._evicted.shape[0]), self.num_heads), dtype=bool)
            grown[: self._evicted.shape[0]] = self._evicted
            self._evicted = grown

    # -------------------------------------------------------------- append
    def _tail(self, precision: str) -> Optional[_Page]:
        """The open tail page if it can take ``precision`` rows; a tail of
        another precision is sealed (paged_kv_store.py:309-324)."""
        if not self._order:
            return None
        page = self.pages[self._order[-1]]
        if page is None or page.sealed:
            return None
        if page.precision != precision:
            page.sealed = True
            return None
        return page

    def append(self, k_new: torch.Tensor, v_new: torch.Tensor, precision: str) -> None:
        """Append tokens after the last one; sealed pages are never touched
        (paged_kv_store.py:248-307)."""
        tokens = self._check_rows(k_new, v_new, precision, "append")
        if tokens == 0:
            return
        k, v = self._device_rows(k_new, v_new)
        self._table = None
        self._grow_ledger(self._max_seq + tokens)
        done = 0
        while done < tokens:
            page = self._tail(precision)
            if page is not None:                    # fill the open tail page
                n = min(self.page_size - page.num_tokens, tokens - done)
                wide = torch.promote_types(page.dtype, k.dtype)
                if wide != page.dtype:
                    self._widen(page, wide)
                self._write_rows(page, k, v, done, n, page.num_tokens)
                page.num_tokens += n
                page.sealed = page.num_tokens == self.page_size
                self._max_seq += n
            elif (tokens - done) // self.page_size >= 2:   # a run of whole pages
                n = self._append_whole_pages(k, v, done, (tokens - done) // self.page_size,
                                             precision)
            else:                                   # one new page
                n = min(self.page_size, tokens - done)
                page = _Page(precision, k.dtype, self._buffers(precision, k.dtype, k.device),
                             self._max_seq, n, n == self.page_size)
                self._write_rows(page, k, v, done, n, 0)
                slot = self._take_slot()
                self.pages[slot] = page
                self._order.append(slot)
                self._max_seq += n
            done += n
        self._stats["appended"] += tokens

    def _append_whole_pages(self, k: torch.Tensor, v: torch.Tensor, t0: int, count: int,
                            precision: str) -> int:
        """``count`` sealed pages for tokens [t0, t0 + count * page_size), one
        allocation per tensor and one launch. Returns the tokens taken."""
        B, H, T, D = k.shape
        P = self.page_size
        bufs = self._buffers(precision, k.dtype, k.device, pages=count)
        _native.call("si_page_write_pages", k.data_ptr(), v.data_ptr(),
                     _native.dtype_code(k.dtype), B, H, T, D, t0, count, _PREC_CODE[precision],
                     self._int4_effective_group, self._ptrs(bufs), P, _native.stream(k.device))
        for i in range(count):
            slot = self._take_slot()
            self.pages[slot] = _Page(precision, k.dtype,
                                     {n: (None if t is None else t[i]) for n, t in bufs.items()},
                                     self._max_seq, P, True)
            self._order.append(slot)
            self._max_seq += P
        return count * P

    # -------------------------------------------------------------- gather
    def gather(self) -> Tuple[torch.Tensor, torch.Tensor]:
        """Dense fp32 (k, v) ``[B, H, S, D]`` (paged_kv_store.py:326-376): S
        is the end of the last page when the pages tile [0, S) without a gap
        (the reference concatenates them), otherwise max_seq with zeros where
        no page is."""
        B, H, D = self.batch_size, self.num_heads, self.head_dim
        live = self._live()
        if not self._order:
            empty = torch.zeros(B, H, 0, D, dtype=torch.float32, device=self.device)
            return empty, empty.clone()
        starts = np.array([p.start_token for p in live], dtype=np.int64)
        ends = np.array([p.end_token for p in live], dtype=np.int64)
        tiled = (len(live) == len(self._order) and len(live) > 0 and starts[0] == 0
                 and bool((starts[1:] == ends[:-1]).all()))
        S = int(ends[-1]) if tiled else self._max_seq
        dev = live[0].buf["k"].device if live else self.device
        make = torch.empty if tiled else torch.zeros
        k_out = make(B, H, S, D, dtype=torch.float32, device=dev)
        v_out = make(B, H, S, D, dtype=torch.float32, device=dev)
        if not live or S == 0:
            return k_out, v_out
        if self._table is None or self._table.device != dev:
            rows = [[_PREC_CODE[p.precision], _native.dtype_code(p.dtype)]
                    + [0 if p.buf[n] is None else p.buf[n].data_ptr() for n in _TENSORS]
                    + [p.start_token, p.num_tokens, p.capacity] for p in live]
            self._table = torch.tensor(rows, dtype=torch.int64).to(dev)
        _native.call("si_page_gather", self._table.data_ptr(), len(live), B, H, S, D,
                     self._int4_effective_group, k_out.data_ptr(), v_out.data_ptr(),
                     _native.stream(dev))
        return k_out, v_out

    # ------------------------------------------------------------- rewrite
    def rewrite_tokens(self, start_token: int, k_new: torch.Tensor, v_new: torch.Tensor,
                       precision: str) -> int:
        """Overwrite token rows [start, start + T) in place through the append
        path's row quantizers (paged_kv_store.py:407-447). Every check runs
        before the first write, so a failed call changes nothing."""
        start = int(start_token)
        tokens = self._check_rows(k_new, v_new, precision, "rewrite")
        if tokens < 1:
            raise ValueError(f"rewrite interval must cover at least one token, got {tokens}")
        end = start + tokens
        if start < 0 or end > self._max_seq:
            raise ValueError(
                f"rewrite interval [{start},{end}) exceeds stored range [0,{self._max_seq})")
        hits = self._rewrite_targets(start, end, precision)
        k, v = self._device_rows(k_new, v_new)
        for page, lo, hi in hits:
            self._write_rows(page, k, v, lo - start, hi - lo, lo - page.start_token)
        self._stats["rewritten_tokens"] += tokens
        self._stats["rewritten_pages"] += len(hits)
        return tokens

    def _rewrite_targets(self, start: int, end: int, precision: str):
        """Pages overlapping [start, end) with their overlaps; raises unless
        they all hold ``precision``, cover the interval and no token in it has
        an evicted head (paged_kv_store.py:486-525)."""
        hits = []
        for page in self._live():
            lo, hi = max(start, page.start_token), min(end, page.end_token)
            if lo >= hi:
                continue
            if page.precision != precision:
                raise ValueError(
                    "rewrite precision does not match hit page: requested "
                    f"{precision}, page holds {page.precision}")
            hits.append((page, lo, hi))
        covered = sum(hi - lo for _, lo, hi in hits)
        if covered != end - start:
            raise ValueError(
                f"rewrite interval [{start},{end}) is not fully covered by pages "
                f"({covered} of {end - start} tokens); evicted holes cannot be rewritten")
        bad = np.flatnonzero(self._evicted[start:end].any(axis=1))
        if bad.size:
            raise ValueError(
                f"rewrite interval [{start},{end}) contains evicted token {start + int(bad[0])}; "
                "evicted positions cannot be rewritten")
        return hits

    # ---------------------------------------------------------- accounting
    def data_plane_bytes(self) -> int:
        """Payload + scale bytes of the filled rows (paged_kv_store.py:527-537)."""
        total = 0
        for p in self._live():
            for name in _TENSORS:
                t = p._view(name)
                if t is not None:
                    total += t.numel() * t.element_size()
        return total

    def resident_bytes(self) -> int:
        """Data bytes + 48 per stored token-head + 16 per pool slot
        (paged_kv_store.py:539-554)."""
        if not self._order:
            return 0
        tokens = sum(p.num_tokens for p in self._live())
        return (self.data_plane_bytes() + 48 * self.batch_size * self.num_heads * tokens
                + 16 * len(self.pages))

    # ------------------------------------------------------------ eviction
    def evict_tokens(self, token_head_set: Set[Tuple[int, int]]) -> int:
        """Page-local eviction (paged_kv_store.py:556-698). Returns the
        (token, head) pairs newly evicted; already evicted or absent pairs
        count for nothing. A token whose every head is newly evicted leaves
        its page (the page splits into runs of survivors); the others keep
        their rows, with the payload of newly evicted heads zeroed (code 0)."""
        if not token_head_set or not self._order:
            return 0
        mask = token_head_mask(token_head_set, self._max_seq, self.num_heads)
        if mask is None:
            return 0
        fresh = mask.reshape(self._max_seq, self.num_heads).astype(bool)
        fresh &= ~self._evicted[: self._max_seq]
        removed = 0
        replaced: Dict[int, List[_Page]] = {}
        for slot in self._order:
            page = self.pages[slot]
            if page is None:
                continue
            rows = fresh[page.start_token: page.end_token]
            n = int(rows.sum())
            if n == 0:
                continue
            removed += n
            self._stats["page_evictions"] += 1
            self._evicted[page.start_token: page.end_token] |= rows
            replaced[slot] = self._survivor_runs(page, rows)
        if removed == 0:
            return 0
        self._table = None
        for slot, runs in replaced.items():
            if not runs:
                self.pages[slot] = None
                self._free.append(slot)
        order: List[int] = []
        for slot in self._order:
            runs = replaced.get(slot)
            if runs is None:
                order.append(slot)
                continue
            for i, run in enumerate(runs):
                target = slot if i == 0 else self._take_slot()
                self.pages[target] = run
                order.append(target)
        self._order = order
        return removed

    def _survivor_runs(self, page: _Page, rows: np.ndarray) -> List[_Page]:
        """New pages for the maximal runs of kept tokens of ``page``; ``rows``
        ([tokens, heads] bool) marks its newly evicted pairs. A token leaves
        when all its heads are newly evicted."""
        kept = ~rows.all(axis=1)
        edges = np.flatnonzero(np.diff(np.concatenate(([False], kept, [False])).astype(np.int8)))
        bounds = edges.reshape(-1, 2)                        # [run, (begin, end)]
        dev = page.buf["k"].device
        fill = 0x88 if page.precision == "int4" else 0        # code 0 in either layout
        out: List[_Page] = []
        for r, (a, b) in enumerate(bounds.tolist()):
            buf = self._buffers(page.precision, page.dtype, dev)
            for name in _TENSORS:
                if buf[name] is not None:
                    buf[name][:, :, : b - a].copy_(page.buf[name][:, :, a:b])
            zero = rows[a:b]                                  # kept tokens: newly evicted heads
            if zero.any():
                sel = torch.from_numpy(np.ascontiguousarray(zero.T)).to(dev)   # [H, run]
                for name in ("k", "v"):
                    view = buf[name][:, :, : b - a]
                    view[:, sel] = fill
            sealed = page.sealed or r < len(bounds) - 1 or (b - a) == self.page_size
            out.append(_Page(page.precision, page.dtype, buf, page.start_token + a, b - a, sealed))
        return out

    def __repr__(self) -> str:
        return (f"PagedKVStore(batch={self.batch_size}, heads={self.num_heads}, "
                f"head_dim={self.head_dim}, page_size={self.page_size}, "
                f"max_seq={self._max_seq}, pages={self.page_count})")
