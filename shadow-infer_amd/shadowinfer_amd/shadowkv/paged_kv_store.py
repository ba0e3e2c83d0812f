"""Paged incremental KV residency with the reference API
(shadowinfer/shadowkv/paged_kv_store.py).

Pages hold one precision for a run of tokens of every (batch, head). Each
page is a set of capacity buffers ``[B, H, page_size, ...]`` allocated once;
``page.k`` / ``page.v`` / ``page.scale_*`` are views of the filled rows
(``[B, H, num_tokens, ...]``, the reference's tensor shapes), so an append
writes the new rows in place (``si_page_write``, the pack's row quantizers)
instead of concatenating and re-allocating the open page, and sealed pages
are never touched. ``gather`` decodes every page in one launch over a device
page table (``si_page_gather``). Page bookkeeping (token order, free slots,
sealing, eviction runs) follows the reference line by line on the host;
the row copies and zero fills of an eviction are device tensor copies.
"""

from __future__ import annotations

from typing import Any, Dict, List, Optional, Set, Tuple

import torch

from .. import _native

_PRECISIONS = ("fp32", "fp16", "int8", "int4")
_PREC_CODE = {"fp32": 0, "fp16": 1, "int8": 2, "int4": 3}


class _Page:
    """One page holding a single precision's quantized payload (views of
    the capacity buffers in ``_buf``)."""

    __slots__ = ("precision", "k", "v", "scale_k", "scale_v", "start_token", "num_tokens",
                 "sealed", "_buf")

    def __init__(self, precision: str, buf: Dict[str, Optional[torch.Tensor]], start_token: int,
                 num_tokens: int, sealed: bool) -> None:
        self.precision = precision
        self._buf = buf
        self.start_token = start_token
        self.sealed = sealed
        self.num_tokens = 0
        self.k = self.v = self.scale_k = self.scale_v = None
        self._set_tokens(num_tokens)

    def _set_tokens(self, n: int) -> None:
        self.num_tokens = n
        for name in ("k", "v", "scale_k", "scale_v"):
            t = self._buf[name]
            setattr(self, name, None if t is None else t[:, :, :n])

    @property
    def end_token(self) -> int:
        return self.start_token + self.num_tokens

    @property
    def capacity(self) -> int:
        return int(self._buf["k"].shape[2])


class PagedKVStore:
    """Page-table-indirected KV storage with incremental appends
    (paged_kv_store.py:63-717). One store covers one layer."""

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
        self.pages: List[Optional[_Page]] = []
        self._order: List[int] = []
        self._free_slots: List[int] = []
        self._max_seq = 0
        self._appended_tokens = 0
        self._page_evictions = 0
        self._rewritten_tokens = 0
        self._rewritten_pages = 0
        self._evicted_pairs: Set[Tuple[int, int]] = set()
        self._dtype: Optional[torch.dtype] = None  # input dtype of the stored pages
        self._table: Optional[torch.Tensor] = None  # device page table, rebuilt after changes

    # ------------------------------------------------------------------ properties
    @property
    def max_seq(self) -> int:
        return self._max_seq

    @property
    def page_count(self) -> int:
        return len(self._order)

    @property
    def open_pages(self) -> int:
        return sum(1 for slot in self._order
                   if self.pages[slot] is not None and not self.pages[slot].sealed)

    @property
    def appended_tokens(self) -> int:
        return self._appended_tokens

    @property
    def page_evictions(self) -> int:
        return self._page_evictions

    @property
    def rewritten_tokens(self) -> int:
        return self._rewritten_tokens

    @property
    def rewritten_pages(self) -> int:
        return self._rewritten_pages

    @property
    def _int4_effective_group(self) -> int:
        if self.head_dim % self.int4_group_size == 0:
            return self.int4_group_size
        return self.head_dim

    # ------------------------------------------------------------------ validation
    def validate_against(self, batch: int, heads: int, head_dim: int) -> None:
        """paged_kv_store.py:148-155."""
        if batch != self.batch_size or heads != self.num_heads or head_dim != self.head_dim:
            raise ValueError(
                "PagedKVStore shape mismatch: store="
                f"({self.batch_size},{self.num_heads},{self.head_dim}) vs "
                f"model=({batch},{heads},{head_dim})")

    def _validate_kv(self, k_new: torch.Tensor, v_new: torch.Tensor, precision: str,
                     what: str) -> None:
        if precision not in _PRECISIONS:
            raise ValueError(f"Unsupported page precision: {precision}")
        if k_new.dim() != 4 or v_new.dim() != 4:
            raise ValueError(
                "k_new/v_new must be 4-D [batch, heads, tokens, head_dim], got "
                f"k.dim={k_new.dim()}, v.dim={v_new.dim()}")
        if k_new.shape != v_new.shape:
            raise ValueError(
                f"k_new/v_new shapes disagree: {tuple(k_new.shape)} vs {tuple(v_new.shape)}")
        if (k_new.shape[0] != self.batch_size or k_new.shape[1] != self.num_heads
                or k_new.shape[3] != self.head_dim):
            raise ValueError(
                f"PagedKVStore {what} shape mismatch: expected "
                f"({self.batch_size},{self.num_heads},T,{self.head_dim}), got "
                f"{tuple(k_new.shape)}")

    # ------------------------------------------------------------------ buffers
    def _new_buffers(self, precision: str, dtype: torch.dtype, dev,
                     count: Optional[int] = None) -> Dict[str, Optional[torch.Tensor]]:
        """Capacity buffers of one page, or of ``count`` pages allocated
        together (a leading page dimension; page i is ``buf[name][i]``)."""
        B, H, P, D = self.batch_size, self.num_heads, self.page_size, self.head_dim
        lead = () if count is None else (count,)

        def empty(*shape, dt):
            return torch.empty(*lead, *shape, dtype=dt, device=dev)

        if precision == "fp32":
            return {"k": empty(B, H, P, D, dt=dtype), "v": empty(B, H, P, D, dt=dtype),
                    "scale_k": None, "scale_v": None}
        if precision == "fp16":
            return {"k": empty(B, H, P, D, dt=torch.float16),
                    "v": empty(B, H, P, D, dt=torch.float16), "scale_k": None, "scale_v": None}
        if precision == "int8":
            return {"k": empty(B, H, P, D, dt=torch.int8), "v": empty(B, H, P, D, dt=torch.int8),
                    "scale_k": empty(B, H, P, 1, dt=dtype), "scale_v": empty(B, H, P, 1, dt=dtype)}
        G = D // self._int4_effective_group
        rb = (D + 1) // 2
        return {"k": empty(B, H, P, rb, dt=torch.uint8), "v": empty(B, H, P, rb, dt=torch.uint8),
                "scale_k": empty(B, H, P, G, 1, dt=dtype), "scale_v": empty(B, H, P, G, 1, dt=dtype)}

    def _write(self, page: _Page, k: torch.Tensor, v: torch.Tensor, t0: int, take: int,
               offset: int) -> None:
        """Rows [offset, offset+take) of the page <- tokens [t0, t0+take) of k/v."""
        B, H, T, D = k.shape
        buf = page._buf
        ptrs = [buf[n].data_ptr() if buf[n] is not None else None
                for n in ("k", "v", "scale_k", "scale_v")]
        _native.call("si_page_write", k.data_ptr(), v.data_ptr(), _native.dtype_code(k.dtype),
                     B, H, T, D, t0, take, _PREC_CODE[page.precision], self._int4_effective_group,
                     _native.table4(ptrs), page.capacity, offset, _native.stream(k.device))

    def _prepare(self, k_new: torch.Tensor, v_new: torch.Tensor):
        _native.require_device(k_new, "PagedKVStore")
        if v_new.device != k_new.device or v_new.dtype != k_new.dtype:
            raise ValueError("k_new and v_new must share device and dtype")
        _native.dtype_code(k_new.dtype)
        return k_new.detach().contiguous(), v_new.detach().contiguous()

    # ------------------------------------------------------------------ append
    def append(self, k_new: torch.Tensor, v_new: torch.Tensor, precision: str) -> None:
        """Append tokens; sealed pages are never touched (paged_kv_store.py:248-307)."""
        self._validate_kv(k_new, v_new, precision, "append")
        tokens = int(k_new.shape[2])
        if tokens == 0:
            return
        k, v = self._prepare(k_new, v_new)
        self._table = None
        if self._dtype is not None and k.dtype != self._dtype:
            self._seal_tail()  # a page holds one input dtype
        self._dtype = k.dtype
        cursor = 0
        while cursor < tokens:
            open_slot = self._open_slot(precision)
            full = (tokens - cursor) // self.page_size
            if open_slot is None and full >= 2:
                # a run of whole new pages: one allocation per buffer, one launch
                self._append_pages(k, v, cursor, full, precision)
                cursor += full * self.page_size
                continue
            if open_slot is None:
                capacity = self.page_size
            else:
                capacity = self.page_size - self.pages[open_slot].num_tokens
            take = min(capacity, tokens - cursor)
            if open_slot is None:
                slot = self._alloc_slot()
                self._order.append(slot)
                page = _Page(precision, self._new_buffers(precision, k.dtype, k.device),
                             self._max_seq, 0, False)
                self._write(page, k, v, cursor, take, 0)
                page._set_tokens(take)
                page.sealed = take == self.page_size
                self.pages[slot] = page
            else:
                page = self.pages[open_slot]
                self._write(page, k, v, cursor, take, page.num_tokens)
                page._set_tokens(page.num_tokens + take)
                page.sealed = page.num_tokens == self.page_size
            cursor += take
            self._max_seq += take
        self._appended_tokens += tokens

    def _append_pages(self, k: torch.Tensor, v: torch.Tensor, t0: int, count: int,
                      precision: str) -> None:
        """``count`` sealed pages holding tokens [t0, t0 + count * page_size)."""
        B, H, T, D = k.shape
        P = self.page_size
        bufs = self._new_buffers(precision, k.dtype, k.device, count=count)
        ptrs = [bufs[n].data_ptr() if bufs[n] is not None else None
                for n in ("k", "v", "scale_k", "scale_v")]
        _native.call("si_page_write_pages", k.data_ptr(), v.data_ptr(), _native.dtype_code(k.dtype),
                     B, H, T, D, t0, count, _PREC_CODE[precision], self._int4_effective_group,
                     _native.table4(ptrs), P, _native.stream(k.device))
        for i in range(count):
            slot = self._alloc_slot()
            self._order.append(slot)
            buf = {n: (None if t is None else t[i]) for n, t in bufs.items()}
            self.pages[slot] = _Page(precision, buf, self._max_seq, P, True)
            self._max_seq += P

    def _seal_tail(self) -> None:
        if self._order:
            page = self.pages[self._order[-1]]
            if page is not None:
                page.sealed = True

    def _open_slot(self, precision: str) -> Optional[int]:
        """paged_kv_store.py:309-324."""
        if not self._order:
            return None
        slot = self._order[-1]
        page = self.pages[slot]
        if page is None or page.sealed:
            return None
        if page.precision != precision:
            page.sealed = True
            return None
        return slot

    def _alloc_slot(self) -> int:
        if self._free_slots:
            return self._free_slots.pop()
        self.pages.append(None)
        return len(self.pages) - 1

    # ------------------------------------------------------------------ gather
    def gather(self) -> Tuple[torch.Tensor, torch.Tensor]:
        """Dense float32 (k, v) ``[B, H, max_seq, D]`` (paged_kv_store.py:326-376):
        page rows decoded in one launch; rows no page covers are zero."""
        B, H, D = self.batch_size, self.num_heads, self.head_dim
        live = [self.pages[s] for s in self._order if self.pages[s] is not None]
        if not self._order:
            empty = torch.zeros(B, H, 0, D, dtype=torch.float32, device=self.device)
            return empty, empty.clone()
        dev = live[0].k.device if live else self.device
        # Pages in token order with no gap: the output ends with the last page
        # (the reference concatenates them); otherwise it spans max_seq with
        # zeros in the holes.
        expected, contiguous = 0, len(live) == len(self._order)
        for p in live:
            if p.start_token != expected:
                contiguous = False
            expected = p.end_token
        S = expected if contiguous else self._max_seq
        alloc = torch.empty if contiguous else torch.zeros
        k_out = alloc(B, H, S, D, dtype=torch.float32, device=dev)
        v_out = alloc(B, H, S, D, dtype=torch.float32, device=dev)
        if not live or S == 0:
            return k_out, v_out
        if self._table is None or self._table.device != dev:
            rows = []
            for p in live:
                b = p._buf
                rows.append([_PREC_CODE[p.precision], b["k"].data_ptr(), b["v"].data_ptr(),
                             b["scale_k"].data_ptr() if b["scale_k"] is not None else 0,
                             b["scale_v"].data_ptr() if b["scale_v"] is not None else 0,
                             p.start_token, p.num_tokens, p.capacity])
            self._table = torch.tensor(rows, dtype=torch.int64).to(dev)
        table = self._table
        _native.call("si_page_gather", table.data_ptr(), int(table.shape[0]),
                     _native.dtype_code(self._dtype), B, H, S, D, self._int4_effective_group,
                     k_out.data_ptr(), v_out.data_ptr(), _native.stream(dev))
        return k_out, v_out

    # ------------------------------------------------------------------ rewrite
    def rewrite_tokens(self, start_token: int, k_new: torch.Tensor, v_new: torch.Tensor,
                       precision: str) -> int:
        """Overwrite token rows [start, start+T) in place through the append
        path's row quantizers (paged_kv_store.py:407-447). Everything is
        validated before the first write."""
        start = int(start_token)
        self._validate_kv(k_new, v_new, precision, "rewrite")
        tokens = int(k_new.shape[2])
        if tokens < 1:
            raise ValueError(f"rewrite interval must cover at least one token, got {tokens}")
        if start < 0 or start + tokens > self._max_seq:
            raise ValueError(
                f"rewrite interval [{start},{start + tokens}) exceeds stored range "
                f"[0,{self._max_seq})")
        end = start + tokens
        hits = self._plan_rewrite(start, end, precision)
        k, v = self._prepare(k_new, v_new)
        if k.dtype != self._dtype:
            raise ValueError(f"rewrite dtype {k.dtype} differs from the stored {self._dtype}")
        for page, g0, g1 in hits:
            self._write(page, k, v, g0 - start, g1 - g0, g0 - page.start_token)
        self._rewritten_tokens += end - start
        self._rewritten_pages += len(hits)
        return end - start

    def _plan_rewrite(self, start: int, end: int, precision: str):
        """paged_kv_store.py:486-525."""
        hits = []
        covered = 0
        for slot in self._order:
            page = self.pages[slot]
            if page is None:
                continue
            lo = max(start, page.start_token)
            hi = min(end, page.end_token)
            if lo >= hi:
                continue
            if page.precision != precision:
                raise ValueError(
                    "rewrite precision does not match hit page: requested "
                    f"{precision}, page holds {page.precision}")
            hits.append((page, lo, hi))
            covered += hi - lo
        if covered != end - start:
            raise ValueError(
                f"rewrite interval [{start},{end}) is not fully covered by pages "
                f"({covered} of {end - start} tokens); evicted holes cannot be rewritten")
        evicted_tokens = {token for token, _ in self._evicted_pairs}
        for token in range(start, end):
            if token in evicted_tokens:
                raise ValueError(
                    f"rewrite interval [{start},{end}) contains evicted token {token}; "
                    "evicted positions cannot be rewritten")
        return hits

    # ------------------------------------------------------------------ accounting
    def data_plane_bytes(self) -> int:
        """Payload + scale bytes of the filled rows (paged_kv_store.py:527-537)."""
        total = 0
        for slot in self._order:
            page = self.pages[slot]
            if page is None:
                continue
            for t in (page.k, page.v, page.scale_k, page.scale_v):
                if t is not None:
                    total += t.numel() * t.element_size()
        return total

    def resident_bytes(self) -> int:
        """paged_kv_store.py:539-554."""
        data = self.data_plane_bytes()
        if not self._order:
            return 0
        tokens = sum(self.pages[s].num_tokens for s in self._order if self.pages[s] is not None)
        return data + 48 * self.batch_size * self.num_heads * tokens + 16 * len(self.pages)

    # ------------------------------------------------------------------ eviction
    def evict_tokens(self, token_head_set: Set[Tuple[int, int]]) -> int:
        """Page-local eviction (paged_kv_store.py:556-609): fully evicted
        tokens leave their page (which splits into runs of survivors),
        partially evicted tokens keep their place with the evicted head rows
        zeroed. Returns the (token, head) pairs newly removed."""
        if not token_head_set or not self._order:
            return 0
        removed = 0
        runs_by_slot: Dict[int, List[_Page]] = {}
        retired: Set[int] = set()
        for slot in list(self._order):
            page = self.pages[slot]
            if page is None:
                continue
            page_removed, runs = self._plan_eviction(page, token_head_set)
            if page_removed == 0:
                continue
            removed += page_removed
            self._page_evictions += 1
            if runs:
                runs_by_slot[slot] = runs
            else:
                retired.add(slot)
        if removed == 0:
            return 0
        self._table = None
        for slot in retired:
            self.pages[slot] = None
            self._free_slots.append(slot)
        new_order: List[int] = []
        for slot in self._order:
            if slot in retired:
                continue
            runs = runs_by_slot.get(slot)
            if runs is None:
                new_order.append(slot)
                continue
            for i, run_page in enumerate(runs):
                if i == 0:
                    self.pages[slot] = run_page
                    new_order.append(slot)
                else:
                    new_slot = self._alloc_slot()
                    self.pages[new_slot] = run_page
                    new_order.append(new_slot)
        self._order = new_order
        return removed

    def _plan_eviction(self, page: _Page, token_head_set: Set[Tuple[int, int]]):
        """paged_kv_store.py:618-698: survivor runs as new pages."""
        removed = 0
        kept: List[bool] = []
        partial: Dict[int, List[int]] = {}
        for i in range(page.num_tokens):
            token = page.start_token + i
            evicted = [h for h in range(self.num_heads)
                       if (token, h) in token_head_set and (token, h) not in self._evicted_pairs]
            removed += len(evicted)
            for h in evicted:
                self._evicted_pairs.add((token, h))
            if len(evicted) == self.num_heads:
                kept.append(False)
            else:
                kept.append(True)
                if evicted:
                    partial[i] = evicted
        if removed == 0:
            return 0, []
        runs: List[Tuple[int, int]] = []
        i, total = 0, page.num_tokens
        while i < total:
            if not kept[i]:
                i += 1
                continue
            j = i
            while j < total and kept[j]:
                j += 1
            runs.append((i, j))
            i = j
        out: List[_Page] = []
        dev = page.k.device
        for run_index, (ri, rj) in enumerate(runs):
            buf = self._new_buffers(page.precision, self._dtype, dev)
            for name in ("k", "v", "scale_k", "scale_v"):
                if buf[name] is not None:
                    buf[name][:, :, : rj - ri].copy_(page._buf[name][:, :, ri:rj])
            fill = 0x88 if page.precision == "int4" else 0  # code 0 in either layout
            for ti, heads in partial.items():
                if ri <= ti < rj:
                    for h in heads:
                        buf["k"][:, h, ti - ri].fill_(fill)
                        buf["v"][:, h, ti - ri].fill_(fill)
            sealed = page.sealed or run_index < len(runs) - 1 or (rj - ri) == self.page_size
            out.append(_Page(page.precision, buf, page.start_token + ri, rj - ri, sealed))
        return removed, out

    # ------------------------------------------------------------------ reset
    def clear(self) -> None:
        """paged_kv_store.py:700-710."""
        self.pages = []
        self._order = []
        self._free_slots = []
        self._max_seq = 0
        self._appended_tokens = 0
        self._page_evictions = 0
        self._rewritten_tokens = 0
        self._rewritten_pages = 0
        self._evicted_pairs = set()
        self._dtype = None
        self._table = None

    def __repr__(self) -> str:
        return (f"PagedKVStore(batch={self.batch_size}, heads={self.num_heads}, "
                f"head_dim={self.head_dim}, page_size={self.page_size}, "
                f"max_seq={self._max_seq}, pages={self.page_count})")
