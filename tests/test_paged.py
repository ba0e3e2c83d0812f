"""PagedKVStore (shadowinfer/shadowkv/paged_kv_store.py) on the device.

The reference pins its paged store to the packed cache:
tests/test_paged_kv_execution.py compares ``gather()`` bit for bit with
``PackedKVCache.pack(...).unpack()`` (and with ``pack -> evict -> unpack``
after evictions), since both quantize per (b, h, token) row. These tests
do the same against the oracle's pack/unpack/evict, over the reference's
scenarios (stepwise appends across page boundaries, group fallback, sealed
page immutability, statistics, byte accounting, validation, mixed
precisions, eviction and slot recycling) plus bf16 inputs, rewrites and a
7B-layer-sized prefill.
"""

import numpy as np
import pytest
import torch

from helpers import DT, to_np
from oracle import oracle as O

B, H, D, S, P = 2, 4, 32, 19, 8
SPLIT = (5, 5, 5, 4)
CODE = {"fp32": 0, "fp16": 1, "int8": 2, "int4": 3}


def _kv(seed, b=B, h=H, s=S, d=D, dtype=torch.float32):
    g = torch.Generator().manual_seed(seed)
    k = torch.randn(b, h, s, d, generator=g) * 2.0
    v = torch.randn(b, h, s, d, generator=g) * 2.0
    return k.to(dtype), v.to(dtype)


def _store(dev, b=B, h=H, d=D, page=P):
    from shadowinfer_amd.shadowkv import PagedKVStore
    return PagedKVStore(b, h, d, page_size=page, device=dev, int4_group_size=16)


def _golden(k, v, precision, evict=()):
    """Oracle pack with every entry at ``precision`` -> evict -> unpack (fp32)."""
    s, h = k.shape[2], k.shape[1]
    codes = np.full((s, h), CODE[precision], np.int8)
    cache = O.kv_pack(to_np(k), to_np(v), DT[k.dtype], codes, 16)
    if evict:
        O.kv_evict(cache, set(evict))
    uk, uv = O.kv_unpack(cache)
    return uk, uv


def _append(store, k, v, precision, split=SPLIT, dev=None):
    t = 0
    for n in split:
        store.append(k[:, :, t:t + n].to(dev), v[:, :, t:t + n].to(dev), precision)
        t += n


def _eq(a, b):
    np.testing.assert_array_equal(to_np(a) if isinstance(a, torch.Tensor) else a,
                                  to_np(b) if isinstance(b, torch.Tensor) else b)


def _pairs(full=(), partial=()):
    out = {(t, h) for t in full for h in range(H)}
    for t, hs in partial:
        out |= {(t, h) for h in hs}
    return out


# ------------------------------------------------------------------ host (CPU)
def test_validation_and_empty_store_on_host():
    from shadowinfer_amd.shadowkv import PagedKVStore
    st = PagedKVStore(B, H, D, page_size=P)
    assert (st.max_seq, st.page_count, st.open_pages, st.appended_tokens, st.page_evictions) == (0,) * 5
    assert st.data_plane_bytes() == 0 and st.resident_bytes() == 0
    k, v = st.gather()
    assert k.shape == (B, H, 0, D) and k.dtype == torch.float32
    st.validate_against(B, H, D)
    for bad in ((B + 1, H, D), (B, H + 1, D), (B, H, D + 8)):
        with pytest.raises(ValueError):
            st.validate_against(*bad)
    x = torch.randn(B, H, 3, D)
    for prec in ("int3", "fp8"):
        with pytest.raises(ValueError):
            st.append(x, x, prec)
    for kb, vb in ((torch.randn(B, H, 3, 16), torch.randn(B, H, 3, 16)),
                   (torch.randn(B, 5, 3, D), torch.randn(B, 5, 3, D)),
                   (torch.randn(3, H, 3, D), torch.randn(3, H, 3, D)),
                   (torch.randn(B, H, D), torch.randn(B, H, D)),
                   (torch.randn(B, H, 3, D), torch.randn(B, H, 3, D + 8))):
        with pytest.raises(ValueError):
            st.append(kb, vb, "fp16")
    assert (st.appended_tokens, st.page_count, st.max_seq) == (0, 0, 0)
    st.append(torch.randn(B, H, 0, D), torch.randn(B, H, 0, D), "int8")  # no-op
    assert st.page_count == 0
    with pytest.raises(ValueError):
        PagedKVStore(B, H, D, page_size=0)


# ------------------------------------------------------------------ HIP (GPU)
@pytest.mark.gpu
@pytest.mark.parametrize("precision", ["fp32", "fp16", "int8", "int4"])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_gather_golden_stepwise(dev, precision, dtype):
    k, v = _kv(2026, dtype=dtype)
    st = _store(dev)
    _append(st, k, v, precision, dev=dev)
    gk, gv = st.gather()
    assert gk.shape == (B, H, S, D) and gk.dtype == torch.float32
    wk, wv = _golden(k, v, precision)
    _eq(gk, wk)
    _eq(gv, wv)
    assert st.page_count == 3 and st.open_pages == 1 and st.appended_tokens == S


@pytest.mark.gpu
def test_single_append_spans_pages_and_group_fallback(dev):
    k, v = _kv(7)
    st = _store(dev)
    st.append(k.to(dev), v.to(dev), "int8")
    _eq(st.gather()[0], _golden(k, v, "int8")[0])
    k, v = _kv(8, s=11, d=24)  # 24 % 16 != 0: one int4 group per row
    st = _store(dev, d=24, page=4)
    _append(st, k, v, "int4", split=(4, 4, 3), dev=dev)
    gk, gv = st.gather()
    wk, wv = _golden(k, v, "int4")
    _eq(gk, wk)
    _eq(gv, wv)
    k, v = _kv(9, s=6, d=45, dtype=torch.bfloat16)  # odd head dim: generic row path
    st = _store(dev, d=45, page=4)
    _append(st, k, v, "int4", split=(3, 3), dev=dev)
    _eq(st.gather()[1], _golden(k, v, "int4")[1])


@pytest.mark.gpu
def test_sealed_pages_immutable_and_statistics(dev):
    k, v = _kv(11)
    st = _store(dev)
    _append(st, k, v, "fp16", split=(5, 5), dev=dev)
    assert len(st.pages) == 2
    p0 = st.pages[0]
    ptr0 = (p0.k.data_ptr(), p0.v.data_ptr())
    _append(st, k[:, :, 10:], v[:, :, 10:], "fp16", split=(5, 4), dev=dev)
    assert len(st.pages) == 3 and st.pages[0] is p0
    assert (st.pages[0].k.data_ptr(), st.pages[0].v.data_ptr()) == ptr0
    p1 = st.pages[1]
    ptr1 = p1.k.data_ptr()
    ek, ev = _kv(12, s=3)
    st.append(ek.to(dev), ev.to(dev), "fp16")
    assert st.appended_tokens == 22 and st.pages[1] is p1 and st.pages[1].k.data_ptr() == ptr1
    assert st.page_count == 3 and st.open_pages == 1 and st.max_seq == 22
    gk, _ = st.gather()
    _eq(gk[:, :, :S], _golden(k, v, "fp16")[0])
    _eq(gk[:, :, S:], _golden(ek, ev, "fp16")[0])


@pytest.mark.gpu
def test_byte_accounting(dev):
    k, v = _kv(13)
    for prec, per in (("fp16", 2 * 2), ("fp32", 4 * 2)):
        st = _store(dev)
        _append(st, k, v, prec, dev=dev)
        assert st.data_plane_bytes() == B * H * S * D * per
        assert st.resident_bytes() == st.data_plane_bytes() + 48 * B * H * S + 16 * len(st.pages)
    G = D // 16
    for prec, per_row in (("int8", 2 * (D + 4)), ("int4", 2 * (D // 2 + G * 4))):
        st = _store(dev)
        _append(st, k, v, prec, dev=dev)
        assert st.data_plane_bytes() == B * H * S * per_row
        assert 0 < st.data_plane_bytes() < B * H * S * D * 2 * 2


@pytest.mark.gpu
def test_mixed_precision_pages(dev):
    k, v = _kv(14, s=8)
    st = _store(dev, page=4)
    st.append(k[:, :, 0:4].to(dev), v[:, :, 0:4].to(dev), "fp16")
    st.append(k[:, :, 4:8].to(dev), v[:, :, 4:8].to(dev), "int8")
    gk, gv = st.gather()
    _eq(gk[:, :, :4], _golden(k[:, :, :4], v[:, :, :4], "fp16")[0])
    _eq(gv[:, :, 4:], _golden(k[:, :, 4:], v[:, :, 4:], "int8")[1])
    # a precision change seals the open tail page
    st = _store(dev, page=8)
    st.append(k[:, :, 0:3].to(dev), v[:, :, 0:3].to(dev), "int4")
    st.append(k[:, :, 3:5].to(dev), v[:, :, 3:5].to(dev), "fp32")
    assert st.page_count == 2 and st.open_pages == 1 and st.pages[0].sealed


@pytest.mark.gpu
@pytest.mark.parametrize("precision,full,partial,removed", [
    ("fp16", (2, 4, 5, 17), ((10, (0, 1)), (12, (2, 3))), 20),
    ("int8", (3, 16), ((9, (0, 2)),), 10),
    ("int4", (5, 15), ((11, (1, 3)),), 10),
    ("fp32", (18,), ((7, (3,)),), 5),
])
def test_evict_golden(dev, precision, full, partial, removed):
    k, v = _kv(2026)
    st = _store(dev)
    _append(st, k, v, precision, dev=dev)
    ev = _pairs(full, partial)
    assert st.evict_tokens(set(ev)) == removed
    gk, gv = st.gather()
    wk, wv = _golden(k, v, precision, ev)
    if 18 in full:  # a trailing hole: the pages end before max_seq
        assert gk.shape[2] == S - 1
        wk, wv = wk[:, :, :S - 1], wv[:, :, :S - 1]
    _eq(gk, wk)
    _eq(gv, wv)


@pytest.mark.gpu
def test_evict_bytes_slots_and_segments(dev):
    k, v = _kv(2026)
    per_token = B * H * D * 2 * 2
    st = _store(dev)
    _append(st, k, v, "fp16", dev=dev)
    before = st.data_plane_bytes()
    assert st.evict_tokens(_pairs((4, 5), ((6, (0, 1)),))) == 10
    assert st.data_plane_bytes() == before - 2 * per_token and st.page_evictions >= 1
    # partial heads save no bytes
    st = _store(dev)
    _append(st, k, v, "fp16", dev=dev)
    before, res = st.data_plane_bytes(), st.resident_bytes()
    assert st.evict_tokens(_pairs((), ((7, (0, 1)), (11, (2, 3))))) == 4
    assert (st.data_plane_bytes(), st.resident_bytes()) == (before, res)
    # a whole page leaves the order and its slot is reused
    k12, v12 = _kv(2026, s=12)
    st = _store(dev, page=4)
    _append(st, k12, v12, "fp16", split=(4, 4, 4), dev=dev)
    assert st.evict_tokens(_pairs((4, 5, 6, 7))) == 16
    assert len(st.pages) == 3 and st.page_count == 2 and st.data_plane_bytes() == 8 * per_token
    mid = st.gather()[0]
    assert mid.shape[2] == 12 and torch.count_nonzero(mid[:, :, 4:8]) == 0
    ek, ev = _kv(2028, s=2)
    st.append(ek.to(dev), ev.to(dev), "fp16")
    assert len(st.pages) == 3 and st.page_count == 3 and st.max_seq == 14
    after = st.gather()[0]
    _eq(after[:, :, 12:], _golden(ek, ev, "fp16")[0])
    _eq(after[:, :, :12], mid)
    # a mid-page hole splits the page
    st = _store(dev)
    _append(st, k, v, "fp16", dev=dev)
    p1, p2 = st.pages[1], st.pages[2]
    assert st.evict_tokens(_pairs((3,))) == 4
    segs = sorted((p.start_token, p.end_token) for p in st.pages if p is not None)
    assert segs == [(0, 3), (4, 8), (8, 16), (16, 19)]
    assert st.pages[1] is p1 and st.pages[2] is p2
    # empty set, absent and already-evicted positions
    assert st.evict_tokens(set()) == 0
    assert st.evict_tokens({(3, 0), (3, 3), (S + 5, 0), (0, H + 3)}) == 0
    ek, ev = _kv(2029, s=2)
    st.append(ek.to(dev), ev.to(dev), "fp16")
    g = st.gather()[0]
    assert g.shape[2] == S + 2 and torch.count_nonzero(g[:, :, 3]) == 0


@pytest.mark.gpu
@pytest.mark.parametrize("precision", ["fp16", "int8", "int4"])
def test_rewrite_tokens_equals_fresh_append(dev, precision):
    k, v = _kv(30)
    k2, v2 = _kv(31)
    st = _store(dev)
    _append(st, k, v, precision, dev=dev)
    n = st.rewrite_tokens(6, k2[:, :, 6:13].to(dev), v2[:, :, 6:13].to(dev), precision)
    assert n == 7 and st.rewritten_tokens == 7 and st.rewritten_pages == 2
    mixed_k = k.clone()
    mixed_v = v.clone()
    mixed_k[:, :, 6:13] = k2[:, :, 6:13]
    mixed_v[:, :, 6:13] = v2[:, :, 6:13]
    gk, gv = st.gather()
    wk, wv = _golden(mixed_k, mixed_v, precision)
    _eq(gk, wk)
    _eq(gv, wv)
    with pytest.raises(ValueError):
        st.rewrite_tokens(15, k2[:, :, :6].to(dev), v2[:, :, :6].to(dev), precision)  # past max_seq
    with pytest.raises(ValueError):
        st.rewrite_tokens(0, k2[:, :, :2].to(dev), v2[:, :, :2].to(dev), "fp32")  # wrong precision
    st.evict_tokens(_pairs((2,)))
    with pytest.raises(ValueError):
        st.rewrite_tokens(1, k2[:, :, :3].to(dev), v2[:, :, :3].to(dev), precision)  # hole


@pytest.mark.gpu
def test_layer_sized_prefill_matches_packed_cache(dev):
    """1 x 32 x 8192 x 128 bf16 int8 prefill in 32-token pages: gather equals
    the device PackedKVCache unpack of the same tokens."""
    from shadowinfer_amd.shadowkv import PackedKVCache, PrecisionPlan
    g = torch.Generator(device=dev).manual_seed(3)
    k = torch.randn(1, 32, 8192, 128, generator=g, device=dev).to(torch.bfloat16)
    v = torch.randn(1, 32, 8192, 128, generator=g, device=dev).to(torch.bfloat16)
    st = _store(dev, b=1, h=32, d=128, page=32)
    st.append(k[:, :, :5000], v[:, :, :5000], "int8")
    st.append(k[:, :, 5000:], v[:, :, 5000:], "int8")
    assert st.page_count == 256
    gk, gv = st.gather()
    codes = torch.full((8192, 32), 2, dtype=torch.int8, device=dev)
    ref = PackedKVCache.pack(k, v, None, plan=PrecisionPlan.from_codes(codes))["packed_kv"]
    rk, rv = ref.unpack()
    assert torch.equal(gk, rk) and torch.equal(gv, rv)


@pytest.mark.gpu
@pytest.mark.parametrize("precision", ["fp32", "fp16", "int8", "int4"])
@pytest.mark.parametrize("dtype,d", [(torch.bfloat16, 32), (torch.float32, 32), (torch.bfloat16, 45)])
def test_page_runs_equal_page_by_page(dev, precision, dtype, d):
    """One append of several whole pages (one allocation, si_page_write_pages)
    leaves the same pages as appending them one page at a time, including
    after a partly filled open page."""
    k, v = _kv(21, s=43, d=d, dtype=dtype)
    a, b = _store(dev, d=d), _store(dev, d=d)
    a.append(k[:, :, :3].to(dev), v[:, :, :3].to(dev), precision)      # open page of 3
    a.append(k[:, :, 3:].to(dev), v[:, :, 3:].to(dev), precision)      # fills it, 4 whole pages, tail
    _append(b, k, v, precision, split=(3, 5, 8, 8, 8, 8, 3), dev=dev)
    assert a.page_count == b.page_count == 6
    for pa, pb in zip(a.pages, b.pages):
        assert (pa.start_token, pa.num_tokens, pa.sealed) == (pb.start_token, pb.num_tokens, pb.sealed)
        for name in ("k", "v", "scale_k", "scale_v"):
            ta, tb = getattr(pa, name), getattr(pb, name)
            assert (ta is None) == (tb is None)
            if ta is not None:
                assert ta.shape == tb.shape and torch.equal(ta, tb), name
    ga, gb = a.gather(), b.gather()
    assert torch.equal(ga[0], gb[0]) and torch.equal(ga[1], gb[1])
    wk, wv = _golden(k, v, precision)
    _eq(ga[0], wk)
    _eq(ga[1], wv)
    assert a.data_plane_bytes() == b.data_plane_bytes()


@pytest.mark.gpu
@pytest.mark.parametrize("precision", ["fp32", "fp16", "int8", "int4"])
def test_pages_of_different_input_dtypes(dev, precision):
    """Appends of bf16 and fp32 rows into one store: a new page keeps the
    dtype of its rows, an open page takes rows of another dtype by widening to
    torch.promote_types of the two (the reference's torch.cat of the page and
    the new rows promotes the same way), and gather decodes every page in its
    own dtype: the result equals the oracle decode of each segment in its
    input dtype."""
    kb, vb = _kv(40, s=16, dtype=torch.bfloat16)
    kf, vf = _kv(41, s=16)
    st = _store(dev)                                                     # pages of 8
    st.append(kb[:, :, :8].to(dev), vb[:, :, :8].to(dev), precision)   # sealed bf16 page
    st.append(kf[:, :, :5].to(dev), vf[:, :, :5].to(dev), precision)   # open fp32 page
    st.append(kb[:, :, 8:10].to(dev), vb[:, :, 8:10].to(dev), precision)  # bf16 rows, fp32 page
    assert st.page_count == 2 and [p.dtype for p in st.pages] == [torch.bfloat16, torch.float32]
    gk, gv = st.gather()
    for got, want in ((gk[:, :, :8], _golden(kb[:, :, :8], vb[:, :, :8], precision)),
                      (gk[:, :, 8:13], _golden(kf[:, :, :5], vf[:, :, :5], precision)),
                      (gk[:, :, 13:15], _golden(kb[:, :, 8:10], vb[:, :, 8:10], precision))):
        _eq(got, want[0])
    _eq(gv[:, :, 8:13], _golden(kf[:, :, :5], vf[:, :, :5], precision)[1])
    # an open bf16 page that receives fp32 rows widens to fp32 (one page)
    st2 = _store(dev)
    st2.append(kb[:, :, :3].to(dev), vb[:, :, :3].to(dev), precision)
    st2.append(kf[:, :, :4].to(dev), vf[:, :, :4].to(dev), precision)
    assert st2.page_count == 1 and st2.pages[0].dtype == torch.float32
    g2k, g2v = st2.gather()
    _eq(g2k[:, :, :3], _golden(kb[:, :, :3], vb[:, :, :3], precision)[0])
    _eq(g2v[:, :, 3:], _golden(kf[:, :, :4], vf[:, :, :4], precision)[1])


@pytest.mark.gpu
def test_rewrite_with_another_input_dtype(dev):
    """fp32 rows rewritten into a bf16 int8 page: quantized in fp32, then the
    scales stored in the page's bf16 (the reference's copy_ into the page)."""
    kb, vb = _kv(42, s=8, dtype=torch.bfloat16)
    kf, vf = _kv(43, s=8)
    st = _store(dev)
    st.append(kb.to(dev), vb.to(dev), "int8")
    st.rewrite_tokens(2, kf[:, :, 2:5].to(dev), vf[:, :, 2:5].to(dev), "int8")
    gk, _ = st.gather()
    rows = to_np(kf[:, :, 2:5])                                          # [B, H, 3, D] fp32
    q, s = O.quant_rows_i8(rows, O.F32)
    s16 = O.from_f32(s, O.BF16)
    want = O.dequant_rows(q, s16, O.BF16, D)
    _eq(gk[:, :, 2:5], want)
    _eq(gk[:, :, :2], _golden(kb[:, :, :2], vb[:, :, :2], "int8")[0])
