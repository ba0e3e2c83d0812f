"""GPU parity tests: PrecisionPlan / PackedKVCache HIP kernels vs the oracle.

Bar: bucket bytes, scales, indices and byte counts bit-exact; unpack output
bit-exact (fp32); eviction and reuse bit-exact with the oracle's restatement
of packed_kv_cache.py.
"""

import numpy as np
import pytest
import torch

from helpers import assert_cache_equal, kv_inputs, mixed_codes, oracle_pack, to_np
from oracle import oracle as O
from shadowinfer_amd.shadowkv import PackedKVCache, PrecisionPlan, codes_to_map

pytestmark = pytest.mark.gpu

DTYPES = [torch.float32, torch.bfloat16, torch.float16]


def _pack(k, v, codes, dev, group_size=16):
    plan = PrecisionPlan.from_codes(torch.from_numpy(codes).to(dev))
    return PackedKVCache.pack(k.to(dev), v.to(dev), None, group_size=group_size,
                              plan=plan)["packed_kv"]


# ----------------------------------------------------------------- plan scan
@pytest.mark.parametrize("S,H", [(1, 1), (5, 3), (64, 4), (512, 8), (4097, 3), (8192, 32)])
def test_plan_from_codes_matches_oracle(dev, S, H):
    rng = np.random.default_rng(S * 131 + H)
    codes = rng.integers(-1, 6, size=(S, H)).astype(np.int8)  # includes unknown -1 and 5
    mask = {(int(t), int(h)): bool(rng.random() < 0.3) for t in range(min(S, 64)) for h in range(H)}
    plan = PrecisionPlan.from_codes(torch.from_numpy(codes).to(dev), reuse_mask=mask)
    ref = O.plan_from_codes(codes, mask)
    assert plan.counts[:4] == [len(ref["groups"][p]) for p in O.PRECISIONS]
    for p in O.PRECISIONS:
        assert plan.flat_indices[p].device.type == "cuda"
        np.testing.assert_array_equal(plan.flat_indices[p].cpu().numpy(), ref["flat_indices"][p])
        assert plan.groups[p] == ref["groups"][p]
    assert plan.evicted_entries == ref["evicted_entries"]
    assert plan.reuse_entries == ref["reuse_entries"]
    np.testing.assert_array_equal(plan.reuse_flat.cpu().numpy(), ref["reuse_flat"])
    assert plan.fingerprint == ref["fingerprint"]


@pytest.mark.parametrize("S,H", [(1, 1), (7, 3), (1000, 3), (8192, 32), (40000, 32)])
def test_plan_scan_lists_matches_scan_then_scatter(dev, S, H):
    """The evict rescan with its flat lists in one pass (si_plan_scan_lists)
    gives the code / slot / counts of si_plan_scan and the lists of
    si_plan_scatter, on the fused path and (40000 x 32: above 2^20 entries)
    on the three-pass fallback; no list is written at or past its capacity."""
    from shadowinfer_amd import _native
    import ctypes
    rng = np.random.default_rng(S + H)
    codes = torch.from_numpy(rng.integers(-1, 6, size=S * H).astype(np.int8)).to(dev)
    mask = torch.from_numpy((rng.random(S * H) < 0.3).astype(np.uint8)).to(dev)
    n = S * H
    sp = _native.stream(dev)
    ws_b = _native.size_query("si_plan_workspace_bytes", n)
    ws = torch.empty(ws_b, dtype=torch.uint8, device=dev)
    code0 = torch.empty(n, dtype=torch.int8, device=dev)
    slot0 = torch.empty(n, dtype=torch.int32, device=dev)
    cnt0 = torch.empty(5, dtype=torch.int64, device=dev)
    _native.call("si_plan_scan", codes.data_ptr(), mask.data_ptr(), n, code0.data_ptr(),
                 slot0.data_ptr(), cnt0.data_ptr(), ws.data_ptr(), ws_b, sp)
    counts = [int(c) for c in cnt0.tolist()]
    ref = [torch.empty(counts[p], dtype=torch.long, device=dev) for p in range(4)]
    _native.call("si_plan_scatter", code0.data_ptr(), slot0.data_ptr(), S, H,
                 _native.table4([r.data_ptr() for r in ref]), _native.table4([None] * 4), sp)
    # lists one row short of the new sizes, inside buffers with a sentinel tail
    cap = [max(c - 1, 0) for c in counts[:4]]
    bufs = [torch.full((c + 8,), -7, dtype=torch.long, device=dev) for c in cap]
    code1 = torch.empty_like(code0)
    slot1 = torch.empty_like(slot0)
    cnt1 = torch.empty_like(cnt0)
    _native.call("si_plan_scan_lists", codes.data_ptr(), mask.data_ptr(), S, H, code1.data_ptr(),
                 slot1.data_ptr(), cnt1.data_ptr(), _native.table4([b.data_ptr() for b in bufs]),
                 (ctypes.c_int64 * 4)(*cap), ws.data_ptr(), ws_b, sp)
    assert torch.equal(code1, code0) and torch.equal(slot1, slot0) and torch.equal(cnt1, cnt0)
    for p in range(4):
        assert torch.equal(bufs[p][: cap[p]], ref[p][: cap[p]])
        assert bool((bufs[p][cap[p]:] == -7).all())


@pytest.mark.parametrize("S,H,B,D,dtype,whole", [(7, 3, 1, 32, torch.float32, False),
                                                  (300, 8, 2, 64, torch.bfloat16, True),
                                                  (1000, 5, 1, 45, torch.float16, False),
                                                  (2048, 32, 1, 128, torch.bfloat16, False)])
def test_evict_passes_match_rescan_and_compaction(dev, S, H, B, D, dtype, whole):
    """si_kv_evict_count + si_kv_evict_flat (the passes PackedKVCache.evict
    runs) give the codes, slots and sizes of si_plan_scan with the mask, the
    lists of si_plan_scatter and the buckets of si_kv_compact_flat. Unknown
    codes (-1, 5) and absent entries come out as code 4 / slot -1; no list is
    written past its new size; a precision with nothing evicted (NULL new
    bucket pointer) keeps its rows; ``whole`` evicts every int4 entry."""
    import ctypes
    from shadowinfer_amd import _native
    from shadowinfer_amd.shadowkv.precision_plan import DeviceGrouping
    k, v = kv_inputs(B, H, S, D, dtype, seed=S)
    codes = mixed_codes(S, H, seed=S + 5, probs=(1, 1, 1, 1), evicted=0.1)
    plan = PrecisionPlan.from_codes(torch.from_numpy(codes).to(dev))
    cache = PackedKVCache.pack(k.to(dev), v.to(dev), None, plan=plan)["packed_kv"]
    code, slot, table, sdt, g = cache.device_state()
    grp = cache._grouping
    n = S * H
    rng = np.random.default_rng(S * 7 + H)
    cnp = code.cpu().numpy()
    m = rng.random(n) < 0.3
    m[cnp == 0] = False          # fp32: nothing evicted, bucket kept as it is
    if whole:
        m[cnp == 3] = True
    mask = torch.from_numpy(m.astype(np.uint8)).to(dev)
    raw = code.clone()             # absent entries given unknown codes too
    absent = np.nonzero(cnp == 4)[0]
    raw[torch.from_numpy(absent[::2]).to(dev)] = -1
    raw[torch.from_numpy(absent[1::2]).to(dev)] = 5
    ref = DeviceGrouping.scan(code, evict_mask=mask)
    ref_flat = ref.flat_lists(S, H)
    sp = _native.stream(dev)
    lib = _native.load()
    old_cnt = (ctypes.c_int64 * 4)(*grp.counts[:4])
    chunks = int(lib.si_kv_evict_chunks(old_cnt))
    words = int(lib.si_kv_evict_chunk_words())
    rows = 64 * words
    assert chunks == sum(-(-c // rows) for c in grp.counts[:4])
    cc = torch.full((max(chunks, 1),), -5, dtype=torch.int32, device=dev)
    bits = torch.full((max(chunks * words, 1),), -5, dtype=torch.int64, device=dev)
    ncode = torch.full((n,), 9, dtype=torch.int8, device=dev)
    nslot = torch.full((n,), -9, dtype=torch.int32, device=dev)
    old_flat = _native.table4([f.data_ptr() for f in grp.flat_lists(S, H)])
    _native.call("si_kv_evict_count", raw.data_ptr(), old_flat, old_cnt, mask.data_ptr(), S, H,
                 ncode.data_ptr(), nslot.data_ptr(), cc.data_ptr(), bits.data_ptr(), sp)
    per = cc[:chunks].cpu().numpy().astype(np.int64)
    pop = [bin(int(x) & (2**64 - 1)).count("1") for x in bits[: chunks * words].cpu().tolist()]
    assert per.tolist() == [sum(pop[words * j: words * j + words]) for j in range(chunks)]
    ends = np.cumsum([-(-c // rows) for c in grp.counts[:4]])
    counts = [int(per[a:b].sum()) for a, b in zip(np.concatenate(([0], ends[:-1])), ends)]
    assert counts == ref.counts[:4]
    assert counts[0] == grp.counts[0] and (not whole or counts[3] == 0)

    def changed_buckets():
        fresh = cache._alloc_buckets(ref.counts, dev, cache._scale_dtype)
        return {name: fresh[name] for name in fresh
                if 0 < ref.counts[_IDX[name]] < grp.counts[_IDX[name]]}

    mine, theirs = changed_buckets(), changed_buckets()
    nflat = [torch.full((c + 4,), -7, dtype=torch.long, device=dev) for c in counts]
    _native.call("si_kv_evict_flat", old_flat, old_cnt, cc.data_ptr(), bits.data_ptr(), S, H, table,
                 _native.table4([f.data_ptr() for f in nflat]), (ctypes.c_int64 * 4)(*counts),
                 cache._bucket_table(mine), nslot.data_ptr(), B, D, g, sdt, sp)
    _native.call("si_kv_compact_flat", slot.data_ptr(), table,
                 _native.table4([f.data_ptr() for f in ref_flat]), (ctypes.c_int64 * 5)(*ref.counts),
                 cache._bucket_table(theirs), S, H, B, D, g, sdt, sp)
    assert torch.equal(ncode, ref.code) and torch.equal(nslot, ref.slot)
    for p in range(4):
        assert torch.equal(nflat[p][: counts[p]], ref_flat[p]), p
        assert bool((nflat[p][counts[p]:] == -7).all()), p
    assert set(mine) == set(theirs) and "fp32" not in mine
    for name, d in mine.items():
        for key, t in d.items():
            if torch.is_tensor(t):
                assert torch.equal(t.view(torch.uint8), theirs[name][key].view(torch.uint8)), (name, key)


_IDX = {"fp32": 0, "fp16": 1, "int8": 2, "int4": 3}


def test_plan_device_matches_host_plan(dev):
    codes = mixed_codes(300, 5, seed=3, probs=(1, 1, 1, 1), evicted=0.1)
    gpu = PrecisionPlan.from_codes(torch.from_numpy(codes).to(dev))
    cpu = PrecisionPlan.from_codes(torch.from_numpy(codes))
    assert gpu.groups == cpu.groups
    assert gpu.evicted_entries == cpu.evicted_entries
    assert gpu.fingerprint == cpu.fingerprint
    for p in O.PRECISIONS:
        assert torch.equal(gpu.flat_indices[p].cpu(), cpu.flat_indices[p])


# ---------------------------------------------------------------------- pack
def test_pack_config1_bit_exact(dev):
    """1 layer, B=1, S=512, H=8, D=64, fp32 K/V, codes uniform over
    {fp16, int8, int4} with a 4-token fp16 sink, int4 group 16."""
    k, v = kv_inputs(1, 8, 512, 64, torch.float32, seed=1)
    codes = mixed_codes(512, 8, seed=1, probs=(0, 1, 1, 1), sink=4)
    cache = _pack(k, v, codes, dev)
    ref = oracle_pack(k, v, codes)
    assert_cache_equal(cache, ref)
    k_out, v_out = cache.unpack()
    rk, rv = O.kv_unpack(ref)
    np.testing.assert_array_equal(k_out.cpu().numpy(), rk)
    np.testing.assert_array_equal(v_out.cpu().numpy(), rv)


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("B,H,S,D,g", [
    (1, 3, 5, 16, 16), (1, 2, 5, 7, 16), (1, 2, 7, 24, 16), (2, 2, 9, 32, 16),
    (1, 4, 16, 128, 16), (2, 3, 6, 48, 16), (3, 2, 5, 64, 32), (1, 2, 33, 128, 128),
    (2, 1, 7, 5, 16), (1, 1, 1, 2, 2), (1, 2, 9, 256, 16),
])
def test_pack_unpack_shapes_bit_exact(dev, dtype, B, H, S, D, g):
    """Shapes of the reference's golden pack tests (odd head_dim row padding,
    batch 2, non-dividing group sizes) plus the fast-path widths."""
    k, v = kv_inputs(B, H, S, D, dtype, seed=B * 1000 + S * 10 + D)
    codes = mixed_codes(S, H, seed=D + S, probs=(1, 1, 1, 1), sink=1, evicted=0.15)
    cache = _pack(k, v, codes, dev, group_size=g)
    ref = oracle_pack(k, v, codes, group_size=g)
    assert_cache_equal(cache, ref)
    k_out, v_out = cache.unpack()
    rk, rv = O.kv_unpack(ref)
    np.testing.assert_array_equal(k_out.cpu().numpy(), rk)
    np.testing.assert_array_equal(v_out.cpu().numpy(), rv)
    k_ref, v_ref = cache.unpack_reference()
    assert torch.equal(k_ref, k_out) and torch.equal(v_ref, v_out)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_pack_layer_7b_bit_exact(dev, dtype):
    """One layer of the 7B shape: B=1, H=32, S=8192, D=128 with 1% outlier
    channels x8, codes 25% fp16 / 50% int8 / 25% int4 and a 4-token fp16 sink."""
    k, v = kv_inputs(1, 32, 8192, 128, dtype, seed=7, outlier_frac=0.01)
    codes = mixed_codes(8192, 32, seed=7, probs=(0, 0.25, 0.5, 0.25), sink=4)
    cache = _pack(k, v, codes, dev)
    ref = oracle_pack(k, v, codes)
    assert_cache_equal(cache, ref)
    k_out, v_out = cache.unpack()
    rk, rv = O.kv_unpack(ref)
    np.testing.assert_array_equal(k_out.cpu().numpy(), rk)
    np.testing.assert_array_equal(v_out.cpu().numpy(), rv)


def test_pack_special_values(dev):
    """Zero rows (scale 1), values at +-amax (+-127 / +-7), ties of the
    half-even rounding and tiny subnormal-scale rows."""
    D = 64
    rows = []
    rows.append(np.zeros(D, np.float32))
    r = np.linspace(-1, 1, D).astype(np.float32); rows.append(r)
    r = np.zeros(D, np.float32); r[0] = 127.0; r[1:9] = np.arange(8) + 0.5; rows.append(r)
    r = np.zeros(D, np.float32); r[0] = 7.0; r[1:16] = np.arange(-7, 8)[:15] + 0.5; rows.append(r)
    r = np.full(D, 1e-39, np.float32); r[3] = -3e-39; rows.append(r)
    r = np.full(D, 6.0e4, np.float32); r[::2] *= -1; rows.append(r)
    r = (np.arange(D) - 31.5).astype(np.float32) / 31.5 * 127; rows.append(r)
    H = len(rows)
    k = torch.from_numpy(np.stack(rows)).reshape(1, H, 1, D)
    for dtype in DTYPES:
        kk = k.to(dtype)
        for code in (1, 2, 3):
            codes = np.full((1, H), code, np.int8)
            cache = _pack(kk, kk, codes, dev)
            assert_cache_equal(cache, oracle_pack(kk, kk, codes))


def test_pack_dict_map_matches_plan(dev):
    """pack() with a precision-map dict (missing -> fp16, 'evicted' skipped,
    unknown names -> fp16) equals the plan-driven pack."""
    k, v = kv_inputs(1, 3, 10, 32, torch.bfloat16, seed=5)
    pmap = {t: {h: ("fp32", "fp16", "int8", "int4", "evicted", "bf16")[(t + 2 * h) % 6]
                for h in range(3)} for t in range(9)}  # token 9 missing -> fp16
    cache = PackedKVCache.pack(k.to(dev), v.to(dev), pmap, group_size=16)["packed_kv"]
    codes = O.pack_map_to_codes(pmap, 10, 3)
    assert_cache_equal(cache, oracle_pack(k, v, codes))


def test_pack_validation_errors(dev):
    k, v = kv_inputs(1, 4, 6, 64, torch.float32, seed=8)
    plan = PrecisionPlan.from_codes(torch.ones(6, 5, dtype=torch.int8, device=dev))
    with pytest.raises(ValueError):
        PackedKVCache.pack(k.to(dev), v.to(dev), None, plan=plan)
    cpu_plan = PrecisionPlan.from_codes(torch.ones(6, 4, dtype=torch.int8))
    with pytest.raises(ValueError):
        PackedKVCache.pack(k.to(dev), v.to(dev), None, plan=cpu_plan)
    good = PrecisionPlan.from_codes(torch.ones(6, 4, dtype=torch.int8, device=dev))
    with pytest.raises(ValueError):
        PackedKVCache.pack(k.to(dev), v[:, :, :5].to(dev), None, plan=good)


def test_pack_is_deterministic(dev):
    k, v = kv_inputs(1, 8, 1000, 128, torch.bfloat16, seed=9)
    codes = mixed_codes(1000, 8, seed=9, probs=(1, 1, 1, 1), evicted=0.1)
    a = _pack(k, v, codes, dev)
    b = _pack(k, v, codes, dev)
    for name in a.packed_data:
        for key in ("k", "v", "scale_k", "scale_v"):
            ta, tb = a.packed_data[name][key], b.packed_data[name][key]
            assert (ta is None and tb is None) or torch.equal(ta, tb)


# ------------------------------------------------------------ unpack routes
@pytest.mark.parametrize("dtype,B,H,S,D", [(torch.bfloat16, 1, 32, 1000, 128),
                                           (torch.float32, 2, 3, 77, 64),
                                           (torch.float16, 2, 5, 130, 128)])
def test_unpack_token_and_bucket_order_agree(dev, dtype, B, H, S, D):
    """si_kv_unpack (64-token tiles sorted by precision) and si_kv_unpack_flat
    (bucket order, used by PackedKVCache.unpack) against the oracle, with
    evicted entries and every precision present."""
    from shadowinfer_amd import _native
    k, v = kv_inputs(B, H, S, D, dtype, seed=S + D)
    codes = mixed_codes(S, H, seed=S, probs=(1, 2, 3, 3), sink=2, evicted=0.1)
    cache = _pack(k, v, codes, dev)
    rk, rv = O.kv_unpack(oracle_pack(k, v, codes))
    fk, fv = cache.unpack()
    np.testing.assert_array_equal(fk.cpu().numpy(), rk)
    np.testing.assert_array_equal(fv.cpu().numpy(), rv)
    code, slot, table, sdt, group = cache.device_state()
    # token-order pack through the ABI into a second set of buckets: same bytes
    from shadowinfer_amd.shadowkv.packed_kv_cache import PackedKVCache as _P
    other = _P(B, H, S, D, device=dev)
    other._group_size, other._scale_dtype, other._grouping = group, dtype, cache._grouping
    other._buckets = other._alloc_buckets(cache._grouping.counts, dev, dtype)
    kd, vd = k.to(dev), v.to(dev)
    _native.call("si_kv_pack", kd.data_ptr(), vd.data_ptr(), _native.dtype_code(dtype),
                 B, H, S, D, group, code.data_ptr(), slot.data_ptr(), other._bucket_table(),
                 _native.stream(dev))
    torch.cuda.synchronize(dev)
    for name, d in cache.packed_data.items():
        for key in ("k", "v", "scale_k", "scale_v"):
            if d[key] is not None:
                assert torch.equal(d[key], other.packed_data[name][key]), (name, key)
    tk = torch.empty(B, H, S, D, dtype=torch.float32, device=dev)
    tv = torch.empty_like(tk)
    _native.call("si_kv_unpack", code.data_ptr(), slot.data_ptr(), table, sdt, B, H, S, D, group,
                 tk.data_ptr(), tv.data_ptr(), _native.stream(dev))
    np.testing.assert_array_equal(tk.cpu().numpy(), rk)
    np.testing.assert_array_equal(tv.cpu().numpy(), rv)


# --------------------------------------------------------------------- evict
def test_evict_config1(dev):
    """Config-1 eviction: the 25% lowest-importance token-heads (stable
    ascending argsort of importance ~ U(0,1) over token-major entries)."""
    k, v = kv_inputs(1, 8, 512, 64, torch.float32, seed=11)
    codes = mixed_codes(512, 8, seed=11, probs=(0, 1, 1, 1), sink=4)
    cache = _pack(k, v, codes, dev)
    ref = oracle_pack(k, v, codes)
    importance = np.random.default_rng(11).random(512 * 8)
    order = np.argsort(importance, kind="stable")[: 512 * 8 // 4]
    victims = {(int(e // 8), int(e % 8)) for e in order}
    removed = cache.evict(victims)
    assert removed == O.kv_evict(ref, victims) == len(victims)
    assert_cache_equal(cache, ref)
    k_out, v_out = cache.unpack()
    rk, rv = O.kv_unpack(ref)
    np.testing.assert_array_equal(k_out.cpu().numpy(), rk)
    np.testing.assert_array_equal(v_out.cpu().numpy(), rv)
    assert cache.evict(victims) == 0  # never resurrected, never counted twice


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_evict_batch2_mixed(dev, dtype):
    k, v = kv_inputs(2, 2, 8, 64, dtype, seed=12)
    codes = np.array([[(t * 2 + h) // 4 % 4 for h in range(2)] for t in range(8)], np.int8)
    cache = _pack(k, v, codes, dev)
    ref = oracle_pack(k, v, codes)
    ordered = sorted(e for d in ref.packed_data.values() for e in d["indices"])
    victims = set(ordered[::4]) | {(100, 0), (0, 7)}  # out-of-range pairs ignored
    assert cache.evict(victims) == O.kv_evict(ref, victims)
    assert_cache_equal(cache, ref)
    assert cache.packed_data["int4"]["group_size"] == 16


def test_evict_whole_buckets_and_empty(dev):
    k, v = kv_inputs(1, 2, 4, 64, torch.float32, seed=13)
    for code in (2, 3):
        codes = np.full((4, 2), code, np.int8)
        cache = _pack(k, v, codes, dev)
        everything = {(t, h) for t in range(4) for h in range(2)}
        assert cache.evict(everything) == 8
        assert cache.memory_bytes() == 0 and cache.resident_bytes() == 0
        ko, vo = cache.unpack()
        assert torch.count_nonzero(ko) == 0 and torch.count_nonzero(vo) == 0
    empty = PackedKVCache(1, 2, 8, 64)
    ko, vo = empty.unpack()
    assert torch.count_nonzero(ko) == 0
    assert empty.evict({(0, 0)}) == 0 and empty.memory_bytes() == 0 and empty.resident_bytes() == 0


# --------------------------------------------------------------------- reuse
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("B,S_prev", [(1, 64), (2, 64), (1, 40)])
def test_apply_reuse_mask_matches_oracle(dev, dtype, B, S_prev):
    S, H, D = 64, 4, 64
    kp, vp = kv_inputs(B, H, S_prev, D, dtype, seed=21)
    kc, vc = kv_inputs(B, H, S, D, dtype, seed=22)
    prev_codes = mixed_codes(S_prev, H, seed=21, probs=(1, 1, 1, 1), evicted=0.1)
    cur_codes = mixed_codes(S, H, seed=22, probs=(1, 1, 1, 1), evicted=0.1)
    cur_codes[:S_prev][np.random.default_rng(5).random((S_prev, H)) < 0.5] = \
        prev_codes[np.random.default_rng(5).random((S_prev, H)) < 0.5]
    prev = _pack(kp, vp, prev_codes, dev)
    cur = _pack(kc, vc, cur_codes, dev)
    rprev = oracle_pack(kp, vp, prev_codes)
    rcur = oracle_pack(kc, vc, cur_codes)
    rng = np.random.default_rng(23)
    mask = {(t, h): bool(rng.random() < 0.5) for t in range(S) for h in range(H)}
    stats = cur.apply_reuse_mask(prev, mask, return_stats=True)
    assert stats == O.kv_apply_reuse_mask(rcur, rprev, mask)
    assert stats["applied"] > 0
    assert_cache_equal(cur, rcur)
    assert cur.apply_reuse_mask(prev, {(0, 0): True}) is None


def test_apply_reuse_mask_tensor_mask_and_full_reuse(dev):
    S, H, D = 32, 4, 128
    kp, vp = kv_inputs(1, H, S, D, torch.bfloat16, seed=31)
    kc, vc = kv_inputs(1, H, S, D, torch.bfloat16, seed=32)
    codes = mixed_codes(S, H, seed=31, probs=(1, 1, 1, 1))
    prev = _pack(kp, vp, codes, dev)
    cur = _pack(kc, vc, codes, dev)
    stats = cur.apply_reuse_mask(prev, torch.ones(S, H, dtype=torch.bool, device=dev),
                                 return_stats=True)
    assert stats == {"applied": S * H, "skipped_precision": 0}
    a = prev.unpack()
    b = cur.unpack()
    assert torch.equal(a[0], b[0]) and torch.equal(a[1], b[1])


def test_apply_reuse_mask_errors(dev):
    k, v = kv_inputs(1, 2, 4, 64, torch.float32, seed=41)
    k2, v2 = kv_inputs(1, 2, 4, 32, torch.float32, seed=42)
    c = np.full((4, 2), 3, np.int8)
    a = _pack(k, v, c, dev, group_size=16)
    b = _pack(k2, v2, c, dev)
    with pytest.raises(ValueError):
        a.apply_reuse_mask(b, {(0, 0): True})
    c32 = _pack(k, v, c, dev, group_size=32)
    with pytest.raises(ValueError):
        a.apply_reuse_mask(c32, {(0, 0): True})
    kb, vb = kv_inputs(2, 2, 4, 64, torch.float32, seed=43)
    with pytest.raises(ValueError):
        _pack(kb, vb, c, dev).apply_reuse_mask(a, {(0, 0): True})


# -------------------------------------------------------------- accounting
def test_memory_and_resident_bytes(dev):
    k, v = kv_inputs(1, 2, 8, 64, torch.float32, seed=51)
    codes = np.array([[(t * 2 + h) % 4 for h in range(2)] for t in range(8)], np.int8)
    cache = _pack(k, v, codes, dev)
    ref = oracle_pack(k, v, codes)
    assert cache.memory_bytes() == ref.memory_bytes()
    assert cache.resident_bytes() == ref.resident_bytes()
    assert cache.data_plane_bytes() == ref.memory_bytes()
    assert cache._precision_for(0, 0) == "fp32" and cache._precision_for(99, 0) == "evicted"
    # int4 bytes = ceil(B*D/2) per entry and tensor (reference test_shadowkv.py:479-502)
    d4 = cache.packed_data["int4"]
    assert d4["k"].numel() == len(d4["indices"]) * 32


def test_codes_map_roundtrip_on_device_plan(dev):
    codes = mixed_codes(16, 4, seed=61, probs=(1, 1, 1, 1), evicted=0.2)
    plan = PrecisionPlan.from_codes(torch.from_numpy(codes).to(dev))
    assert codes_to_map(plan.codes) == codes_to_map(torch.from_numpy(codes))


@pytest.mark.gpu
def test_evict_tensor_mask_matches_set(dev):
    """evict() with an [S, H] mask tensor equals evict() with the reference's
    set of (t, h) pairs, and both equal the oracle's compaction."""
    B, H, S, D = 2, 4, 70, 64
    k, v = kv_inputs(B, H, S, D, torch.bfloat16, seed=9)
    codes = mixed_codes(S, H, seed=9, probs=(1, 1, 1, 1), evicted=0.1)
    plan = PrecisionPlan.from_codes(torch.from_numpy(codes).to(dev))
    a = PackedKVCache.pack(k.to(dev), v.to(dev), None, plan=plan)["packed_kv"]
    b = PackedKVCache.pack(k.to(dev), v.to(dev), None, plan=plan)["packed_kv"]
    m = np.random.default_rng(9).random((S, H)) < 0.3
    pairs = {(int(t), int(h)) for t, h in zip(*np.nonzero(m))}
    ref = oracle_pack(k, v, codes)
    removed = O.kv_evict(ref, pairs)
    assert a.evict(pairs) == removed
    assert b.evict(torch.from_numpy(m).to(dev)) == removed
    assert_cache_equal(a, ref)
    assert_cache_equal(b, ref)
    assert b.evict(torch.zeros(S, H, dtype=torch.bool, device=dev)) == 0
    with pytest.raises(ValueError):
        b.evict(torch.zeros(S, H + 1, dtype=torch.bool, device=dev))


@pytest.mark.gpu
@pytest.mark.parametrize("dtype,shape", [(torch.bfloat16, (1, 8, 300, 128)),
                                         (torch.float32, (2, 3, 50, 45))])
def test_token_and_bucket_order_copies_agree(dev, dtype, shape):
    """si_kv_reuse / si_kv_compact (token order) and si_kv_reuse_flat /
    si_kv_compact_flat (bucket order, what PackedKVCache uses) write the same
    buckets and the same stats."""
    import ctypes
    from shadowinfer_amd import _native
    B, H, S, D = shape
    k, v = kv_inputs(B, H, S, D, dtype, seed=S)
    k2, v2 = kv_inputs(B, H, S, D, dtype, seed=S + 1)
    codes = mixed_codes(S, H, seed=S, probs=(1, 1, 1, 1), evicted=0.1)
    pcodes = codes.copy()
    pcodes[np.random.default_rng(S).random((S, H)) < 0.3] = 2
    plan = PrecisionPlan.from_codes(torch.from_numpy(codes).to(dev))
    pplan = PrecisionPlan.from_codes(torch.from_numpy(pcodes).to(dev))
    prev = PackedKVCache.pack(k2.to(dev), v2.to(dev), None, plan=pplan)["packed_kv"]
    a = PackedKVCache.pack(k.to(dev), v.to(dev), None, plan=plan)["packed_kv"]
    b = PackedKVCache.pack(k.to(dev), v.to(dev), None, plan=plan)["packed_kv"]
    mask = torch.from_numpy(np.random.default_rng(S + 2).random((S, H)) < 0.5).to(dev)
    st_a = a.apply_reuse_mask(prev, mask, return_stats=True)       # bucket order
    stats = torch.zeros(2, dtype=torch.int64, device=dev)
    code, slot, _, sdt, g = b.device_state()
    pcode, pslot, ptable, _, _ = prev.device_state()
    _native.call("si_kv_reuse", code.data_ptr(), slot.data_ptr(), b._bucket_table(), S,
                 pcode.data_ptr(), pslot.data_ptr(), ptable, S,
                 mask.reshape(-1).to(torch.uint8).data_ptr(), H, B, D, g, sdt, stats.data_ptr(),
                 _native.stream(dev))
    assert st_a == {"applied": int(stats[0]), "skipped_precision": int(stats[1])}
    for name, da in a.packed_data.items():
        for key in ("k", "v", "scale_k", "scale_v"):
            if da[key] is not None:
                assert torch.equal(da[key], b.packed_data[name][key]), (name, key)
    # compaction: the API (bucket order) against the token-order entry point
    ev = torch.from_numpy(np.random.default_rng(S + 3).random((S, H)) < 0.25).to(dev)
    old_code, old_slot, old_table, _, _ = b.device_state()
    keep = {n: {kk: (t.clone() if torch.is_tensor(t) else t) for kk, t in d.items()}
            for n, d in b._buckets.items()}
    from shadowinfer_amd.shadowkv.precision_plan import DeviceGrouping
    new = DeviceGrouping.scan(old_code, evict_mask=ev.reshape(-1).to(torch.uint8))
    fresh = b._alloc_buckets(new.counts, dev, b._scale_dtype)
    _native.call("si_kv_compact", old_code.data_ptr(), old_slot.data_ptr(), b._bucket_table(keep),
                 new.code.data_ptr(), new.slot.data_ptr(), b._bucket_table(fresh), S * H, B, D, g,
                 sdt, _native.stream(dev))
    a.evict(ev)
    for name, da in a._buckets.items():
        for key in ("k", "v", "scale_k", "scale_v"):
            if da.get(key) is not None:
                assert torch.equal(da[key], fresh[name][key]), (name, key)
