"""Seeded random sweep of the packed KV path against the oracle: pack (bucket
order, through PackedKVCache), apply_reuse_mask from a previous cache of
another length and code mixture, evict, unpack. Shapes cover B > 1, odd head
dims (generic row paths), fp32 / fp16 / bf16 inputs, empty buckets and evicted
entries; every step must match the oracle bit for bit
(packed_kv_cache.py:43-878)."""

import numpy as np
import pytest
import torch

from helpers import DT, assert_cache_equal, kv_inputs, oracle_pack, to_np
from oracle import oracle as O
from shadowinfer_amd.shadowkv import PackedKVCache, PrecisionPlan

DTYPES = (torch.float32, torch.float16, torch.bfloat16)
HEAD_DIMS = (16, 32, 45, 64, 96, 128)


def _case(seed):
    rng = np.random.default_rng(seed)
    B = int(rng.integers(1, 4))
    H = int(rng.integers(1, 9))
    S = int(rng.integers(1, 160))
    D = int(rng.choice(HEAD_DIMS))
    dtype = DTYPES[int(rng.integers(0, 3))]
    probs = rng.random(5) * (rng.random(5) < 0.8)  # some precisions absent
    probs[1] += 1e-3
    codes = rng.choice(5, size=(S, H), p=probs / probs.sum()).astype(np.int8)
    S_prev = int(rng.integers(1, S + 20))
    pcodes = rng.choice(5, size=(S_prev, H), p=probs / probs.sum()).astype(np.int8)
    same = rng.random((min(S, S_prev), H)) < 0.6  # mostly the same precision as now
    pcodes[:min(S, S_prev)][same] = codes[:min(S_prev, S)][same]
    return rng, B, H, S, D, dtype, codes, S_prev, pcodes


@pytest.mark.gpu
@pytest.mark.parametrize("seed", range(24))
def test_random_pack_reuse_evict_unpack(dev, seed):
    rng, B, H, S, D, dtype, codes, S_prev, pcodes = _case(seed)
    k, v = kv_inputs(B, H, S, D, dtype, seed=seed, outlier_frac=0.05)
    kp, vp = kv_inputs(B, H, S_prev, D, dtype, seed=seed + 1000)
    plan = PrecisionPlan.from_codes(torch.from_numpy(codes).to(dev))
    pplan = PrecisionPlan.from_codes(torch.from_numpy(pcodes).to(dev))
    cache = PackedKVCache.pack(k.to(dev), v.to(dev), None, plan=plan)["packed_kv"]
    prev = PackedKVCache.pack(kp.to(dev), vp.to(dev), None, plan=pplan)["packed_kv"]
    ref = oracle_pack(k, v, codes)
    pref = oracle_pack(kp, vp, pcodes)
    assert_cache_equal(cache, ref)
    assert_cache_equal(prev, pref)
    # reuse: the reference's dict mask, including flags outside the current range
    flags = rng.random((S + 3, H)) < 0.5
    mask = {(int(t), int(h)): True for t, h in zip(*np.nonzero(flags))}
    st = cache.apply_reuse_mask(prev, mask, return_stats=True)
    want = O.kv_apply_reuse_mask(ref, pref, mask)
    assert st == want, (st, want)
    assert_cache_equal(cache, ref)
    # evict a random subset (the reference's set of pairs)
    victims = {(int(t), int(h)) for t, h in zip(*np.nonzero(rng.random((S, H)) < 0.3))}
    assert cache.evict(victims) == O.kv_evict(ref, victims)
    assert_cache_equal(cache, ref)
    assert cache.memory_bytes() == ref.memory_bytes()
    ku, vu = cache.unpack()
    rk, rv = O.kv_unpack(ref)
    np.testing.assert_array_equal(ku.cpu().numpy(), rk)
    np.testing.assert_array_equal(vu.cpu().numpy(), rv)
    assert ku.dtype == torch.float32 and tuple(ku.shape) == (B, H, S, D)


@pytest.mark.gpu
@pytest.mark.parametrize("seed", range(12))
def test_random_packed_attention(dev, seed):
    """Fused dequant + attention against the oracle's double-precision attention
    over the unpacked K/V (relL2 <= 1e-3), both output layouts."""
    from shadowinfer_amd.shadowkv import packed_attention
    rng, B, H, S, _, dtype, codes, _, _ = _case(seed + 500)
    D = int(rng.choice((64, 128)))
    Sq = int(rng.integers(1, 300))
    k, v = kv_inputs(B, H, S, D, dtype, seed=seed, outlier_frac=0.05)
    q, _ = kv_inputs(B, H, Sq, D, torch.bfloat16, seed=seed + 7)
    plan = PrecisionPlan.from_codes(torch.from_numpy(codes).to(dev))
    cache = PackedKVCache.pack(k.to(dev), v.to(dev), None, plan=plan)["packed_kv"]
    out = packed_attention(q.to(dev), cache)
    tok = packed_attention(q.to(dev), cache, token_major=True)
    assert torch.equal(tok, out.transpose(1, 2))
    rk, rv = O.kv_unpack(oracle_pack(k, v, codes))
    want = O.attention(O.to_f32(to_np(q), DT[torch.bfloat16]), rk, rv).astype(np.float64)
    got = out.cpu().double().numpy()
    rel = np.linalg.norm(got - want) / max(np.linalg.norm(want), 1e-30)
    assert rel <= 1e-3, rel
