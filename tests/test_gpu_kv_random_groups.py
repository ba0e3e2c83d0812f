"""Seeded random layers through the PackedKVCache cycle with the knobs the
sweep in test_gpu_kv_random.py keeps fixed: int4 group sizes that do and do not
divide the head dim (8, 16, 32, D / 3, D), head dims from 2 to 256, up to 600
tokens and 12 heads, sink tokens. Pack (packed_kv_cache.py:43-365), unpack
(:535-656), apply_reuse_mask from a shorter previous cache with its own codes
(:753-854) and evict of a set that includes out-of-range and absent pairs
(:666-751), each against the oracle bit for bit (buckets, scales, indices,
byte counts, the reuse stats and the removed count)."""

import numpy as np
import pytest
import torch

from helpers import assert_cache_equal, kv_inputs, mixed_codes, oracle_pack
from oracle import oracle as O
from shadowinfer_amd.shadowkv import PackedKVCache, PrecisionPlan

pytestmark = pytest.mark.gpu

_DTYPES = [torch.float32, torch.bfloat16, torch.float16]
_DIMS = [2, 5, 7, 16, 24, 32, 45, 48, 64, 96, 100, 128, 256]


def _pack(k, v, codes, dev, g):
    plan = PrecisionPlan.from_codes(torch.from_numpy(codes).to(dev))
    return PackedKVCache.pack(k.to(dev), v.to(dev), None, group_size=g, plan=plan)["packed_kv"]


def _unpack_equal(cache, ref):
    k_out, v_out = cache.unpack()
    rk, rv = O.kv_unpack(ref)
    np.testing.assert_array_equal(k_out.cpu().numpy(), rk)
    np.testing.assert_array_equal(v_out.cpu().numpy(), rv)


@pytest.mark.parametrize("seed", range(40))
def test_random_layer_cycle(dev, seed):
    rng = np.random.default_rng(9000 + seed)
    B, H, S = int(rng.integers(1, 4)), int(rng.integers(1, 13)), int(rng.integers(1, 601))
    D = int(rng.choice(_DIMS))
    dtype = _DTYPES[int(rng.integers(0, 3))]
    g = int(rng.choice([16, 8, 32, max(2, D // 3), max(2, D)]))
    probs = tuple(float(x) for x in rng.random(4) + 0.05)
    sink, evicted = int(rng.integers(0, 5)), float(rng.random() * 0.3)

    k, v = kv_inputs(B, H, S, D, dtype, seed=seed)
    codes = mixed_codes(S, H, seed=seed + 1, probs=probs, sink=sink, evicted=evicted)
    cache = _pack(k, v, codes, dev, g)
    ref = oracle_pack(k, v, codes, group_size=g)
    assert_cache_equal(cache, ref)
    _unpack_equal(cache, ref)

    s_prev = int(rng.integers(1, S + 1))
    kp, vp = kv_inputs(B, H, s_prev, D, dtype, seed=seed + 7)
    cp = mixed_codes(s_prev, H, seed=seed + 9, probs=probs, sink=sink, evicted=evicted)
    prev = _pack(kp, vp, cp, dev, g)
    ref_prev = oracle_pack(kp, vp, cp, group_size=g)
    mask = {(t, h): bool(rng.random() < 0.6) for t in range(S) for h in range(H)
            if rng.random() < 0.7}
    stats = cache.apply_reuse_mask(prev, mask, return_stats=True)
    assert stats == O.kv_apply_reuse_mask(ref, ref_prev, mask)
    assert_cache_equal(cache, ref)

    pairs = {(int(rng.integers(0, S + 3)), int(rng.integers(0, H + 1)))
             for _ in range(int(rng.integers(0, S * H // 2 + 2)))}
    assert cache.evict(pairs) == O.kv_evict(ref, pairs)
    assert_cache_equal(cache, ref)
    _unpack_equal(cache, ref)
