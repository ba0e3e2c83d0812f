"""Seeded random PagedKVStore sessions on the GPU: appends of random lengths
and precisions (pages of 1 to 32 tokens, a precision change sealing the open
page), then an eviction of random (token, head) pairs, against the oracle's
pack -> evict -> unpack of the same tokens, as the reference pins its store
(tests/test_paged_kv_execution.py). gather() concatenates pages that tile
[0, end) without a gap (paged_kv_store.py:326-376), so fully evicted trailing
tokens shorten it while any other gap keeps the stored length with zeros."""

import numpy as np
import pytest
import torch

from helpers import DT, to_np
from oracle import oracle as O

pytestmark = pytest.mark.gpu

_CODE = {"fp32": 0, "fp16": 1, "int8": 2, "int4": 3}


@pytest.mark.parametrize("seed", range(30))
def test_random_session_vs_oracle(dev, seed):
    from shadowinfer_amd.shadowkv import PagedKVStore
    rng = np.random.default_rng(3000 + seed)
    B, H = int(rng.integers(1, 3)), int(rng.integers(1, 6))
    D = int(rng.choice([16, 24, 32, 45, 64, 128]))
    page = int(rng.choice([1, 4, 8, 16, 32]))
    dtype = [torch.float32, torch.bfloat16][int(rng.integers(0, 2))]
    store = PagedKVStore(B, H, D, page_size=page, device=dev, int4_group_size=16)
    ks, vs, codes = [], [], []
    for step in range(int(rng.integers(1, 8))):
        n = int(rng.integers(0, 40))
        prec = ["fp32", "fp16", "int8", "int4"][int(rng.integers(0, 4))]
        g = torch.Generator().manual_seed(seed * 100 + step)
        k = (torch.randn(B, H, n, D, generator=g) * 2).to(dtype)
        v = (torch.randn(B, H, n, D, generator=g) * 2).to(dtype)
        store.append(k.to(dev), v.to(dev), prec)
        ks.append(k)
        vs.append(v)
        codes += [_CODE[prec]] * n
    k, v = torch.cat(ks, 2), torch.cat(vs, 2)
    S = k.shape[2]
    code_map = np.repeat(np.array(codes, np.int8)[:, None], H, 1).reshape(S, H)
    cache = O.kv_pack(to_np(k), to_np(v), DT[dtype], code_map, 16)
    gk, gv = store.gather()
    uk, uv = O.kv_unpack(cache)
    np.testing.assert_array_equal(to_np(gk), uk)
    np.testing.assert_array_equal(to_np(gv), uv)
    if S == 0:
        return
    pairs = {(int(rng.integers(0, S)), int(rng.integers(0, H)))
             for _ in range(int(rng.integers(0, S * H // 2 + 1)))}
    assert store.evict_tokens(pairs) == O.kv_evict(cache, pairs)
    gk, gv = store.gather()
    uk, uv = O.kv_unpack(cache)
    gone = np.array([all((t, h) in pairs for h in range(H)) for t in range(S)])
    kept = np.nonzero(~gone)[0]
    end = 0 if len(kept) == 0 else int(kept[-1]) + 1
    if not gone[:end].any():  # the pages tile [0, end): gather() stops there
        uk, uv = uk[:, :, :end], uv[:, :, :end]
    np.testing.assert_array_equal(to_np(gk), uk)
    np.testing.assert_array_equal(to_np(gv), uv)
