"""Committed golden fixtures (tests/golden/, written by tests/golden/make_golden.py
from CPU torch running the reference's op chain) against the oracle (CPU) and
the HIP path (GPU): packed buckets, scales, unpack, evict, apply_reuse_mask,
plan fingerprints and INT8Linear, bit for bit."""

import hashlib
import json
import os
import sys

import numpy as np
import pytest
import torch

from helpers import bits, to_np
from oracle import oracle as O

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
sys.path.insert(0, GOLDEN)
import make_golden as G  # noqa: E402  (input generators of the fixtures)

KV_CASES = [("kv_f32_b1h4s24d64.npz", torch.float32, (1, 4, 24, 64)),
            ("kv_bf16_b2h3s17d48.npz", torch.bfloat16, (2, 3, 17, 48)),
            ("kv_bf16_b1h2s9d45.npz", torch.bfloat16, (1, 2, 9, 45))]
NAMES = ("fp32", "fp16", "int8", "int4")
REUSE_CASE = "reuse_bf16_b2h4s24p16d32.npz"


def _load(name):
    return np.load(os.path.join(GOLDEN, name), allow_pickle=False)


def _tensor(arr, dtype):
    if dtype == torch.float32:
        return torch.from_numpy(np.ascontiguousarray(arr))
    return torch.from_numpy(arr.view(np.int16).copy()).view(dtype)


def _sha(a):
    return hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()


def _config1():
    with open(os.path.join(GOLDEN, "config1_digests.json")) as f:
        ref = json.load(f)
    B, H, S, D = ref["shape"]
    s = ref["seeds"]
    k = G.gen_f32((B, H, S, D), s["k"])
    v = G.gen_f32((B, H, S, D), s["v"])
    codes = G.gen_codes(S, H, s["codes"], choices=(1, 2, 3), sink=4)
    assert _sha(codes) == ref["codes_sha256"]
    imp = G.gen_uniform(S * H, s["importance"])
    drop = {(int(e // H), int(e % H)) for e in np.argsort(imp, kind="stable")[: (S * H) // 4]}
    reuse = G.gen_uniform(S * H, s["reuse"]) < 0.5
    return ref, k, v, codes, drop, reuse


def _reuse_inputs():
    """The reuse fixture: the reference's dict mask over every current token-head
    (False ones included) and the previous cache's post-pack evictions."""
    z = _load(REUSE_CASE)
    S, H = z["codes"].shape
    mask = {(t, h): bool(z["mask"][t, h]) for t in range(S) for h in range(H)}
    drop = {(int(t), int(h)) for t, h in z["drop"].tolist()}
    stats = {"applied": int(z["applied"]), "skipped_precision": int(z["skipped_precision"])}
    return z, mask, drop, stats


def _check_buckets(z, view, as_bytes):
    for p in NAMES:
        if f"{p}.k" not in z.files:
            assert p not in view
            continue
        d = view[p]
        assert [tuple(e) for e in z[f"{p}.indices"].tolist()] == list(d["indices"])
        for key in ("k", "v", "scale_k", "scale_v"):
            if f"{p}.{key}" in z.files:
                np.testing.assert_array_equal(as_bytes(d[key]), z[f"{p}.{key}"].reshape(-1).view(np.uint8),
                                              err_msg=f"{p}.{key}")


# ------------------------------------------------------------------ oracle (CPU)
@pytest.mark.parametrize("name,dtype,shape", KV_CASES)
def test_oracle_matches_golden_kv(name, dtype, shape):
    z = _load(name)
    dt = {torch.float32: O.F32, torch.bfloat16: O.BF16}[dtype]
    cache = O.kv_pack(z["k"], z["v"], dt, z["codes"], 16)
    for p in NAMES:
        if f"{p}.k" not in z.files:
            assert p not in cache.packed_data
            continue
        d = cache.packed_data[p]
        assert [tuple(e) for e in z[f"{p}.indices"].tolist()] == d["indices"]
        for key in ("k", "v", "scale_k", "scale_v"):
            if f"{p}.{key}" in z.files:
                np.testing.assert_array_equal(np.ascontiguousarray(d[key]).reshape(-1).view(np.uint8),
                                              z[f"{p}.{key}"].reshape(-1).view(np.uint8), err_msg=f"{p}.{key}")
    uk, uv = O.kv_unpack(cache)
    np.testing.assert_array_equal(uk.view(np.uint32), z["unpack_k"].view(np.uint32))
    np.testing.assert_array_equal(uv.view(np.uint32), z["unpack_v"].view(np.uint32))


def test_oracle_matches_golden_config1():
    ref, k, v, codes, drop, reuse = _config1()
    cache = O.kv_pack(k, v, O.F32, codes, ref["group"])
    got = {f"{p}.{key}": _sha(d[key]) for p, d in cache.packed_data.items()
           for key in ("k", "v", "scale_k", "scale_v") if d[key] is not None}
    assert got == ref["buckets"]
    assert {p: len(d["indices"]) for p, d in cache.packed_data.items()} == ref["counts"]
    assert cache.memory_bytes() == ref["memory_bytes"]
    uk, uv = O.kv_unpack(cache)
    assert (_sha(uk), _sha(uv)) == (ref["unpack_k"], ref["unpack_v"])
    assert O.kv_evict(cache, drop) == ref["evict_removed"]
    got = {f"{p}.{key}": _sha(d[key]) for p, d in cache.packed_data.items()
           for key in ("k", "v", "scale_k", "scale_v") if d[key] is not None}
    assert got == ref["evict_buckets"]
    uk, uv = O.kv_unpack(cache)
    assert (_sha(uk), _sha(uv)) == (ref["evict_unpack_k"], ref["evict_unpack_v"])
    S, H = codes.shape
    assert O.plan_from_codes(codes)["fingerprint"] == ref["fingerprint_no_reuse"]
    mask = {(e // H, e % H): True for e in np.nonzero(reuse)[0]}
    assert O.plan_from_codes(codes, mask)["fingerprint"] == ref["fingerprint_reuse"]


def test_oracle_matches_golden_reuse():
    """apply_reuse_mask from a shorter previous cache with evicted and
    cross-precision entries: copied rows, untouched rows and both counters."""
    z, mask, drop, stats = _reuse_inputs()
    cur = O.kv_pack(z["k"], z["v"], O.BF16, z["codes"], 16)
    prev = O.kv_pack(z["k_prev"], z["v_prev"], O.BF16, z["codes_prev"], 16)
    assert O.kv_evict(prev, drop) == len(drop)
    assert O.kv_apply_reuse_mask(cur, prev, mask) == stats
    _check_buckets(z, cur.packed_data, lambda a: np.ascontiguousarray(a).reshape(-1).view(np.uint8))
    uk, uv = O.kv_unpack(cur)
    np.testing.assert_array_equal(uk.view(np.uint32), z["unpack_k"].view(np.uint32))
    np.testing.assert_array_equal(uv.view(np.uint32), z["unpack_v"].view(np.uint32))


def test_golden_reuse_covers_every_branch():
    """The fixture exercises every outcome of the reference's loop
    (packed_kv_cache.py:797-808): same-bucket copies in all four buckets,
    cross-bucket skips, and masked entries the previous cache does not hold
    (code 4, evicted after packing, or beyond its seq_len), which count in
    neither counter."""
    z, mask, drop, stats = _reuse_inputs()
    codes, prev = z["codes"], z["codes_prev"]
    seen = {}
    for (t, h), on in mask.items():
        if not on or codes[t, h] == 4:
            continue
        if t >= prev.shape[0]:
            kind = "beyond"
        elif prev[t, h] == 4:
            kind = "prev_code4"
        elif (t, h) in drop:
            kind = "prev_evicted"
        elif prev[t, h] == codes[t, h]:
            kind = "same_" + NAMES[codes[t, h]]
        else:
            kind = "cross"
        seen[kind] = seen.get(kind, 0) + 1
    for kind in ("same_fp32", "same_fp16", "same_int8", "same_int4", "cross", "prev_code4",
                 "prev_evicted", "beyond"):
        assert seen.get(kind, 0) >= 1, kind
    assert stats["applied"] == sum(v for k, v in seen.items() if k.startswith("same_"))
    assert stats["skipped_precision"] == seen["cross"]


def test_oracle_matches_golden_int8_linear():
    z = _load("int8_linear_m8k128n96.npz")
    qT, sw = O.int8_weight_quant(z["w"])
    np.testing.assert_array_equal(qT, z["qweight_kn"])
    np.testing.assert_array_equal(sw.view(np.uint32), z["weight_scale"].view(np.uint32))
    out, acc, q, s = O.int8_linear_forward(z["x"], O.BF16, qT, sw)
    np.testing.assert_array_equal(q, z["act_q"])
    np.testing.assert_array_equal(s.view(np.uint32), z["act_scale"].view(np.uint32))
    np.testing.assert_array_equal(acc, z["acc"])
    np.testing.assert_array_equal(out, z["out"])
    outb, _, _, _ = O.int8_linear_forward(z["x"], O.BF16, qT, sw, z["bias"])
    np.testing.assert_array_equal(outb, z["out_bias"])


# ------------------------------------------------------------------ HIP path (GPU)
def _device_pack(k, v, codes, dev):
    from shadowinfer_amd.shadowkv import PackedKVCache, PrecisionPlan
    plan = PrecisionPlan.from_codes(torch.from_numpy(codes).to(dev))
    return PackedKVCache.pack(k.to(dev), v.to(dev), None, group_size=16, plan=plan)["packed_kv"]


@pytest.mark.gpu
@pytest.mark.parametrize("name,dtype,shape", KV_CASES)
def test_hip_matches_golden_kv(dev, name, dtype, shape):
    z = _load(name)
    cache = _device_pack(_tensor(z["k"], dtype), _tensor(z["v"], dtype), z["codes"], dev)
    view = cache.packed_data
    for p in NAMES:
        if f"{p}.k" not in z.files:
            assert p not in view
            continue
        d = view[p]
        assert [tuple(e) for e in z[f"{p}.indices"].tolist()] == d["indices"]
        for key in ("k", "v", "scale_k", "scale_v"):
            if f"{p}.{key}" in z.files:
                np.testing.assert_array_equal(bits(d[key]), z[f"{p}.{key}"].reshape(-1).view(np.uint8),
                                              err_msg=f"{p}.{key}")
    uk, uv = cache.unpack()
    np.testing.assert_array_equal(to_np(uk).view(np.uint32), z["unpack_k"].view(np.uint32))
    np.testing.assert_array_equal(to_np(uv).view(np.uint32), z["unpack_v"].view(np.uint32))


@pytest.mark.gpu
def test_hip_matches_golden_config1(dev):
    from shadowinfer_amd.shadowkv import PrecisionPlan
    ref, k, v, codes, drop, reuse = _config1()
    cache = _device_pack(torch.from_numpy(k), torch.from_numpy(v), codes, dev)

    def digests():
        return {f"{p}.{key}": _sha(to_np(d[key])) for p, d in cache.packed_data.items()
                for key in ("k", "v", "scale_k", "scale_v") if d[key] is not None}

    assert digests() == ref["buckets"]
    assert cache.memory_bytes() == ref["memory_bytes"]
    uk, uv = cache.unpack()
    assert (_sha(to_np(uk)), _sha(to_np(uv))) == (ref["unpack_k"], ref["unpack_v"])
    assert cache.evict(drop) == ref["evict_removed"]
    assert digests() == ref["evict_buckets"]
    uk, uv = cache.unpack()
    assert (_sha(to_np(uk)), _sha(to_np(uv))) == (ref["evict_unpack_k"], ref["evict_unpack_v"])
    S, H = codes.shape
    dcodes = torch.from_numpy(codes).to(dev)
    assert PrecisionPlan.from_codes(dcodes).fingerprint == ref["fingerprint_no_reuse"]
    mask = {(int(e // H), int(e % H)): True for e in np.nonzero(reuse)[0]}
    assert PrecisionPlan.from_codes(dcodes, reuse_mask=mask).fingerprint == ref["fingerprint_reuse"]


@pytest.mark.gpu
def test_hip_matches_golden_reuse(dev):
    z, mask, drop, stats = _reuse_inputs()
    cur = _device_pack(_tensor(z["k"], torch.bfloat16), _tensor(z["v"], torch.bfloat16), z["codes"], dev)
    prev = _device_pack(_tensor(z["k_prev"], torch.bfloat16), _tensor(z["v_prev"], torch.bfloat16),
                        z["codes_prev"], dev)
    assert prev.evict(drop) == len(drop)
    assert cur.apply_reuse_mask(prev, mask, return_stats=True) == stats
    _check_buckets(z, cur.packed_data, bits)
    uk, uv = cur.unpack()
    np.testing.assert_array_equal(to_np(uk).view(np.uint32), z["unpack_k"].view(np.uint32))
    np.testing.assert_array_equal(to_np(uv).view(np.uint32), z["unpack_v"].view(np.uint32))


@pytest.mark.gpu
def test_hip_matches_golden_int8_linear(dev):
    from shadowinfer_amd.ffn_optimizer import INT8Linear
    z = _load("int8_linear_m8k128n96.npz")
    N, K = z["w"].shape
    for with_bias in (False, True):
        lin = torch.nn.Linear(K, N, bias=with_bias)
        with torch.no_grad():
            lin.weight.copy_(torch.from_numpy(z["w"]))
            if with_bias:
                lin.bias.copy_(torch.from_numpy(z["bias"]))
        layer = INT8Linear.from_linear(lin.to(dev))
        np.testing.assert_array_equal(layer.qweight.cpu().numpy(), z["qweight_kn"])
        np.testing.assert_array_equal(layer.weight_scale.cpu().numpy().view(np.uint32),
                                      z["weight_scale"].view(np.uint32))
        out = layer(_tensor(z["x"], torch.bfloat16).to(dev))
        np.testing.assert_array_equal(to_np(out), z["out_bias" if with_bias else "out"])
