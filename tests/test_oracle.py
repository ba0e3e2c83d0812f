"""Pins of the oracle (CPU only).

Each function of oracle/ is checked against something other than its own
formula: the reference tests' known answers, library routines (torch's dtype
conversions and CPU op chain, numpy's float16, int64 matmul, float64
softmax), closed forms, brute force on tiny inputs, and invariants - chosen so
that a dropped term, a wrong sign/index or a transposed operand fails.
"""

import hashlib
import struct

import numpy as np
import pytest
import torch

from helpers import to_np
from oracle import oracle as O

RNG = np.random.default_rng(20261201)


def _bits_sample(n):
    """Random fp32 bit patterns plus specials (zeros, subnormals, inf, NaN, ties)."""
    u = RNG.integers(0, 2**32, size=n, dtype=np.uint64).astype(np.uint32)
    special = np.array([0, 0x80000000, 1, 0x807fffff, 0x7f7fffff, 0x7f800000, 0xff800000,
                        0x7fc00000, 0x3f808000, 0x3f818000, 0x3f800001, 0x477fe000, 0x477ff000,
                        0x477fefff, 0x38800000, 0x387fffff, 0x33800000, 0x33000000], np.uint32)
    return np.concatenate([u, special]).view(np.float32)


# ----------------------------------------------------------------- dtypes
def test_bf16_rounding_matches_torch():
    x = _bits_sample(2_000_000)
    ours = O.from_f32(x, O.BF16)
    ref = torch.from_numpy(x).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    finite = np.isfinite(x)
    np.testing.assert_array_equal(ours[finite], ref[finite])
    assert np.all((ours[np.isnan(x)] & 0x7fff) > 0x7f80)


def test_f16_rounding_matches_numpy():
    x = _bits_sample(2_000_000)
    ours = O.from_f32(x, O.F16)
    with np.errstate(over="ignore"):
        ref = x.astype(np.float16).view(np.uint16)
    ok = ~np.isnan(x)
    np.testing.assert_array_equal(ours[ok], ref[ok])


def test_widening_is_exact_for_every_pattern():
    h = np.arange(65536, dtype=np.uint16)
    f16 = O.to_f32(h, O.F16)
    ref16 = h.view(np.float16).astype(np.float32)
    ok = ~np.isnan(ref16)
    np.testing.assert_array_equal(f16[ok].view(np.uint32), ref16[ok].view(np.uint32))
    bf = O.to_f32(h, O.BF16)
    refbf = torch.from_numpy(h.view(np.int16)).view(torch.bfloat16).float().numpy()
    ok = ~np.isnan(refbf)
    np.testing.assert_array_equal(bf[ok].view(np.uint32), refbf[ok].view(np.uint32))


# ------------------------------------------------------------ quantizers
def _torch_int8(t):
    """The reference's op chain (utils/quantization.py:138-141) on CPU torch."""
    scale = t.abs().max(dim=-1, keepdim=True)[0] / 127.0
    scale = torch.where(scale == 0, torch.ones_like(scale), scale)
    return torch.round(t / scale).clamp(-128, 127).to(torch.int8), scale


def _torch_int4(t, g):
    r = t.reshape(*t.shape[:-1], t.shape[-1] // g, g)
    scale = r.abs().max(dim=-1, keepdim=True)[0] / 7.0
    scale = torch.where(scale == 0, torch.ones_like(scale), scale)
    return torch.round(r / scale).clamp(-8, 7).to(torch.int8), scale


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
def test_quant_rows_match_torch_op_chain(dtype):
    g = torch.Generator().manual_seed(5)
    x = (torch.randn(257, 64, generator=g) * torch.rand(257, 1, generator=g) * 10).to(dtype)
    x[3] = 0
    dt = {torch.float32: O.F32, torch.bfloat16: O.BF16, torch.float16: O.F16}[dtype]
    q, s = O.quant_rows_i8(to_np(x), dt)
    tq, ts = _torch_int8(x)
    np.testing.assert_array_equal(q, tq.numpy())
    np.testing.assert_array_equal(s, to_np(ts))
    q4, s4 = O.quant_rows_i4(to_np(x), dt, 16)
    tq4, ts4 = _torch_int4(x, 16)
    np.testing.assert_array_equal(q4, tq4.numpy())
    np.testing.assert_array_equal(s4, to_np(ts4))


def test_quant_known_answers():
    # reference test_kernels.py:72-77: scale of [1,-2,3,-4] is 4/127
    q, s = O.quant_rows_i8(np.array([[1.0, -2.0, 3.0, -4.0]], np.float32), O.F32)
    assert s[0, 0] == np.float32(4.0) / np.float32(127.0)
    assert q.tolist() == [[32, -64, 95, -127]]
    q, s = O.quant_rows_i8(np.zeros((2, 8), np.float32), O.F32)  # zero row -> scale 1
    assert np.all(s == 1) and np.all(q == 0)
    # +-amax -> +-127 (int8), +-7 (int4)
    q, _ = O.quant_rows_i8(np.array([[-5.0, 5.0, 0.0, 1.0]], np.float32), O.F32)
    assert q[0, 0] == -127 and q[0, 1] == 127
    q4, s4 = O.quant_rows_i4(np.array([[-3.5, 3.5] + [0.0] * 14], np.float32), O.F32, 16)
    assert q4[0, 0, 0] == -7 and q4[0, 0, 1] == 7 and s4[0, 0, 0] == np.float32(0.5)
    # half-even ties: x/s = 0.5 -> 0, 1.5 -> 2, 2.5 -> 2, -2.5 -> -2 (s = 1 for amax 127)
    q, s = O.quant_rows_i8(np.array([[127.0, 0.5, 1.5, 2.5, -2.5, -0.5]], np.float32), O.F32)
    assert s[0, 0] == 1.0 and q.tolist() == [[127, 0, 2, 2, -2, 0]]


def test_int8_clamp_is_asymmetric_on_bf16():
    """bf16 rounding of the scale can push |x/s| to 127.5: +127.5 rounds to 128
    and clamps to 127, -127.5 rounds to -128 and stays (clamp(-128, 127))."""
    found = None
    for h in range(0x3f80, 0x4000):  # bf16 amax in [1, 2)
        a = np.array([h], np.uint16)
        af = O.to_f32(a, O.BF16)[0]
        s = O.to_f32(O.from_f32(np.array([af / np.float32(127.0)], np.float32), O.BF16), O.BF16)[0]
        qq = O.to_f32(O.from_f32(np.array([af / s], np.float32), O.BF16), O.BF16)[0]
        if qq == 127.5:
            found = h
            break
    assert found is not None
    row = np.zeros((2, 8), np.uint16)
    row[0, 0] = found
    row[1, 0] = found | 0x8000
    q, _ = O.quant_rows_i8(row, O.BF16)
    assert q[0, 0] == 127 and q[1, 0] == -128
    tq, _ = _torch_int8(torch.from_numpy(row.view(np.int16)).view(torch.bfloat16))
    np.testing.assert_array_equal(q, tq.numpy())


def test_quant_error_bound_invariant():
    x = RNG.standard_normal((500, 64)).astype(np.float32)
    q, s = O.quant_rows_i8(x, O.F32)
    err = np.abs(x - q.astype(np.float32) * s)
    assert np.all(err <= s * 0.5 * (1 + 1e-5))
    q4, s4 = O.quant_rows_i4(x, O.F32, 16)
    err4 = np.abs(x.reshape(500, 4, 16) - q4.astype(np.float32) * s4)
    assert np.all(err4 <= s4 * 0.5 * (1 + 1e-5))


# ------------------------------------------------------------- int4 bytes
def test_int4_all_nibble_pairs_and_padding():
    hi, lo = np.meshgrid(np.arange(-8, 8), np.arange(-8, 8), indexing="ij")
    codes = np.stack([hi.ravel(), lo.ravel()], 1).reshape(1, -1).astype(np.int8)
    packed = O.pack_int4_rows(codes)[0]
    np.testing.assert_array_equal(packed, ((hi.ravel() + 8) << 4 | (lo.ravel() + 8)).astype(np.uint8))
    odd = np.array([[-8, 7, 3]], np.int8)  # odd length: zero low nibble pad
    assert O.pack_int4_rows(odd).tolist() == [[0x0F, 0xB0]]
    for L in (1, 2, 7, 23, 128):
        c = RNG.integers(-8, 8, size=(3, L)).astype(np.int8)
        np.testing.assert_array_equal(O.unpack_int4_rows(O.pack_int4_rows(c), L), c)
        t = torch.from_numpy(c[0].copy())  # reference Quantizer.pack_int4 op chain
        off = (t + 8).to(torch.uint8)
        if off.numel() % 2:
            off = torch.cat([off, torch.zeros(1, dtype=torch.uint8)])
        np.testing.assert_array_equal(O.pack_int4_flat(c[0]), ((off[0::2] << 4) | (off[1::2] & 15)).numpy())


# ------------------------------------------------------------------- plan
def test_plan_map_codes_known_answers():
    """reference tests/test_dense_precision.py:181-216 (UT-10.1)."""
    pm = {0: {0: "fp32", 2: "evicted"}, 1: {1: "int8"}, 2: {0: "int4", 1: "fp16", 2: "fp32"},
          4: {2: "evicted"}}
    codes = O.map_to_codes(pm, 5, 3)
    assert codes[0, 1] == 1 and codes[3, 0] == 1 and codes[0, 2] == 4 and codes[4, 2] == 4
    assert codes[0, 0] == 0 and codes[1, 1] == 2 and codes[2, 0] == 3
    with pytest.raises(ValueError):
        O.map_to_codes({0: {0: "bf16"}}, 1, 1, strict=True)
    assert O.map_to_codes({0: {0: "bf16"}}, 1, 1, strict=False)[0, 0] == 1


def test_plan_grouping_and_fingerprint():
    """UT-8.1 (reference tests/test_kv_plan.py:87-157): token-major groups,
    flat = h*S + t, fingerprint stable and sensitive to codes and reuse."""
    S, H = 5, 3
    names = ("fp32", "fp16", "int8", "int4")
    pm = {t: {h: names[(t + h) % 4] for h in range(H)} for t in range(S)}
    codes = O.map_to_codes(pm, S, H)
    mask = {(0, 0): True, (1, 2): True, (2, 0): True, (3, 1): False, (4, 1): True}
    plan = O.plan_from_codes(codes, mask)
    for p in names:
        exp = [(t, h) for t in range(S) for h in range(H) if pm[t][h] == p]
        assert plan["groups"][p] == exp
        assert plan["flat_indices"][p].tolist() == [h * S + t for t, h in exp]
    assert plan["reuse_entries"] == [(0, 0), (1, 2), (2, 0), (4, 1)]
    assert len(plan["fingerprint"]) == 64
    assert O.plan_from_codes(codes, mask)["fingerprint"] == plan["fingerprint"]
    c2 = codes.copy()
    c2[0, 0] = 2
    assert O.plan_from_codes(c2, mask)["fingerprint"] != plan["fingerprint"]
    m2 = dict(mask)
    m2[(3, 1)] = True
    assert O.plan_from_codes(codes, m2)["fingerprint"] != plan["fingerprint"]
    assert O.plan_from_codes(codes, None)["reuse_flat"].size == 0
    # digest covers exactly (S, H) then the codes then the reuse flats
    d = hashlib.sha256(struct.pack("<QQ", S, H) + codes.tobytes()
                       + np.array([0, 2 * S + 1, 2, 1 * S + 4], "<i8").tobytes())
    assert d.hexdigest() == plan["fingerprint"]


# --------------------------------------------------------------- kv cache
def _per_entry_pack(k, v, dt, codes, g):
    """The reference's per-entry golden pack (packed_kv_cache.py:390-533): one
    Quantizer call and one flat int4 pack per (t, h), concatenated."""
    B, H, S, D = k.shape
    geff = g if D % g == 0 else D
    out = {}
    for p, name in enumerate(("fp32", "fp16", "int8", "int4")):
        ent = [(t, h) for t in range(S) for h in range(H) if codes[t, h] == p]
        if not ent:
            continue
        if name in ("fp32", "fp16"):
            dst = O.F32 if name == "fp32" else O.F16
            out[name] = {"k": np.stack([O.convert(k[:, h, t, :], dt, dst) for t, h in ent]),
                         "indices": ent}
        elif name == "int8":
            qs = [O.quant_rows_i8(np.ascontiguousarray(k[:, h, t, :]), dt) for t, h in ent]
            out[name] = {"k": np.stack([q for q, _ in qs]), "scale_k": np.stack([s for _, s in qs]),
                         "indices": ent}
        else:
            parts, scales = [], []
            for t, h in ent:
                q, s = O.quant_rows_i4(np.ascontiguousarray(k[:, h, t, :]), dt, geff)
                parts.append(O.pack_int4_flat(q.reshape(-1)))
                scales.append(s)
            out[name] = {"k": np.concatenate(parts), "scale_k": np.concatenate(scales),
                         "indices": ent}
    return out


@pytest.mark.parametrize("B,H,S,D,g", [(1, 3, 5, 16, 16), (1, 2, 5, 7, 16), (1, 2, 7, 24, 16),
                                       (2, 2, 9, 32, 16), (1, 4, 16, 128, 16), (2, 1, 4, 5, 16)])
@pytest.mark.parametrize("dt", [O.F32, O.BF16])
def test_vectorized_pack_equals_per_entry_pack(B, H, S, D, g, dt):
    """The reference's golden-pack test shapes (tests/test_pipeline_overhead.py:
    94-130, odd head_dim row padding included)."""
    x = RNG.standard_normal((2, B, H, S, D)).astype(np.float32)
    k, v = (O.from_f32(x[0], dt), O.from_f32(x[1], dt))
    codes = RNG.integers(0, 5, size=(S, H)).astype(np.int8)
    cache = O.kv_pack(k, v, dt, codes, g)
    ref = _per_entry_pack(k, v, dt, codes, g)
    assert set(cache.packed_data) == set(ref)
    for name, r in ref.items():
        d = cache.packed_data[name]
        assert d["indices"] == r["indices"]
        np.testing.assert_array_equal(d["k"].reshape(-1).view(np.uint8), r["k"].reshape(-1).view(np.uint8))
        if "scale_k" in r:
            np.testing.assert_array_equal(d["scale_k"].reshape(-1), r["scale_k"].reshape(-1))
    # byte accounting closed form (packed_kv_cache.py:856-863)
    ssz = 4 if dt == O.F32 else 2
    G = D // (g if D % g == 0 else D)
    per = {0: 2 * 4 * B * D, 1: 2 * 2 * B * D, 2: 2 * (B * D + B * ssz),
           3: 2 * ((B * D + 1) // 2 + B * G * ssz)}
    assert cache.memory_bytes() == sum(per[c] for c in codes.ravel() if c < 4)


def test_unpack_roundtrip_properties():
    B, H, S, D = 2, 3, 40, 32
    x = RNG.standard_normal((2, B, H, S, D)).astype(np.float32)
    k, v = O.from_f32(x[0], O.BF16), O.from_f32(x[1], O.BF16)
    codes = RNG.integers(0, 5, size=(S, H)).astype(np.int8)
    cache = O.kv_pack(k, v, O.BF16, codes, 16)
    ku, vu = O.kv_unpack(cache)
    kf = O.to_f32(k, O.BF16)
    for t in range(S):
        for h in range(H):
            c = codes[t, h]
            got, want = ku[:, h, t, :], kf[:, h, t, :]
            if c == 4:
                assert np.all(got == 0)
            elif c in (0, 1):  # bf16 -> fp32 / fp16 are exact for N(0,1) values here
                np.testing.assert_array_equal(got, O.to_f32(O.from_f32(want, O.F16), O.F16) if c == 1 else want)
            elif c == 2:
                # |x - q s| <= s/2 plus the bf16 rounding of x/s (<= 127 * 2^-9 steps)
                amax = np.abs(want).max(axis=-1, keepdims=True)
                assert np.all(np.abs(got - want) <= amax / 127 * (0.5 + 127 / 512 + 0.01))
            else:
                w = want.reshape(B, D // 16, 16)
                amax = np.abs(w).max(axis=-1, keepdims=True)
                err = np.abs(got.reshape(B, D // 16, 16) - w)
                assert np.all(err <= amax / 7 * (0.5 + 7 / 512 + 0.01))


def test_evict_and_reuse_invariants():
    B, H, S, D = 1, 2, 16, 32
    x = RNG.standard_normal((4, B, H, S, D)).astype(np.float32)
    codes = (np.arange(S * H).reshape(S, H) // 3 % 4).astype(np.int8)
    cache = O.kv_pack(x[0], x[1], O.F32, codes, 16)
    before_bytes = cache.memory_bytes()
    ku0, _ = O.kv_unpack(cache)
    victims = {(t, h) for t in range(0, S, 3) for h in range(H)}
    removed = O.kv_evict(cache, victims)
    assert removed == len(victims)
    per = {0: 2 * 4 * D, 1: 2 * 2 * D, 2: 2 * (D + 4), 3: 2 * (D // 2 + 2 * 4)}
    assert before_bytes - cache.memory_bytes() == sum(per[codes[t, h]] for t, h in victims)
    ku1, _ = O.kv_unpack(cache)
    for t in range(S):
        for h in range(H):
            if (t, h) in victims:
                assert np.all(ku1[:, h, t] == 0)
            else:
                np.testing.assert_array_equal(ku1[:, h, t], ku0[:, h, t])
    assert O.kv_evict(cache, victims) == 0
    for d in cache.packed_data.values():  # order stays token-major
        assert d["indices"] == sorted(d["indices"])
    # reuse: same-precision entries copied, cross-precision counted
    prev = O.kv_pack(x[2], x[3], O.F32, codes, 16)
    cur_codes = codes.copy()
    cur_codes[1, 0] = (codes[1, 0] + 1) % 4
    cur = O.kv_pack(x[0], x[1], O.F32, cur_codes, 16)
    mask = {(t, h): True for t in range(S) for h in range(H)}
    stats = O.kv_apply_reuse_mask(cur, prev, mask)
    assert stats == {"applied": S * H - 1, "skipped_precision": 1}
    kc, _ = O.kv_unpack(cur)
    kp, _ = O.kv_unpack(prev)
    same = cur_codes == codes
    for t in range(S):
        for h in range(H):
            if same[t, h]:
                np.testing.assert_array_equal(kc[:, h, t], kp[:, h, t])


# -------------------------------------------------------------- INT8 FFN
def test_int8_linear_matches_torch_and_int64():
    g = torch.Generator().manual_seed(3)
    w = torch.randn(48, 64, generator=g) * 0.02
    w[5] = 0
    qT, sw = O.int8_weight_quant(w.numpy())
    # reference from_linear op chain (int8_linear.py:70-74)
    ts = (w.abs().amax(dim=1) / 127.0).clamp_min(1e-8)
    tq = torch.round(w / ts.unsqueeze(1)).clamp(-127, 127).to(torch.int8)
    np.testing.assert_array_equal(qT, tq.t().numpy())
    np.testing.assert_array_equal(sw, ts.numpy())
    assert sw[5] == np.float32(1e-8)
    x = (torch.randn(10, 64, generator=g) * 3).to(torch.bfloat16)
    x[2] = 0
    out, acc, q, s = O.int8_linear_forward(to_np(x), O.BF16, qT, sw, None)
    xf = x.float()
    tsx = (xf.abs().amax(dim=1) / 127.0).clamp_min(1e-8)
    tqx = torch.round(xf / tsx.unsqueeze(1)).clamp(-127, 127).to(torch.int8)
    np.testing.assert_array_equal(q, tqx.numpy())
    np.testing.assert_array_equal(s, tsx.numpy())
    assert q.min() >= -127  # clamp is symmetric for INT8Linear
    np.testing.assert_array_equal(acc, (q.astype(np.int64) @ qT.astype(np.int64)).astype(np.int32))
    np.testing.assert_array_equal(acc, torch._int_mm(tqx, tq.t().contiguous()).numpy())
    ref = (torch.from_numpy(acc).float() * (tsx.unsqueeze(1) * ts.unsqueeze(0))).to(torch.bfloat16)
    np.testing.assert_array_equal(out, to_np(ref))
    bias = np.linspace(-1, 1, 48).astype(np.float32)
    outb = O.int8_epilogue(acc, s, sw, bias, O.F32)
    refb = torch.from_numpy(acc).float() * (tsx.unsqueeze(1) * ts.unsqueeze(0)) + torch.from_numpy(bias)
    np.testing.assert_array_equal(outb, refb.numpy())


def test_gemm_brute_force_tiny():
    a = RNG.integers(-128, 128, size=(3, 5)).astype(np.int8)
    b = RNG.integers(-128, 128, size=(5, 4)).astype(np.int8)
    c = O.gemm_i8(a, b)
    for m in range(3):
        for n in range(4):
            assert c[m, n] == sum(int(a[m, k]) * int(b[k, n]) for k in range(5))


# -------------------------------------------------------------- attention
def test_attention_matches_float64_softmax():
    q = RNG.standard_normal((2, 7, 16)).astype(np.float32)
    k = RNG.standard_normal((2, 11, 16)).astype(np.float32)
    v = RNG.standard_normal((2, 11, 16)).astype(np.float32)
    out = O.attention(q, k, v)
    s = np.einsum("bid,bjd->bij", q.astype(np.float64), k.astype(np.float64)) / 4.0
    p = np.exp(s - s.max(-1, keepdims=True))
    p /= p.sum(-1, keepdims=True)
    np.testing.assert_allclose(out, np.einsum("bij,bjd->bid", p, v.astype(np.float64)), rtol=1e-6, atol=1e-6)
    # equal keys -> uniform weights -> mean of the values
    ke = np.repeat(k[:, :1], 11, axis=1)
    np.testing.assert_allclose(O.attention(q, ke, v), np.broadcast_to(v.mean(1, keepdims=True), q.shape[:2] + (16,)),
                               rtol=1e-5, atol=1e-6)
