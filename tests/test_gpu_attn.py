"""GPU tests of the fused dequantize + bidirectional attention over a packed KV
cache. Reference: unpack() -> softmax(q k^T / sqrt(D)) v with no mask, in
double precision (the oracle at small sizes, a float64 torch computation on
the device at the full sizes). Tolerance: relative L2 <= 1e-3.
"""

import math

import numpy as np
import pytest
import torch

from helpers import kv_inputs, mixed_codes, oracle_pack
from oracle import oracle as O
from shadowinfer_amd import _native
from shadowinfer_amd.shadowkv import PackedKVCache, PrecisionPlan, packed_attention

pytestmark = pytest.mark.gpu

TOL = 1e-3


def _rel_l2(a, b):
    a = torch.as_tensor(a).double()
    b = torch.as_tensor(b).double()
    return (torch.linalg.vector_norm(a - b) / torch.linalg.vector_norm(b)).item()


def _pack(k, v, codes, dev, group_size=16):
    plan = PrecisionPlan.from_codes(torch.from_numpy(codes).to(dev))
    return PackedKVCache.pack(k.to(dev), v.to(dev), None, group_size=group_size,
                              plan=plan)["packed_kv"]


@pytest.mark.parametrize("qdtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("B,H,Sq,Skv,D", [(1, 2, 128, 64, 128), (2, 2, 100, 200, 128),
                                          (1, 3, 130, 257, 64), (1, 1, 1, 1, 64)])
def test_attention_small_vs_oracle(dev, qdtype, B, H, Sq, Skv, D):
    k, v = kv_inputs(B, H, Skv, D, torch.bfloat16, seed=Skv + D, outlier_frac=0.02)
    codes = mixed_codes(Skv, H, seed=Skv, probs=(1, 1, 2, 1), sink=min(4, Skv), evicted=0.05)
    cache = _pack(k, v, codes, dev)
    g = torch.Generator().manual_seed(Sq)
    q = torch.randn(B, H, Sq, D, generator=g).to(qdtype)
    out = packed_attention(q.to(dev), cache)
    assert out.dtype == torch.float32 and out.shape == (B, H, Sq, D)
    rk, rv = O.kv_unpack(oracle_pack(k, v, codes))
    ref = O.attention(q.float().numpy().reshape(B * H, Sq, D), rk.reshape(B * H, Skv, D),
                      rv.reshape(B * H, Skv, D)).reshape(B, H, Sq, D)
    assert _rel_l2(out.float().cpu(), ref) <= TOL


@pytest.mark.parametrize("D,qdtype,g", [(64, torch.float16, 8), (64, torch.bfloat16, 16),
                                        (128, torch.float16, 16), (128, torch.bfloat16, 8)])
def test_attention_fp32_inputs_outlier_channels(dev, D, qdtype, g):
    """fp32 K/V with 5% outlier channels (x8) and queries at 1.5 sigma, every
    precision present: peaked scores, where K rounded to fp16 is most of the
    error (8.1-8.6e-4 on these cases; up to 1.25e-3 in a random sweep of such
    inputs). Caches of fp32 inputs carry K as fp16 hi + lo, which leaves Q's
    and P's fp16 rounding (4.2-4.7e-4 here), so they are held to 6e-4."""
    B, H, Sq, Skv = 2, 2, 600, 1400
    k, v = kv_inputs(B, H, Skv, D, torch.float32, seed=D + g, outlier_frac=0.05)
    codes = mixed_codes(Skv, H, seed=D * g, probs=(1, 1, 1, 1), sink=4, evicted=0.1)
    cache = _pack(k, v, codes, dev, group_size=g)
    q = (torch.randn(B, H, Sq, D, generator=torch.Generator().manual_seed(D - g)) * 1.5).to(qdtype)
    out = packed_attention(q.to(dev), cache)
    rk, rv = O.kv_unpack(oracle_pack(k, v, codes, group_size=g))
    ref = O.attention(q.float().numpy().reshape(B * H, Sq, D), rk.reshape(B * H, Skv, D),
                      rv.reshape(B * H, Skv, D)).reshape(B, H, Sq, D)
    assert _rel_l2(out.float().cpu(), ref) <= 6e-4


def _dense_reference(q, k, v):
    """float64 softmax(q k^T / sqrt(D)) v on the device, one head at a time."""
    B, H, Sq, D = q.shape
    out = torch.empty(B, H, Sq, D, dtype=torch.float64, device=q.device)
    for b in range(B):
        for h in range(H):
            qh = q[b, h].double()
            kt = k[b, h].double().t().contiguous()
            s = (qh @ kt) / math.sqrt(D)
            p = torch.softmax(s, dim=-1)
            out[b, h] = p @ v[b, h].double()
    return out


@pytest.mark.parametrize("S", [2048, 8192])
def test_attention_config4(dev, S):
    """B=1, 32 heads, head_dim 128, K/V bf16 with 1% outlier channels packed
    with the 25/50/25 fp16/int8/int4 mixture and a 4-token sink; Q bf16."""
    H, D = 32, 128
    k, v = kv_inputs(1, H, S, D, torch.bfloat16, seed=S, outlier_frac=0.01)
    codes = mixed_codes(S, H, seed=S, probs=(0, 0.25, 0.5, 0.25), sink=4)
    cache = _pack(k, v, codes, dev)
    g = torch.Generator().manual_seed(S + 1)
    q = torch.randn(1, H, S, D, generator=g).to(torch.bfloat16).to(dev)
    out = packed_attention(q, cache)
    ku, vu = cache.unpack()
    ref = _dense_reference(q, ku, vu)
    err = (torch.linalg.vector_norm(out.double() - ref) / torch.linalg.vector_norm(ref)).item()
    assert err <= TOL, err


def test_attention_evicted_entries_take_part(dev):
    """Evicted token-heads act as zero keys/values (score 0), as after unpack()."""
    H, S, D = 2, 64, 64
    k, v = kv_inputs(1, H, S, D, torch.bfloat16, seed=77)
    codes = np.full((S, H), 2, np.int8)
    codes[S // 2:] = 4
    cache = _pack(k, v, codes, dev)
    q = torch.randn(1, H, 16, D).to(torch.bfloat16)
    out = packed_attention(q.to(dev), cache)
    rk, rv = O.kv_unpack(oracle_pack(k, v, codes))
    ref = O.attention(q.float().numpy().reshape(H, 16, D), rk.reshape(H, S, D), rv.reshape(H, S, D))
    assert _rel_l2(out.float().cpu().reshape(H, 16, D), ref) <= TOL


def test_attention_low_precision_output(dev):
    """bf16/fp16 outputs are the fp32 result rounded once (bf16 rounding alone
    is ~1e-3 relative, so they are checked against the rounded fp32 output)."""
    k, v = kv_inputs(1, 2, 96, 128, torch.bfloat16, seed=5)
    cache = _pack(k, v, mixed_codes(96, 2, seed=5, probs=(1, 1, 1, 1)), dev)
    q = torch.randn(1, 2, 64, 128).to(torch.bfloat16).to(dev)
    ref = packed_attention(q, cache)
    for dt in (torch.bfloat16, torch.float16):
        out = packed_attention(q, cache, out_dtype=dt)
        assert out.dtype == dt
        assert torch.equal(out, ref.to(dt))


def test_attention_errors(dev):
    k, v = kv_inputs(1, 2, 16, 64, torch.bfloat16, seed=1)
    cache = _pack(k, v, np.full((16, 2), 1, np.int8), dev)
    with pytest.raises(ValueError):
        packed_attention(torch.randn(1, 3, 8, 64, device=dev, dtype=torch.bfloat16), cache)
    with pytest.raises(TypeError):
        packed_attention(torch.randn(1, 2, 8, 64, device=dev), cache)


@pytest.mark.gpu
@pytest.mark.parametrize("D", [64, 128])
def test_attention_entry_points_agree(dev, D):
    """si_attn_packed_fwd / _tokens (slot lists built on every call) and
    si_attn_packed_fwd_built (lists built once per plan) give the same bits,
    and a cache repacked with the same plan reuses the plan's lists."""
    from shadowinfer_amd import _native
    B, H, S = 2, 3, 200
    k, v = kv_inputs(B, H, S, D, torch.bfloat16, seed=D)
    q, _ = kv_inputs(B, H, S, D, torch.bfloat16, seed=D + 1)
    codes = mixed_codes(S, H, seed=D, probs=(1, 1, 1, 1), evicted=0.1)
    plan = PrecisionPlan.from_codes(torch.from_numpy(codes).to(dev))
    cache = PackedKVCache.pack(k.to(dev), v.to(dev), None, plan=plan)["packed_kv"]
    qd = q.to(dev)
    code, slot, table, sdt, group = cache.device_state()
    ws_bytes = _native.size_query("si_attn_workspace_bytes", H, S)
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device=dev)
    for entry, tm in (("si_attn_packed_fwd", False), ("si_attn_packed_fwd_tokens", True)):
        shape = (B, S, H, D) if tm else (B, H, S, D)
        out = torch.empty(shape, dtype=torch.float32, device=dev)
        _native.call(entry, qd.data_ptr(), _native.dtype_code(qd.dtype), B, H, S, D,
                     code.data_ptr(), slot.data_ptr(), table, sdt, S, group,
                     float(1 / D ** 0.5), out.data_ptr(), _native.dtype_code(torch.float32),
                     ws.data_ptr(), ws_bytes, _native.stream(dev))
        got = packed_attention(qd, cache, token_major=tm)
        assert torch.equal(got, out)
    again = PackedKVCache.pack((k * 2).to(dev), v.to(dev), None, plan=plan)["packed_kv"]
    assert again.attention_lists() is cache.attention_lists()


@pytest.mark.gpu
@pytest.mark.parametrize("D", [64, 128])
def test_attention_offset_widths_agree(dev, D):
    """Caches below 2^31 bytes address bucket rows with 32-bit offsets; larger
    ones with 64-bit addresses. si_tune_attn_offset64 selects the 64-bit path at
    any size: both give the same bits, and both match the oracle."""
    B, H, S = 2, 3, 300
    k, v = kv_inputs(B, H, S, D, torch.bfloat16, seed=D + 7, outlier_frac=0.02)
    codes = mixed_codes(S, H, seed=D + 7, probs=(1, 1, 2, 1), sink=4, evicted=0.05)
    cache = _pack(k, v, codes, dev)
    g = torch.Generator().manual_seed(D)
    q = torch.randn(B, H, S, D, generator=g).to(torch.bfloat16).to(dev)
    narrow = packed_attention(q, cache)
    lib = _native.load()
    lib.si_tune_attn_offset64(1)
    try:
        wide = packed_attention(q, cache)
    finally:
        lib.si_tune_attn_offset64(0)
    assert torch.equal(narrow, wide)
    rk, rv = O.kv_unpack(oracle_pack(k, v, codes))
    ref = O.attention(q.float().cpu().numpy().reshape(B * H, S, D), rk.reshape(B * H, S, D),
                      rv.reshape(B * H, S, D)).reshape(B, H, S, D)
    assert _rel_l2(wide.float().cpu(), ref) <= TOL


@pytest.mark.gpu
def test_attention_extreme_scales(dev):
    """Rows whose int8/int4 scales leave the range where a packed fp16 multiply
    rounds like the fp32 product (scales below 2^-14, or q * s near the fp16
    limit) take the decode's fp32 route; the result still matches the oracle."""
    B, H, S, D = 1, 2, 256, 128
    k, v = kv_inputs(B, H, S, D, torch.bfloat16, seed=5)
    k, v = k.float(), v.float()
    k[:, :, 10:20] *= 1e-4                      # int8 scale ~3e-6, int4 ~5e-5: below 2^-14
    v[:, :, 10:20] *= 1e-4
    big = v[:, :, 30:40]
    v[:, :, 30:40] = big / big.abs().amax(dim=-1, keepdim=True) * 65000.0  # s*128 > 65504
    k, v = k.to(torch.bfloat16), v.to(torch.bfloat16)
    codes = mixed_codes(S, H, seed=5, probs=(1, 1, 2, 1), sink=4)
    codes[10:20, 0] = 2
    codes[10:20, 1] = 3
    codes[30:40, 0] = 2
    codes[30:40, 1] = 3
    cache = _pack(k, v, codes, dev)
    g = torch.Generator().manual_seed(3)
    q = torch.randn(B, H, S, D, generator=g).to(torch.bfloat16)
    out = packed_attention(q.to(dev), cache)
    rk, rv = O.kv_unpack(oracle_pack(k, v, codes))
    assert np.isfinite(rv).all()
    ref = O.attention(q.float().numpy().reshape(B * H, S, D), rk.reshape(B * H, S, D),
                      rv.reshape(B * H, S, D)).reshape(B, H, S, D)
    assert _rel_l2(out.float().cpu(), ref) <= TOL
