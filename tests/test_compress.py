"""Plan-driven compression fused with the pack (ShadowKVAgent._compress_kv_with_plan,
shadowinfer/shadowkv/shadowkv_agent.py:1698-1809).

CPU: the oracle's working copy is pinned against the reference's op chain run
in CPU torch (index_select per precision group, ``.half()``,
Quantizer.quantize_int8/int4 as torch ops, ``index_copy_`` of
``qk.to(dtype)``, reuse rows from the previous K/V).

GPU: ``compress_kv_with_plan`` (one ``si_kv_pack_copy`` pass) against the
oracle: the working copy bit for bit, and the buckets equal to a plain pack.
"""

import numpy as np
import pytest
import torch

from helpers import DT, assert_cache_equal, kv_inputs, mixed_codes, oracle_pack, to_np
from oracle import oracle as O


def _torch_quant_i8(x):
    """quantization.py:120-142 as torch ops in the input dtype."""
    scale = x.abs().amax(dim=-1, keepdim=True) / 127.0
    scale = torch.where(scale == 0, torch.ones_like(scale), scale)
    return torch.round(x / scale).clamp(-128, 127).to(torch.int8)


def _torch_quant_i4(x, g):
    """quantization.py:144-178."""
    shp = x.shape
    xg = x.reshape(*shp[:-1], shp[-1] // g, g)
    scale = xg.abs().amax(dim=-1, keepdim=True) / 7.0
    scale = torch.where(scale == 0, torch.ones_like(scale), scale)
    return torch.round(xg / scale).clamp(-8, 7).to(torch.int8).reshape(shp)


def _torch_working_copy(k, codes, group, prev=None, reuse=()):
    """shadowkv_agent.py:1727-1797 restated with torch ops on CPU tensors."""
    B, H, S, D = k.shape
    out = torch.zeros_like(k)
    kf = k.reshape(B, H * S, D)
    of = out.view(B, H * S, D)
    g = group if D % group == 0 else D
    for code in range(4):
        ent = [(t, h) for t in range(S) for h in range(H) if codes[t, h] == code]
        if not ent:
            continue
        flat = torch.tensor([h * S + t for t, h in ent], dtype=torch.long)
        grp = kf.index_select(1, flat).permute(1, 0, 2)
        if code == 0:
            q = grp
        elif code == 1:
            q = grp.half()
        elif code == 2:
            q = _torch_quant_i8(grp)
        else:
            q = _torch_quant_i4(grp, g)
        of.index_copy_(1, flat, q.permute(1, 0, 2).to(out.dtype).contiguous())
    if prev is not None and reuse:
        rflat = torch.tensor([h * S + t for t, h in reuse], dtype=torch.long)
        of.index_copy_(1, rflat, prev.reshape(B, H * S, D).index_select(1, rflat))
    return out


@pytest.mark.parametrize("dtype,shape", [(torch.bfloat16, (2, 3, 17, 48)),
                                         (torch.float32, (1, 4, 24, 64)),
                                         (torch.bfloat16, (1, 2, 9, 45))])
def test_oracle_working_copy_matches_reference_chain(dtype, shape):
    B, H, S, D = shape
    k, _ = kv_inputs(B, H, S, D, dtype, seed=S + D, outlier_frac=0.05)
    prev, _ = kv_inputs(B, H, S, D, dtype, seed=S + D + 1)
    codes = mixed_codes(S, H, seed=D, probs=(1, 1, 1, 1), sink=1, evicted=0.15)
    reuse = [(t, h) for t in range(S) for h in range(H) if (3 * t + h) % 5 == 0]
    want = _torch_working_copy(k, codes, 16, prev, reuse)
    got, _ = O.compress_working_copy(to_np(k), to_np(k), DT[dtype], codes, 16, to_np(prev),
                                     to_np(prev), reuse)
    np.testing.assert_array_equal(got, to_np(want))


# ------------------------------------------------------------------ HIP (GPU)
def _plan(codes, dev, reuse=()):
    from shadowinfer_amd.shadowkv import PrecisionPlan
    return PrecisionPlan.from_codes(torch.from_numpy(codes).to(dev),
                                    reuse_mask={e: True for e in reuse} or None)


@pytest.mark.gpu
@pytest.mark.parametrize("dtype,shape", [(torch.bfloat16, (1, 32, 8192, 128)),
                                         (torch.bfloat16, (2, 3, 17, 48)),
                                         (torch.float32, (1, 4, 24, 64)),
                                         (torch.float16, (2, 4, 33, 128)),
                                         (torch.bfloat16, (1, 2, 9, 45)),
                                         (torch.float32, (3, 2, 10, 20))])
@pytest.mark.parametrize("with_reuse", [False, True])
def test_hip_compress_matches_oracle(dev, dtype, shape, with_reuse):
    from shadowinfer_amd.shadowkv import PackedKVCache, compress_kv_with_plan
    B, H, S, D = shape
    k, v = kv_inputs(B, H, S, D, dtype, seed=B * S + D, outlier_frac=0.02)
    kp, vp = kv_inputs(B, H, S, D, dtype, seed=B * S + D + 7)
    codes = mixed_codes(S, H, seed=S, probs=(1, 2, 3, 3), sink=min(4, S), evicted=0.1)
    rng = np.random.default_rng(S)
    reuse = [(int(t), int(h)) for t, h in zip(*np.nonzero(rng.random((S, H)) < 0.3))] \
        if with_reuse else []
    plan = _plan(codes, dev, reuse)
    res = compress_kv_with_plan(k.to(dev), v.to(dev), kp.to(dev) if with_reuse else None,
                                vp.to(dev) if with_reuse else None, plan)
    wk, wv = O.compress_working_copy(to_np(k), to_np(v), DT[dtype], codes, 16,
                                     to_np(kp), to_np(vp), reuse)
    np.testing.assert_array_equal(to_np(res["k"]), wk)
    np.testing.assert_array_equal(to_np(res["v"]), wv)
    assert res["k"].dtype == dtype and res["k"].shape == k.shape
    # the buckets are those of a plain pack
    assert_cache_equal(res["packed_kv"], oracle_pack(k, v, codes))
    plain = PackedKVCache.pack(k.to(dev), v.to(dev), None, plan=plan)["packed_kv"]
    assert res["memory_bytes"] == plain.memory_bytes()


@pytest.mark.gpu
def test_hip_compress_scale_maps_and_errors(dev):
    from shadowinfer_amd.shadowkv import compress_kv_with_plan
    B, H, S, D = 2, 3, 12, 32
    k, v = kv_inputs(B, H, S, D, torch.bfloat16, seed=5)
    codes = mixed_codes(S, H, seed=5, probs=(1, 1, 1, 1), sink=0)
    reuse = [(0, 0), (3, 2), (7, 1)]
    plan = _plan(codes, dev, reuse)
    kd, vd = k.to(dev), v.to(dev)
    res = compress_kv_with_plan(kd, vd, kd, vd, plan, build_scale_map=True)
    data = res["packed_kv"].packed_data
    smk = res["scale_k_map"]
    assert set(smk) == {(t, h) for t in range(S) for h in range(H)} - set(reuse)
    for name, d in data.items():
        for i, entry in enumerate(d["indices"]):
            if entry in reuse:
                continue
            if name in ("fp32", "fp16"):
                assert smk[entry] is None
            elif name == "int8":
                assert torch.equal(smk[entry], d["scale_k"][i:i + 1])
            else:
                G = d["scale_k"].shape[1]
                assert torch.equal(smk[entry], d["scale_k"].view(-1, B, G, 1)[i:i + 1])
    with pytest.raises(ValueError):
        compress_kv_with_plan(kd[:, :2], vd[:, :2], None, None, plan)
    with pytest.raises(ValueError):
        compress_kv_with_plan(kd, vd, kd, None, plan)
    with pytest.raises(ValueError):
        compress_kv_with_plan(kd, vd, kd[:, :, :6], vd[:, :, :6], plan)
