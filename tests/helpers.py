"""Shared helpers for the parity tests: seeded inputs and tensor <-> oracle
array conversion (bf16/fp16 as uint16 bit patterns)."""

from __future__ import annotations

import numpy as np
import torch

from oracle import oracle as O

DT = {torch.float32: O.F32, torch.float16: O.F16, torch.bfloat16: O.BF16}


def to_np(t: torch.Tensor) -> np.ndarray:
    """CPU numpy view of a tensor; fp16/bf16 become uint16 bit patterns."""
    t = t.detach().to("cpu").contiguous()
    if t.dtype in (torch.float16, torch.bfloat16):
        return t.view(torch.int16).numpy().view(np.uint16)
    return t.numpy()


def bits(t: torch.Tensor) -> np.ndarray:
    """Raw bytes of a tensor as uint8 (for bit-exact comparisons)."""
    t = t.detach().to("cpu").contiguous()
    return t.reshape(-1).view(torch.uint8).numpy()


def kv_inputs(B, H, S, D, dtype, seed, outlier_frac=0.0):
    g = torch.Generator().manual_seed(seed)
    k = torch.randn(B, H, S, D, generator=g)
    v = torch.randn(B, H, S, D, generator=g)
    if outlier_frac > 0:
        nout = max(1, int(round(D * outlier_frac)))
        ch = torch.randperm(D, generator=g)[:nout]
        k[..., ch] *= 8
        v[..., ch] *= 8
    return k.to(dtype), v.to(dtype)


def mixed_codes(S, H, seed, probs=(0.0, 1 / 3, 1 / 3, 1 / 3), sink=4, evicted=0.0):
    """int8 [S, H] codes drawn from ``probs`` over (fp32, fp16, int8, int4), the
    first ``sink`` tokens forced to fp16, a fraction ``evicted`` set to 4."""
    rng = np.random.default_rng(seed)
    codes = rng.choice(4, size=(S, H), p=np.array(probs) / np.sum(probs)).astype(np.int8)
    if evicted > 0:
        codes[rng.random((S, H)) < evicted] = 4
    codes[:sink, :] = 1
    return codes


def oracle_pack(k: torch.Tensor, v: torch.Tensor, codes: np.ndarray, group_size=16):
    return O.kv_pack(to_np(k), to_np(v), DT[k.dtype], codes, group_size)


def assert_cache_equal(cache, ref):
    """Bucket tensors of a device PackedKVCache equal the oracle's arrays bit for bit."""
    view = cache.packed_data
    assert set(view) == set(ref.packed_data), (set(view), set(ref.packed_data))
    for name, rdata in ref.packed_data.items():
        data = view[name]
        assert data["indices"] == rdata["indices"], name
        for key in ("k", "v", "scale_k", "scale_v"):
            if rdata[key] is None:
                assert data[key] is None, (name, key)
                continue
            t = data[key]
            assert tuple(t.shape) == tuple(rdata[key].shape), (name, key, t.shape, rdata[key].shape)
            np.testing.assert_array_equal(bits(t), np.ascontiguousarray(rdata[key]).reshape(-1).view(np.uint8),
                                          err_msg=f"{name}.{key}")
        if name == "int4":
            assert data["byte_offsets"] == rdata["byte_offsets"]
            assert data["group_size"] == rdata["group_size"]
            assert data["num_groups"] == rdata["num_groups"]
    assert cache.memory_bytes() == ref.memory_bytes()
