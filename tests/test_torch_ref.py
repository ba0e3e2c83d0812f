"""CPU: the torch restatement of the reference's op chain that bench.py times
as its CPU baseline (oracle/torch_ref.py) computes what the oracle computes:
bucket bytes, scales, index lists and unpacked values bit for bit, and the
INT8Linear forward bit for bit (int32 product exact, same epilogue)."""

import numpy as np
import pytest
import torch

from helpers import DT, kv_inputs, mixed_codes, to_np
from oracle import oracle as O
from oracle import torch_ref as TR


@pytest.mark.parametrize("dtype,B,H,S,D", [(torch.bfloat16, 1, 4, 40, 64),
                                           (torch.float32, 2, 3, 17, 48),
                                           (torch.bfloat16, 1, 2, 9, 45)])
def test_torch_pack_unpack_equals_oracle(dtype, B, H, S, D):
    k, v = kv_inputs(B, H, S, D, dtype, seed=S + D, outlier_frac=0.05)
    codes = mixed_codes(S, H, seed=D, probs=(1, 1, 1, 1), evicted=0.1)
    groups, flat = TR.plan_from_codes(torch.from_numpy(codes))
    packed = TR.pack_with_plan(k, v, groups, flat, 16)
    ref = O.kv_pack(to_np(k), to_np(v), DT[dtype], codes, 16)
    assert set(packed) == set(ref.packed_data)
    for name, d in ref.packed_data.items():
        got = packed[name]
        assert got["indices"] == d["indices"], name
        for key in ("k", "v", "scale_k", "scale_v"):
            if d[key] is None:
                assert got.get(key) is None
                continue
            np.testing.assert_array_equal(to_np(got[key]).reshape(-1).view(np.uint8),
                                          np.ascontiguousarray(d[key]).reshape(-1).view(np.uint8))
        if name == "int4":
            assert got["byte_offsets"] == d["byte_offsets"]
    ko, vo = TR.unpack(packed, B, H, S, D)
    rk, rv = O.kv_unpack(ref)
    np.testing.assert_array_equal(ko.numpy(), rk)
    np.testing.assert_array_equal(vo.numpy(), rv)


@pytest.mark.parametrize("M,K,N", [(1, 128, 96), (16, 256, 200), (33, 512, 64)])
def test_torch_int8_linear_equals_oracle(M, K, N):
    g = torch.Generator().manual_seed(M + K)
    w = torch.randn(N, K, generator=g) * 0.02
    qw, sw = TR.int8_weight(w)
    rq, rs = O.int8_weight_quant(w.numpy())
    np.testing.assert_array_equal(qw.numpy(), rq)
    np.testing.assert_array_equal(sw.numpy(), rs)
    x = torch.randn(M, K, generator=g).to(torch.bfloat16)
    bias = torch.randn(N, generator=g)
    y = TR.int8_linear_forward(x, qw, sw, bias)
    ry, _, _, _ = O.int8_linear_forward(to_np(x), O.BF16, rq, rs, bias.numpy())
    np.testing.assert_array_equal(to_np(y), ry)
