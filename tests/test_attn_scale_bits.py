"""Bit identities the packed-attention decode relies on (CPU only).

The decode multiplies int8/int4 codes by their scale in fp16 when every scale
of a tile lies in a range where that product rounds like the reference's fp32
product (h_exact in csrc/si_attn.hip). Inside that range a bf16 scale is
turned into fp16 by integer arithmetic on its bits: (bits << 3) - (112 << 10).
These tests check that identity against numpy's fp16 conversion on every bf16
pattern of the range, and that the range itself holds only positive normal
fp16 values with |q * s| <= 65504 for the code range.
"""

import numpy as np
import pytest

RANGES = {"int8": (0x3880, 0x43FF, 128), "int4": (0x3880, 0x45FF, 8)}


def _bf16_to_f32(bits):
    return (bits.astype(np.uint32) << 16).view(np.float32)


@pytest.mark.parametrize("kind", sorted(RANGES))
def test_bf16_scale_bits_to_fp16(kind):
    lo, hi, _ = RANGES[kind]
    bits = np.arange(lo, hi + 1, dtype=np.uint32)
    want = _bf16_to_f32(bits).astype(np.float16).view(np.uint16)
    got = (((bits << 3) - 0x1C000) & 0xFFFF).astype(np.uint16)
    np.testing.assert_array_equal(got, want)
    # a wrong rebias (127 -> 16 instead of 15) fails the same check
    bad = (((bits << 3) - 0x1BC00) & 0xFFFF).astype(np.uint16)
    assert (bad != want).all()


@pytest.mark.parametrize("kind", sorted(RANGES))
def test_scale_range_is_exact_in_fp16(kind):
    lo, hi, qmax = RANGES[kind]
    s = _bf16_to_f32(np.arange(lo, hi + 1, dtype=np.uint32)).astype(np.float64)
    assert s.min() == 2.0 ** -14                       # smallest normal fp16
    assert (s * qmax <= 65504.0).all()                 # products stay finite in fp16
    assert (s.astype(np.float16).astype(np.float64) == s).all()
    # the patterns just outside the range break one of the two conditions
    below = _bf16_to_f32(np.array([lo - 1], np.uint32)).astype(np.float64)[0]
    above = _bf16_to_f32(np.array([hi + 1], np.uint32)).astype(np.float64)[0]
    assert below < 2.0 ** -14 and above * qmax > 65504.0
