"""The fp32 -> bf16 rounding every kernel uses (gfx950's v_cvt_pk_bf16_f32,
NaN mapped to 0x7FC0) equals round-to-nearest-even bit arithmetic on all
2^32 fp32 bit patterns (si_check_bf16_convert runs the comparison on the
device). That bit arithmetic is the oracle's, which test_oracle.py pins to
torch's own bf16 cast."""

import pytest
import torch

from shadowinfer_amd import _native

pytestmark = pytest.mark.gpu


def test_bf16_conversion_all_fp32_patterns(dev):
    counts = torch.zeros(2, dtype=torch.int64, device=dev)
    _native.call("si_check_bf16_convert", counts.data_ptr(), _native.stream(dev))
    torch.cuda.synchronize(dev)
    assert counts.tolist() == [0, 0], "pair / single-value conversion mismatches"

