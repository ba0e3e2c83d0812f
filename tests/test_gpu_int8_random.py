"""Seeded random shapes through every INT8 GEMM path the tile choice can take
(weight streaming at several column widths, split K, 64x64 / 64x128 / 128x128 / 256x128 /
256x192 / 256x256 tiles, the register-staged tile for K not a multiple of 64,
the scalar kernel for K not a multiple of 16, the row-streaming kernel):
int32 results against the exact float64 product, and the INT8Linear epilogue
(int8_linear.py:102-115) against the oracle bit for bit."""

import numpy as np
import pytest
import torch

from oracle import oracle as O
from shadowinfer_amd import _native


def _shape(seed):
    rng = np.random.default_rng(seed)
    M = int(rng.choice([int(rng.integers(1, 33)), int(rng.integers(33, 700)),
                        int(rng.integers(700, 2500))]))
    N = int(rng.integers(1, 6000))
    K = int(rng.choice([64 * int(rng.integers(1, 96)), 128 * int(rng.integers(1, 48)),
                        16 * int(rng.integers(1, 200)), int(rng.integers(1, 300))]))
    return rng, M, N, K


def _gemm(a, b_nk, entry, sx=None, sw=None, bias=None, out_dtype=torch.bfloat16):
    M, K = a.shape
    N = b_nk.shape[0]
    ws_b = _native.size_query("si_gemm_workspace_bytes", M, N, K)
    ws = torch.empty(max(ws_b, 1), dtype=torch.uint8, device=a.device)
    st = _native.stream(a.device)
    if entry == "i32":
        c = torch.empty(M, N, dtype=torch.int32, device=a.device)
        _native.call("si_gemm_i8i8_i32", a.data_ptr(), b_nk.data_ptr(), M, N, K, c.data_ptr(),
                     ws.data_ptr(), ws_b, st)
        return c
    out = torch.empty(M, N, dtype=out_dtype, device=a.device)
    _native.call("si_gemm_i8_dequant", a.data_ptr(), sx.data_ptr(), b_nk.data_ptr(), sw.data_ptr(),
                 None if bias is None else bias.data_ptr(), M, N, K, out.data_ptr(),
                 _native.dtype_code(out_dtype), ws.data_ptr(), ws_b, st)
    return out


@pytest.mark.gpu
@pytest.mark.parametrize("seed", range(20))
def test_random_gemm_exact(dev, seed):
    rng, M, N, K = _shape(seed)
    g = torch.Generator().manual_seed(seed)
    a = torch.randint(-127, 128, (M, K), generator=g, dtype=torch.int8).to(dev)
    b = torch.randint(-127, 128, (N, K), generator=g, dtype=torch.int8).to(dev)
    c = _gemm(a, b, "i32")
    want = (a.double() @ b.double().t()).to(torch.int64)
    assert torch.equal(c.to(torch.int64), want), (M, N, K)


@pytest.mark.gpu
@pytest.mark.parametrize("seed", range(12))
def test_random_dequant_epilogue_vs_oracle(dev, seed):
    rng, M, N, K = _shape(seed + 100)
    M, N = min(M, 200), min(N, 1000)  # the oracle GEMM runs on the host
    g = torch.Generator().manual_seed(seed)
    a = torch.randint(-127, 128, (M, K), generator=g, dtype=torch.int8)
    b = torch.randint(-127, 128, (N, K), generator=g, dtype=torch.int8)
    sx = torch.rand(M, generator=g) * 0.05 + 1e-4
    sw = torch.rand(N, generator=g) * 0.01 + 1e-5
    bias = torch.randn(N, generator=g) if seed % 2 else None
    acc = O.gemm_i8(a.numpy(), b.numpy().T)
    for dt in (torch.bfloat16, torch.float32):
        out = _gemm(a.to(dev), b.to(dev), "dequant", sx.to(dev), sw.to(dev),
                    None if bias is None else bias.to(dev), dt)
        want = O.int8_epilogue(acc, sx.numpy(), sw.numpy(), None if bias is None else bias.numpy(),
                               O.BF16 if dt == torch.bfloat16 else O.F32)
        got = out.cpu()
        got = got.view(torch.int16).numpy().view(np.uint16) if dt == torch.bfloat16 else got.numpy()
        np.testing.assert_array_equal(got, want)


@pytest.mark.gpu
@pytest.mark.parametrize("seed", range(16))
def test_random_row_stream_exact(dev, seed):
    """Shapes of the row-streaming kernel (K a multiple of 256, 16-48 weight
    rows per CU, up to 128 activation rows, ragged last blocks): int32 against
    the exact product, and the bf16 / fp32 epilogues against the oracle's
    epilogue over that product."""
    rng = np.random.default_rng(500 + seed)
    M, N, K = int(rng.integers(1, 129)), int(rng.integers(3841, 12289)), 256 * int(rng.integers(1, 44))
    g = torch.Generator(device=dev).manual_seed(seed)
    a = torch.randint(-127, 128, (M, K), generator=g, device=dev, dtype=torch.int8)
    b = torch.randint(-127, 128, (N, K), generator=g, device=dev, dtype=torch.int8)
    want = (a.double() @ b.double().t()).to(torch.int64)
    assert torch.equal(_gemm(a, b, "i32").to(torch.int64), want), (M, N, K)
    sx = torch.rand(M, generator=g, device=dev) * 0.05 + 1e-4
    sw = torch.rand(N, generator=g, device=dev) * 0.01 + 1e-5
    bias = torch.randn(N, generator=g, device=dev) if seed % 2 else None
    acc = want.to(torch.int32).cpu().numpy()
    for dt in (torch.bfloat16, torch.float32):
        got = _gemm(a, b, "dequant", sx, sw, bias, dt).cpu()
        ref = O.int8_epilogue(acc, sx.cpu().numpy(), sw.cpu().numpy(),
                              None if bias is None else bias.cpu().numpy(),
                              O.BF16 if dt == torch.bfloat16 else O.F32)
        got = got.view(torch.int16).numpy().view(np.uint16) if dt == torch.bfloat16 else got.numpy()
        np.testing.assert_array_equal(got, ref)
