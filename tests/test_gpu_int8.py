"""GPU parity tests for the INT8 FFN linear (int8_linear.py) and the Quantizer.

Bar: quantized weights/activations, scales and int32 accumulators bit-exact
with the oracle; the bf16/fp32 output of INT8Linear bit-exact too (the
epilogue follows the reference's rounding order exactly).
"""

import numpy as np
import pytest
import torch
import torch.nn as nn

from helpers import DT, bits, to_np
from oracle import oracle as O
from shadowinfer_amd import _native
from shadowinfer_amd.ffn_optimizer import INT8Linear, dequantized_weight, quantize_ffn_modules
from shadowinfer_amd.kernels import _pack_int4, _unpack_int4
from shadowinfer_amd.utils import Quantizer

pytestmark = pytest.mark.gpu


def _gemm_i32(a: torch.Tensor, b_kn: torch.Tensor) -> torch.Tensor:
    """si_gemm_i8i8_i32 through the C ABI; ``b_kn`` is the reference's [K, N]
    operand, passed to the library in its [N, K] layout."""
    M, K = a.shape
    N = b_kn.shape[1]
    b = b_kn.t().contiguous()
    c = torch.empty(M, N, dtype=torch.int32, device=a.device)
    ws_bytes = _native.size_query("si_gemm_workspace_bytes", M, N, K)
    ws = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=a.device)
    _native.call("si_gemm_i8i8_i32", a.data_ptr(), b.data_ptr(), M, N, K, c.data_ptr(),
                 ws.data_ptr(), ws_bytes, _native.stream(a.device))
    return c


def _act_quant(x: torch.Tensor):
    M, K = x.shape
    q = torch.empty(M, K, dtype=torch.int8, device=x.device)
    s = torch.empty(M, dtype=torch.float32, device=x.device)
    _native.call("si_act_quant_i8", x.data_ptr(), _native.dtype_code(x.dtype), M, K, q.data_ptr(),
                 s.data_ptr(), _native.stream(x.device))
    return q, s


def _exact_i32(a: torch.Tensor, b: torch.Tensor) -> torch.Tensor:
    """Exact integer product on the device: float64 sums of int8 products stay
    below 2^53, so the float64 GEMM is exact."""
    return (a.double() @ b.double()).to(torch.int64)


@pytest.mark.parametrize("M,K,N", [(1, 64, 16), (5, 128, 96), (16, 4096, 11008),
                                   (64, 4096, 11008), (33, 256, 48), (300, 512, 272),
                                   (7, 40, 24), (3, 17, 5), (100, 96, 48), (65, 4096, 200),
                                   (900, 1024, 300), (17, 11008, 4096), (16, 11008, 4096),
                                   (16, 4096, 22016), (3, 512, 5000), (20, 2048, 5),
                                   (70, 4096, 33), (130, 11008, 7), (500, 2048, 100),
                                   # one block per CU over ceil(N / 256) rows: ragged last
                                   # block, one k stage, 48-row blocks, a 1-row last block
                                   (1, 256, 4100), (31, 768, 6000), (32, 4096, 12288),
                                   (9, 1280, 3841), (24, 512, 4096)])
def test_gemm_i32_bit_exact_vs_oracle(dev, M, K, N):
    g = torch.Generator().manual_seed(M * 7 + K + N)
    a = torch.randint(-127, 128, (M, K), generator=g, dtype=torch.int8)
    b = torch.randint(-127, 128, (K, N), generator=g, dtype=torch.int8)
    c = _gemm_i32(a.to(dev), b.to(dev)).cpu().numpy()
    np.testing.assert_array_equal(c, O.gemm_i8(a.numpy(), b.numpy()))


@pytest.mark.parametrize("M,K,N", [(256, 4096, 11008), (1024, 4096, 11008),
                                   (2048, 4096, 22016), (2048, 11008, 4096),
                                   (24, 4096, 11008), (48, 11008, 4096), (128, 4096, 11008),
                                   (128, 11008, 4096), (40, 4096, 22016), (100, 4096, 1000),
                                   (256, 11008, 4096), (384, 11008, 4096), (200, 4096, 3000),
                                   (129, 4096, 11008), (200, 4096, 11000), (256, 4096, 12288),
                                   # row streaming with 3..8 16-row activation fragments
                                   (33, 4096, 11008), (80, 4096, 8192), (100, 4096, 6000),
                                   (112, 4096, 12288), (96, 1280, 11008), (48, 1024, 5000),
                                   (64, 512, 5001), (128, 768, 4099), (61, 256, 8190)])
def test_gemm_i32_large_m_exact(dev, M, K, N):
    """FFN shapes (up, fused gate|up and down) against the exact float64 product:
    large M on the 256-row tiles, 129..256 rows of the up projection on the
    128x96 tiles (ragged rows and columns included), 17..128 rows on the
    64x64 / 64x128 / 128x128 tiles with and without split K or streamed per CU
    over 17-48 weight rows (ragged last blocks, three or four LDS stages), and
    the down projection split in K up to 512 rows."""
    g = torch.Generator().manual_seed(M + K)
    a = torch.randint(-127, 128, (M, K), generator=g, dtype=torch.int8).to(dev)
    b = torch.randint(-127, 128, (K, N), generator=g, dtype=torch.int8).to(dev)
    c = _gemm_i32(a, b)
    assert torch.equal(c.to(torch.int64), _exact_i32(a, b))


@pytest.mark.parametrize("N", [(1 << 22) - 8, (1 << 22) + 8])
def test_gemm_i32_wide_output(dev, N):
    """Output rows of 4M columns, just below and just above the width where the
    int32 epilogue leaves its 32-bit-offset buffer stores for per-element ones:
    sampled columns (both ends and a random set) against the exact product."""
    M, K = 33, 128
    g = torch.Generator(device=dev).manual_seed(N)
    a = torch.randint(-127, 128, (M, K), generator=g, device=dev, dtype=torch.int8)
    w = torch.randint(-127, 128, (N, K), generator=g, device=dev, dtype=torch.int8)  # [N, K]
    c = torch.empty(M, N, dtype=torch.int32, device=dev)
    ws_bytes = _native.size_query("si_gemm_workspace_bytes", M, N, K)
    ws = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=dev)
    _native.call("si_gemm_i8i8_i32", a.data_ptr(), w.data_ptr(), M, N, K, c.data_ptr(),
                 ws.data_ptr(), ws_bytes, _native.stream(dev))
    cols = torch.cat([torch.arange(0, 512, device=dev), torch.arange(N - 512, N, device=dev),
                      torch.randint(0, N, (4096,), generator=g, device=dev)])
    want = (a.double() @ w[cols].double().t()).to(torch.int64)
    assert torch.equal(c[:, cols].to(torch.int64), want)


def test_gemm_extreme_values_no_overflow(dev):
    """All -127 x -127 over K=4096: the largest accumulator the layer can produce."""
    a = torch.full((16, 4096), -127, dtype=torch.int8, device=dev)
    b = torch.full((4096, 64), -127, dtype=torch.int8, device=dev)
    assert torch.all(_gemm_i32(a, b) == 4096 * 127 * 127)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32, torch.float16])
@pytest.mark.parametrize("M,K", [(16, 4096), (7, 128), (1024, 4096), (5, 2048), (2, 8192),
                                 (3, 11008), (4, 100), (9, 3000)])
def test_act_quant_bit_exact(dev, dtype, M, K):
    g = torch.Generator().manual_seed(M + K)
    x = torch.randn(M, K, generator=g).to(dtype)
    x[0] = 0  # zero row -> scale 1e-8
    q, s = _act_quant(x.to(dev))
    rq, rs = O.int8_act_quant(to_np(x), DT[dtype])
    np.testing.assert_array_equal(q.cpu().numpy(), rq)
    np.testing.assert_array_equal(s.cpu().numpy().view(np.uint32), rs.view(np.uint32))


def test_weight_quant_bit_exact(dev):
    g = torch.Generator().manual_seed(3)
    w = torch.randn(11008, 4096, generator=g) * 0.02
    w[5] = 0
    lin = nn.Linear(4096, 11008, bias=False)
    with torch.no_grad():
        lin.weight.copy_(w)
    q = INT8Linear.from_linear(lin.to(dev))
    rq, rs = O.int8_weight_quant(w.numpy())
    np.testing.assert_array_equal(q.qweight.cpu().numpy(), rq)
    np.testing.assert_array_equal(q.weight_scale.cpu().numpy().view(np.uint32), rs.view(np.uint32))
    assert q.qweight.shape == (4096, 11008) and q.qweight.dtype == torch.int8


@pytest.fixture(scope="module")
def ffn_layer(dev):
    g = torch.Generator().manual_seed(2)
    w = torch.randn(11008, 4096, generator=g) * 0.02
    lin = nn.Linear(4096, 11008, bias=False)
    with torch.no_grad():
        lin.weight.copy_(w)
    return lin, INT8Linear.from_linear(lin.to(dev)), w


@pytest.mark.parametrize("M", [16, 64, 256, 1024])
def test_int8_linear_config2_bit_exact(dev, ffn_layer, M):
    """X [M, 4096] bf16 ~ N(0,1), W [11008, 4096] ~ N(0, 0.02): quantized
    activations and scales, int32 accumulators and the bf16 output bit-exact."""
    _, layer, w = ffn_layer
    g = torch.Generator().manual_seed(100 + M)
    x = torch.randn(M, 4096, generator=g).to(torch.bfloat16)
    out = layer(x.to(dev))
    assert out.dtype == torch.bfloat16 and out.shape == (M, 11008)
    rq, rs = O.int8_act_quant(to_np(x), O.BF16)
    qd, sd = _act_quant(x.to(dev))
    np.testing.assert_array_equal(qd.cpu().numpy(), rq)
    acc = _gemm_i32(qd, layer.qweight)
    if M <= 64:
        np.testing.assert_array_equal(acc.cpu().numpy(), O.gemm_i8(rq, layer.qweight.cpu().numpy()))
    else:
        assert torch.equal(acc.to(torch.int64), _exact_i32(qd, layer.qweight))
    ref = O.int8_epilogue(acc.cpu().numpy(), rs, layer.weight_scale.cpu().numpy(), None, O.BF16)
    np.testing.assert_array_equal(to_np(out), ref)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_int8_linear_bias_bit_exact(dev, dtype):
    torch.manual_seed(1)
    lin = nn.Linear(128, 96, bias=True)
    layer = INT8Linear.from_linear(lin.to(dev))
    x = torch.randn(64, 128).to(dtype)
    out = layer(x.to(dev))
    ref, _, _, _ = O.int8_linear_forward(to_np(x), DT[dtype], layer.qweight.cpu().numpy(),
                                         layer.weight_scale.cpu().numpy(),
                                         layer.bias.cpu().numpy())
    np.testing.assert_array_equal(to_np(out), ref)


# --- reference test_int8_ffn.py behaviours, on the device ------------------
def _rel_l2(a, b):
    a, b = a.detach().float(), b.detach().float()
    return (torch.linalg.vector_norm(a - b) / torch.linalg.vector_norm(b).clamp_min(1e-12)).item()


@pytest.mark.parametrize("bias", [False, True])
def test_relative_error_shape_dtype(dev, bias):
    torch.manual_seed(0)
    lin = nn.Linear(128, 96, bias=bias).to(dev)
    layer = INT8Linear.from_linear(lin)
    x = torch.randn(64, 128, device=dev)
    out = layer(x)
    assert out.shape == (64, 96) and out.dtype == x.dtype
    assert _rel_l2(out, lin(x)) <= 0.03
    assert layer.qweight.shape == (128, 96) and layer.weight_scale.dtype == torch.float32
    assert (layer.bias is not None) == bias


def test_batched_and_1d_inputs(dev):
    torch.manual_seed(2)
    layer = INT8Linear.from_linear(nn.Linear(128, 96, bias=True).to(dev))
    x = torch.randn(2, 5, 128, device=dev)
    batched = layer(x)
    assert batched.shape == (2, 5, 96)
    assert torch.equal(batched, layer(x.reshape(-1, 128)).reshape(2, 5, 96))
    single = layer(x[0, 0])
    assert single.shape == (96,) and torch.equal(single, batched[0, 0])


@pytest.mark.parametrize("kind", ["zero", "constant", "large"])
def test_extreme_inputs_finite(dev, kind):
    torch.manual_seed(3)
    layer = INT8Linear.from_linear(nn.Linear(128, 96, bias=True).to(dev))
    x = {"zero": torch.zeros(4, 128), "constant": torch.full((4, 128), 0.5),
         "large": torch.randn(4, 128) * 1e4}[kind].to(dev)
    out = layer(x)
    assert bool(torch.isfinite(out).all())


def test_state_dict_uses_reference_layout(dev):
    """The state dict holds the reference's qweight [K, N]; loading it (or a
    reference-made state dict) restores the same layer."""
    torch.manual_seed(4)
    layer = INT8Linear.from_linear(nn.Linear(128, 96, bias=True).to(dev))
    sd = layer.state_dict()
    assert set(sd) == {"qweight", "weight_scale", "bias"}
    assert sd["qweight"].shape == (128, 96) and sd["qweight"].is_contiguous()
    fresh = INT8Linear(torch.zeros(128, 96, dtype=torch.int8, device=dev),
                       torch.ones(96, device=dev), bias=torch.zeros(96, device=dev))
    fresh.load_state_dict(sd)
    assert torch.equal(fresh.qweight, layer.qweight)
    x = torch.randn(8, 128, device=dev)
    assert torch.equal(fresh(x), layer(x))
    built = INT8Linear(sd["qweight"], sd["weight_scale"], sd["bias"])
    assert torch.equal(built(x), layer(x))


def test_empty_invalid_and_memory(dev):
    layer = INT8Linear.from_linear(nn.Linear(128, 96, bias=True).to(dev))
    assert layer(torch.empty(0, 128, device=dev)).shape == (0, 96)
    with pytest.raises(ValueError):
        layer(torch.randn(4, 127, device=dev))
    assert layer.memory_bytes() == 128 * 96 + 4 * 96 + 4 * 96
    assert layer.dense_equivalent_bytes() == 4 * 128 * 96 + 4 * 96
    assert layer.using_int_mm
    dq = dequantized_weight(layer)
    assert dq.shape == (128, 96)


def test_quantize_ffn_modules(dev):
    class MLP(nn.Module):
        def __init__(self):
            super().__init__()
            self.up_proj = nn.Linear(64, 128)
            self.down_proj = nn.Linear(128, 64)

    class Block(nn.Module):
        def __init__(self):
            super().__init__()
            self.mlp = MLP()
            self.other = nn.Linear(64, 64)

    model = Block().to(dev)
    stats = quantize_ffn_modules(model, keep_fp32_reference=True)
    assert stats["supported"] and stats["modules"] == 2 and not stats["fallback"]
    assert isinstance(model.mlp.up_proj, INT8Linear) and isinstance(model.other, nn.Linear)
    again = quantize_ffn_modules(model)
    assert again["modules"] == 2
    assert quantize_ffn_modules(nn.Linear(4, 4).to(dev)) == {"supported": False}


# --- Quantizer on the device ----------------------------------------------
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
def test_quantizer_int8_int4_bit_exact(dev, dtype):
    g = torch.Generator().manual_seed(9)
    x = torch.randn(10, 3, 64, generator=g).to(dtype)
    q, s = Quantizer.quantize_int8(x.to(dev))
    rq, rs = O.quant_rows_i8(to_np(x), DT[dtype])
    np.testing.assert_array_equal(q.cpu().numpy(), rq)
    np.testing.assert_array_equal(bits(s), rs.reshape(-1).view(np.uint8))
    q4, s4 = Quantizer.quantize_int4(x.to(dev), group_size=16)
    rq4, rs4 = O.quant_rows_i4(to_np(x), DT[dtype], 16)
    assert q4.shape == (10, 3, 4, 16) and s4.shape == (10, 3, 4, 1)
    np.testing.assert_array_equal(q4.cpu().numpy(), rq4)
    np.testing.assert_array_equal(bits(s4), rs4.reshape(-1).view(np.uint8))
    dq = Quantizer.dequantize_int8(q, s)
    np.testing.assert_array_equal(dq.cpu().numpy(), O.dequant_rows(rq, rs, DT[dtype], 64))
    dq4 = Quantizer.dequantize_int4(q4, s4)
    assert dq4.shape == (10, 3, 64)
    with pytest.raises(ValueError):
        Quantizer.quantize_int4(x.to(dev), group_size=24)


def test_quantizer_dequant_broadcasts_like_torch(dev):
    """dequantize_* is q.float() * scale with any broadcastable scale
    (quantization.py:180-219): per-row, per-group, per-tensor, 0-d (also a 0-d
    CPU scale, which torch broadcasts onto a device tensor), per-element and a
    scale with more leading dims; bf16/fp16/fp32 scales; the empty round trip."""
    g = torch.Generator().manual_seed(3)
    q = torch.randint(-128, 128, (6, 5, 32), generator=g, dtype=torch.int8)
    qd = q.to(dev)
    cases = [torch.rand(6, 5, 1, generator=g), torch.rand(1, generator=g),
             torch.rand((), generator=g), torch.rand(5, 32, generator=g),
             torch.rand(6, 5, 32, generator=g), torch.rand(3, 1, 1, 1, generator=g)]
    for sc in cases:
        for dt in (torch.float32, torch.bfloat16, torch.float16):
            s_ = sc.to(dt)
            got = Quantizer.dequantize_int8(qd, s_.to(dev))
            want = q.float() * s_
            assert got.shape == want.shape and got.dtype == torch.float32
            assert torch.equal(got.cpu(), want)
            want_o = O.to_f32(to_np(q.expand(want.shape).contiguous()).astype(np.float32), O.F32) \
                * O.to_f32(to_np(s_.expand(want.shape).contiguous()), DT[dt])
            np.testing.assert_array_equal(got.cpu().numpy(), want_o)
    s0 = torch.tensor(0.5)
    assert torch.equal(Quantizer.dequantize_int8(qd, s0).cpu(), q.float() * s0)
    q4 = torch.randint(-8, 8, (4, 3, 2, 16), generator=g, dtype=torch.int8)
    for sc in (torch.rand(4, 3, 2, 1, generator=g), torch.rand((), generator=g)):
        got = Quantizer.dequantize_int4(q4.to(dev), sc.to(dev))
        want = (q4.float() * sc).reshape(4, 3, -1)
        assert torch.equal(got.cpu(), want)
    for fn in (Quantizer.quantize_int8, lambda t: Quantizer.quantize_int4(t, group_size=16)):
        qe, se = fn(torch.empty(0, 16, device=dev))
        de = Quantizer.dequantize_int8(qe, se)
        assert de.shape == (0, 16) and de.dtype == torch.float32
    with pytest.raises(TypeError):
        Quantizer.dequantize_int8(qd, torch.rand(6, 5, 1, dtype=torch.float64, device=dev))
    with pytest.raises(RuntimeError):
        Quantizer.dequantize_int8(qd, torch.rand(7, 1, device=dev))


def test_quantizer_known_answers(dev):
    """Scale of [1, -2, 3, -4] is 4/127 (reference test_kernels.py:72-77);
    zero rows get scale 1 and codes 0."""
    q, s = Quantizer.quantize_int8(torch.tensor([[1.0, -2.0, 3.0, -4.0]], device=dev))
    assert abs(s.item() - 4.0 / 127.0) < 1e-6
    assert q.tolist() == [[32, -64, 95, -127]]
    q0, s0 = Quantizer.quantize_int8(torch.zeros(2, 8, device=dev))
    assert torch.all(s0 == 1) and torch.all(q0 == 0)


@pytest.mark.parametrize("n", [0, 1, 2, 23, 128, 1001])
def test_int4_pack_unpack(dev, n):
    g = torch.Generator().manual_seed(n)
    t = torch.randint(-8, 8, (n,), generator=g, dtype=torch.int8)
    packed = Quantizer.pack_int4(t.to(dev))
    assert packed.dtype == torch.uint8 and packed.numel() == (n + 1) // 2
    np.testing.assert_array_equal(packed.cpu().numpy(), O.pack_int4_flat(t.numpy()))
    assert torch.equal(Quantizer.unpack_int4(packed, n).cpu(), t)
    assert torch.equal(_unpack_int4(_pack_int4(t.to(dev)), n).cpu(), t)


def test_int4_all_nibble_pairs(dev):
    """Every (hi, lo) pair of codes in [-8, 7] packs to ((hi+8) << 4) | (lo+8)."""
    hi, lo = torch.meshgrid(torch.arange(-8, 8), torch.arange(-8, 8), indexing="ij")
    t = torch.stack([hi.reshape(-1), lo.reshape(-1)], dim=1).reshape(-1).to(torch.int8)
    packed = Quantizer.pack_int4(t.to(dev)).cpu()
    expected = ((hi.reshape(-1) + 8) << 4) | (lo.reshape(-1) + 8)
    assert torch.equal(packed.to(torch.int64), expected)


# --- the down projection's residual add fused into the epilogue ------------
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("M,K,N,bias", [(16, 4096, 11008, False), (8, 320, 3000, True),
                                        (64, 4096, 11008, False), (48, 11008, 4096, True),
                                        (300, 512, 272, True), (5, 40, 24, False),
                                        (128, 4000, 300, False), (200, 128, 9600, True),
                                        (100, 4096, 6000, True), (64, 512, 5001, True),
                                        (128, 768, 4100, False)])
def test_gemm_dequant_add_bit_exact(dev, dtype, M, K, N, bias):
    """si_gemm_i8_dequant_add = T(residual + T(acc * (sx * sw) [+ bias])), the
    INT8Linear output rounded to T and added to the residual stream in T
    (diffusion_llama.py:421-423), on shapes that reach the row-streaming,
    weight-streaming, 64x64, split-K, 128x96, large-tile, register-staged and
    scalar kernels; also in place (out is the residual buffer)."""
    from oracle import denoise_ref as R
    g = torch.Generator().manual_seed(M + 3 * K + N)
    a = torch.randint(-127, 128, (M, K), generator=g, dtype=torch.int8)
    b = torch.randint(-127, 128, (N, K), generator=g, dtype=torch.int8)
    sx = torch.rand(M, generator=g) * 0.05 + 1e-3
    sw = torch.rand(N, generator=g) * 1e-3 + 1e-5
    bs = torch.randn(N, generator=g) if bias else None
    resid = (torch.randn(M, N, generator=g) * 4).to(dtype)
    dt = DT[dtype]
    ffn = O.int8_epilogue(O.gemm_i8(a.numpy(), b.numpy().T), sx.numpy(), sw.numpy(),
                          None if bs is None else bs.numpy(), dt)
    want = R.add(to_np(resid), ffn, dt)
    ad, bd, sxd, swd = a.to(dev), b.to(dev), sx.to(dev), sw.to(dev)
    bsd = None if bs is None else bs.to(dev)
    ws_bytes = _native.size_query("si_gemm_workspace_bytes", M, N, K)
    ws = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=dev)
    rd = resid.to(dev)
    for in_place in (False, True):
        out = rd.clone() if in_place else torch.empty(M, N, dtype=dtype, device=dev)
        src = out if in_place else rd
        _native.call("si_gemm_i8_dequant_add", ad.data_ptr(), sxd.data_ptr(), bd.data_ptr(),
                     swd.data_ptr(), _native.ptr(bsd), src.data_ptr(), M, N, K, out.data_ptr(),
                     _native.dtype_code(dtype), ws.data_ptr(), ws_bytes, _native.stream(dev))
        np.testing.assert_array_equal(to_np(out), want)


@pytest.mark.parametrize("M,K,N", [(16, 4096, 11008), (64, 128, 96), (2048, 11008, 4096)])
def test_int8_linear_forward_add_bit_exact(dev, M, K, N):
    """si_int8_linear_forward_add: the whole INT8Linear forward (activation
    quantization, GEMM, epilogue) then the residual add, bf16."""
    from oracle import denoise_ref as R
    torch.manual_seed(M + K)
    lin = nn.Linear(K, N, bias=(M == 64))
    layer = INT8Linear.from_linear(lin.to(dev))
    g = torch.Generator().manual_seed(M)
    x = torch.randn(M, K, generator=g).to(torch.bfloat16)
    resid = torch.randn(M, N, generator=g).to(torch.bfloat16)
    ref, _, _, _ = O.int8_linear_forward(to_np(x), O.BF16, layer.qweight.cpu().numpy(),
                                         layer.weight_scale.cpu().numpy(),
                                         None if layer.bias is None else layer.bias.cpu().numpy())
    want = R.add(to_np(resid), ref, O.BF16)
    xd, rd = x.to(dev), resid.to(dev)
    out = torch.empty(M, N, dtype=torch.bfloat16, device=dev)
    ws_bytes = _native.size_query("si_int8_linear_workspace_bytes", M, K, N)
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device=dev)
    _native.call("si_int8_linear_forward_add", xd.data_ptr(), _native.DT_BF16, M, K, N,
                 layer.qweight_nk.data_ptr(), layer.weight_scale.data_ptr(),
                 _native.ptr(layer.bias), rd.data_ptr(), out.data_ptr(), ws.data_ptr(), ws_bytes,
                 _native.stream(dev))
    np.testing.assert_array_equal(to_np(out), want)
