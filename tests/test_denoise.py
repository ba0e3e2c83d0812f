"""Denoising step of a Llama-shaped diffusion LM on packed KV + INT8 FFN
(models/diffusion_llama.py:311-424, execution/step_reuse.py,
execution/block_decoding.py:118-158).

CPU: the float64 reference of the row kernels (oracle/denoise_ref.py) is pinned
by closed forms and invariants, and the unmasking rule by the reference's own
known-answer construction (tests/test_block_decoding.py:51-88: logits rows of a
prescribed confidence, per-element rule with smallest-index ties).

GPU: every kernel of the step against that reference; then a whole two-layer
model, stage by stage from the GPU's own stage inputs (bit-exact for the packed
KV, the int8 activations, the INT8 GEMM outputs and the residual add; at most
one unit in the last place for the fp32-arithmetic row kernels; relL2 bounds
written below for the bf16 library GEMMs and attention), and end to end.
Step reuse and the unmasking loop are checked on the same model.
"""

import math

import numpy as np
import pytest
import torch
import torch.nn.functional as F
from scipy.special import expit

from helpers import DT, assert_cache_equal, to_np
from oracle import denoise_ref as R
from oracle import oracle as O


def _mono(bits_arr):
    """Monotonic integer image of float bit patterns (uint16 or uint32/fp32)."""
    a = np.ascontiguousarray(bits_arr)
    if a.dtype == np.float32:
        i = a.view(np.int32).astype(np.int64)
        return np.where(i < 0, -(i & 0x7FFFFFFF), i)
    i = a.astype(np.int64)
    return np.where(i & 0x8000, -(i & 0x7FFF), i)


def ulp_diff(a, b):
    return np.abs(_mono(a) - _mono(b))


def assert_row_kernel_close(got, want, dtype, max_ulp=1):
    """fp32-arithmetic row kernels: each rounding to a 16-bit dtype lands on the
    reference's value or its neighbour (rarely), so a chain of r roundings
    stays within r units in the last place; fp32 outputs keep the fp32
    reduction/contraction error (relative 3e-5)."""
    if dtype == torch.float32:
        np.testing.assert_allclose(got, want, rtol=3e-5, atol=1e-6)
        return
    d = ulp_diff(got, want)
    assert d.max() <= max_ulp and (d > 0).mean() <= 1e-2, (int(d.max()), float((d > 0).mean()))


def rel_l2(a, b):
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    return float(np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-30))


def f32(x, dt):
    return O.to_f32(np.ascontiguousarray(x), dt)


# ----------------------------------------------------------------- CPU pins
def _t16(a):
    """uint16 bf16 bit patterns -> CPU bf16 tensor."""
    return torch.from_numpy(np.ascontiguousarray(a).view(np.int16)).view(torch.bfloat16)


def test_rmsnorm_ref_closed_form_and_invariants():
    # constant row c: y = c / sqrt(c^2 + eps) (catches eps outside the sqrt)
    for c, eps in ((1e-3, 1e-5), (2.0, 1e-6), (-0.5, 0.0)):
        x = np.full((1, 64), c, np.float32)
        y = R.rmsnorm(x, O.F32, np.ones(64, np.float32), eps)
        np.testing.assert_allclose(y, c / math.sqrt(c * c + eps), rtol=1e-6)
    rng = np.random.default_rng(0)
    x = rng.standard_normal((5, 96)).astype(np.float32)
    w = rng.uniform(0.5, 1.5, 96).astype(np.float32)
    y = R.rmsnorm(x, O.F32, w, 0.0)
    # unit weight, eps 0: every row has RMS 1; scale-free; linear in w
    y1 = R.rmsnorm(x, O.F32, np.ones(96, np.float32), 0.0)
    np.testing.assert_allclose(np.sqrt((y1.astype(np.float64) ** 2).mean(-1)), 1.0, rtol=1e-6)
    np.testing.assert_array_equal(R.rmsnorm(4 * x, O.F32, w, 0.0), y)
    np.testing.assert_array_equal(R.rmsnorm(x, O.F32, 2 * w, 0.0), 2 * y)


@pytest.mark.parametrize("K", [64, 4096])
def test_rmsnorm_ref_is_the_torch_op_chain(K):
    """DiffusionLlamaRMSNorm.forward's ops run in CPU bf16 torch (a power-of-two
    K, where torch's CPU mean and its GPU mean round alike) give the oracle's
    bits on every row it does not flag; rounding once instead of per op would
    differ on most rows."""
    g = torch.Generator().manual_seed(K)
    x = (torch.randn(384, K, generator=g) * 3).to(torch.bfloat16)
    w = (torch.rand(K, generator=g) + 0.5).to(torch.bfloat16)
    want = to_np(x / torch.sqrt(x.pow(2).mean(-1, keepdim=True) + 1e-5) * w)
    y, amb = R.rmsnorm(to_np(x), O.BF16, to_np(w), 1e-5, return_ambiguous=True)
    assert amb.mean() < 0.05
    np.testing.assert_array_equal(y[~amb], want[~amb])
    once = O.from_f32((f32(to_np(x), O.BF16).astype(np.float64) / np.sqrt(
        (f32(to_np(x), O.BF16).astype(np.float64) ** 2).mean(-1, keepdims=True) + 1e-5)
        * f32(to_np(w), O.BF16)).astype(np.float32), O.BF16)
    assert (once != want).any(-1).mean() > 0.5


def test_rope_ref_rotation():
    B, S, H, D = 1, 9, 2, 64
    rng = np.random.default_rng(1)
    inv = 1.0 / (10000.0 ** (np.arange(0, D, 2, dtype=np.float64) / D))
    ang = np.outer(np.arange(S), inv)
    emb = np.concatenate([ang, ang], -1)
    cos, sin = np.cos(emb).astype(np.float32), np.sin(emb).astype(np.float32)
    qkv = rng.standard_normal((B * S, 3 * H * D)).astype(np.float32)
    q, k, v = R.rope_split(qkv, O.F32, cos, sin, B, S, H, D)
    x = qkv.reshape(B, S, 3, H, D).transpose(2, 0, 3, 1, 4)
    np.testing.assert_array_equal(v, x[2])
    np.testing.assert_array_equal(q[:, :, 0], x[0][:, :, 0])      # position 0: identity
    h = D // 2
    # pair norms are preserved
    n_in = x[0][..., :h] ** 2 + x[0][..., h:] ** 2
    n_out = q[..., :h].astype(np.float64) ** 2 + q[..., h:].astype(np.float64) ** 2
    np.testing.assert_allclose(n_out, n_in, rtol=1e-5)
    # sign convention of rotate_half: e_0 at position p -> (cos p, ..., sin p at d = D/2)
    e = np.zeros((B * S, 3 * H * D), np.float32)
    e[:, 0] = 1.0
    qe, _, _ = R.rope_split(e, O.F32, cos, sin, B, S, H, D)
    np.testing.assert_allclose(qe[0, 0, :, 0], np.cos(np.arange(S)), rtol=1e-6, atol=1e-7)
    np.testing.assert_allclose(qe[0, 0, :, h], np.sin(np.arange(S)), rtol=1e-6, atol=1e-7)
    # scores depend only on the position difference
    a, b = rng.standard_normal(D), rng.standard_normal(D)
    one = np.zeros((S, 3 * H * D), np.float32)
    one[:, :D] = a
    one[:, H * D:H * D + D] = b
    qq, kk, _ = R.rope_split(one, O.F32, cos, sin, 1, S, H, D)
    s1 = float(np.dot(qq[0, 0, 5], kk[0, 0, 2]))
    s2 = float(np.dot(qq[0, 0, 8], kk[0, 0, 5]))
    assert abs(s1 - s2) < 1e-4 * max(1.0, abs(s1))


def _rotate_half(t):
    h = t.shape[-1] // 2
    return torch.cat((-t[..., h:], t[..., :h]), dim=-1)


def test_rope_ref_is_the_torch_op_chain():
    """q * cos + rotate_half(q) * sin in CPU bf16 torch (diffusion_llama.py:288-292,
    372-373): bit for bit (no reduction is involved)."""
    B, S, H, D = 2, 40, 3, 128
    g = torch.Generator().manual_seed(5)
    qkv = (torch.randn(B * S, 3 * H * D, generator=g) * 2).to(torch.bfloat16)
    inv = 1.0 / (10000.0 ** (torch.arange(0, D, 2, dtype=torch.float32) / D))
    emb = torch.outer(torch.arange(S, dtype=torch.float32), inv)
    emb = torch.cat((emb, emb), -1)
    cos, sin = emb.cos().to(torch.bfloat16), emb.sin().to(torch.bfloat16)
    x = qkv.view(B, S, 3, H, D)
    rq, rk, rv = R.rope_split(to_np(qkv), O.BF16, to_np(cos), to_np(sin), B, S, H, D)
    for j, got in ((0, rq), (1, rk)):
        t = x[:, :, j].transpose(1, 2)
        np.testing.assert_array_equal(got, to_np(t * cos + _rotate_half(t) * sin))
    np.testing.assert_array_equal(rv, to_np(x[:, :, 2].transpose(1, 2)))


def test_swiglu_ref_is_the_torch_op_chain():
    """F.silu(gate) * up in CPU bf16 torch (diffusion_llama.py:333): equal on
    every element the oracle does not flag, and a zero gate gives zero."""
    g = torch.Generator().manual_seed(2)
    gate = (torch.randn(64, 1024, generator=g) * 4).to(torch.bfloat16)
    up = torch.randn(64, 1024, generator=g).to(torch.bfloat16)
    h, amb = R.swiglu(np.concatenate([to_np(gate), to_np(up)], 1), O.BF16, return_ambiguous=True)
    want = to_np(F.silu(gate) * up)
    assert amb.mean() < 0.01
    np.testing.assert_array_equal(h[~amb], want[~amb])
    gf = f32(to_np(gate), O.BF16).astype(np.float64)
    assert ulp_diff(O.from_f32((gf * expit(gf)).astype(np.float32), O.BF16),
                    to_np(F.silu(gate))).max() <= 1
    z = R.swiglu(np.zeros((1, 16), np.float32), O.F32)
    np.testing.assert_array_equal(z, 0.0)


def _bf16_bits(x):
    return O.from_f32(np.asarray(x, np.float32), O.BF16)


def test_argmax_conf_ref_known_answers():
    """softmax(logits).max(-1) in bf16 (block_decoding.py:146-147).
    Row 0: logits 0 and 0.001 have probabilities that round to the same bf16
    value, so the FIRST index wins although index 1 holds the larger logit.
    Row 1: a NaN gives NaN and index 0. Row 2: +inf likewise. Row 3: -inf
    entries have probability 0 and do not take part; the tie of the two 3.0
    logits goes to the first."""
    rows = [[0.0, 0.001, -3.0, -3.0], [0.0, float("nan"), 1.0, 2.0],
            [0.0, 1.0, float("inf"), 2.0], [float("-inf"), 3.0, float("-inf"), 3.0]]
    lg = _bf16_bits(rows)
    tok, conf = R.argmax_conf(lg, O.BF16)
    ref_p = torch.softmax(_t16(lg), -1)
    rc, rt = ref_p.max(-1)
    np.testing.assert_array_equal(tok, rt.numpy())
    np.testing.assert_array_equal(conf, to_np(rc))
    assert f32(lg, O.BF16)[0, 1] > f32(lg, O.BF16)[0, 0]
    assert tok[0] == 0 and tok[1] == 0 and tok[2] == 0 and tok[3] == 1
    assert np.isnan(f32(conf[1:3], O.BF16)).all()
    assert f32(conf[3:], O.BF16)[0] == 0.5


@pytest.mark.parametrize("dtype,V,scale", [(torch.bfloat16, 1000, 0.05), (torch.bfloat16, 32000, 1.0),
                                           (torch.float32, 1000, 0.05)])
def test_argmax_conf_ref_is_the_torch_op_chain(dtype, V, scale):
    """torch.softmax(logits, -1).max(-1) in CPU torch on random logits equals
    the oracle on every row it does not flag; the argmax of the logits (the
    rule this replaces) differs from it on a sizeable share of bf16 rows."""
    g = torch.Generator().manual_seed(V)
    lg = (torch.randn(192, V, generator=g) * scale).to(dtype)
    c, t = torch.softmax(lg, -1).max(-1)
    rt, rc, amb = R.argmax_conf(to_np(lg), DT[dtype], return_ambiguous=True)
    assert amb.mean() < 0.05
    np.testing.assert_array_equal(rt[~amb], t.numpy()[~amb])
    if dtype == torch.float32:
        np.testing.assert_allclose(rc, to_np(c), rtol=2 * R.SUM_REL_ERR)
    else:
        np.testing.assert_array_equal(rc[~amb], to_np(c)[~amb])
    if dtype == torch.bfloat16 and scale < 1:
        assert (lg.float().argmax(-1).numpy() != rt).mean() > 0.02


def _conf_row(conf, token, vocab):
    """Logits whose max softmax probability is ``conf`` at ``token``
    (the construction of the reference's tests/test_block_decoding.py:51-57)."""
    row = np.full(vocab, math.log((1.0 - conf) / (conf * (vocab - 1))), np.float32)
    row[token] = 0.0
    return row


def test_schedule_ref_known_answers():
    V = 16
    confs = [[0.95, 0.2, 0.91, 0.5], [0.3, 0.6, 0.6, 0.1], [0.99, 0.99, 0.2, 0.2]]
    toks = [[3, 4, 5, 6], [1, 2, 3, 4], [7, 8, 9, 10]]
    logits = np.stack([np.stack([_conf_row(c, t, V) for c, t in zip(cr, tr)])
                       for cr, tr in zip(confs, toks)])
    masked = np.array([[1, 1, 1, 1], [1, 1, 1, 0], [0, 0, 0, 0]], bool)
    tok, conf = R.argmax_conf(logits, O.F32)
    np.testing.assert_array_equal(tok, np.array(toks))
    np.testing.assert_allclose(conf, np.array(confs), rtol=1e-5)
    unmask, fb = R.schedule(conf, masked, 0.9, O.F32)
    # row 0: both above 0.9; row 1: fallback, tie 0.6/0.6 -> smaller index;
    # row 2: nothing masked
    np.testing.assert_array_equal(unmask, [[1, 0, 1, 0], [0, 1, 0, 0], [0, 0, 0, 0]])
    np.testing.assert_array_equal(fb, [False, True, False])


def test_schedule_ref_threshold_in_the_logits_dtype():
    """A bf16 confidence of 0.8984375 (= bf16(0.9)) reaches the 0.9 threshold,
    as torch's bf16 comparison with a Python float decides; 0.89453125 does not.
    Two tied bf16 confidences fall back to the smaller position."""
    conf = _bf16_bits([[0.8984375, 0.5], [0.89453125, 0.5], [0.25, 0.25]])
    masked = np.ones((3, 2), bool)
    unmask, fb = R.schedule(conf, masked, 0.9, O.BF16)
    want = (_t16(conf) >= 0.9).numpy()
    np.testing.assert_array_equal(unmask[0], want[0])
    np.testing.assert_array_equal(unmask, [[1, 0], [1, 0], [1, 0]])
    np.testing.assert_array_equal(fb, [False, True, True])


# ------------------------------------------------------------------ GPU
def _need_lib():
    from shadowinfer_amd import _native
    _native.load()


def _assert_rows_equal(got, want, amb, dtype):
    """Equal bits on every row the oracle does not flag (16-bit dtypes); fp32
    rows keep the fp32 reduction-order error."""
    if dtype == torch.float32:
        np.testing.assert_allclose(got, want, rtol=4 * R.SUM_REL_ERR, atol=1e-30)
        return
    assert amb.mean() < 0.05
    np.testing.assert_array_equal(got[~amb], want[~amb])


@pytest.mark.gpu
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("M,K", [(1, 8), (37, 256), (64, 4096), (5, 11008), (3, 16384)])
def test_rmsnorm_kernel(dev, dtype, M, K):
    """RMSNorm as the reference's op chain: against the oracle and against the
    same torch ops on the GPU; with the residual add fused in front."""
    from shadowinfer_amd.execution import row_ops
    g = torch.Generator().manual_seed(M * 7 + K)
    x = (torch.randn(M, K, generator=g) * 3).to(dtype)
    o = torch.randn(M, K, generator=g).to(dtype)
    w = (torch.rand(K, generator=g) + 0.5).to(dtype)
    y, q, s, _ = row_ops.rmsnorm(x.to(dev), w.to(dev), 1e-5, want_y=True, want_q=True)
    dt = DT[dtype]
    want, amb = R.rmsnorm(to_np(x), dt, to_np(w), 1e-5, return_ambiguous=True)
    _assert_rows_equal(to_np(y), want, amb, dtype)
    xd, wd = x.to(dev), w.to(dev)
    torch_y = xd / torch.sqrt(xd.pow(2).mean(-1, keepdim=True) + 1e-5) * wd
    _assert_rows_equal(to_np(y), to_np(torch_y), amb, dtype)
    qr, sr = O.int8_act_quant(to_np(y), dt)      # fused quantization of the kernel's own y
    np.testing.assert_array_equal(to_np(q), qr)
    np.testing.assert_array_equal(to_np(s), sr)
    _, q2, s2, _ = row_ops.rmsnorm(x.to(dev), w.to(dev), 1e-5, want_y=False, want_q=True)
    assert torch.equal(q2, q) and torch.equal(s2, s)
    # residual add + RMSNorm: x1 = x + o in the dtype, then the same chain
    y3, q3, s3, x1 = row_ops.rmsnorm(x.to(dev), w.to(dev), 1e-5, want_q=True, residual=o.to(dev))
    np.testing.assert_array_equal(to_np(x1), R.add(to_np(x), to_np(o), dt))
    assert torch.equal(x1, xd + o.to(dev))
    want3, amb3 = R.rmsnorm(to_np(x1), dt, to_np(w), 1e-5, return_ambiguous=True)
    _assert_rows_equal(to_np(y3), want3, amb3, dtype)
    qr3, sr3 = O.int8_act_quant(to_np(y3), dt)
    np.testing.assert_array_equal(to_np(q3), qr3)
    np.testing.assert_array_equal(to_np(s3), sr3)


@pytest.mark.gpu
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("B,S,H,D", [(1, 7, 3, 64), (2, 33, 4, 128), (1, 256, 32, 128)])
def test_rope_kernel(dev, dtype, B, S, H, D):
    """Bit-exact to the oracle and to q * cos + rotate_half(q) * sin on the GPU."""
    from shadowinfer_amd.execution import row_ops
    g = torch.Generator().manual_seed(S * H + D)
    qkv = torch.randn(B * S, 3 * H * D, generator=g).to(dtype)
    inv = 1.0 / (10000.0 ** (torch.arange(0, D, 2, dtype=torch.float32) / D))
    emb = torch.outer(torch.arange(S, dtype=torch.float32), inv)
    emb = torch.cat((emb, emb), -1)
    cos, sin = emb.cos().to(dtype), emb.sin().to(dtype)
    q, k, v = row_ops.rope_split(qkv.to(dev), cos.to(dev), sin.to(dev), B, S, H, D)
    dt = DT[dtype]
    rq, rk, rv = R.rope_split(to_np(qkv), dt, to_np(cos), to_np(sin), B, S, H, D)
    np.testing.assert_array_equal(to_np(q), rq)
    np.testing.assert_array_equal(to_np(k), rk)
    np.testing.assert_array_equal(to_np(v), rv)
    x = qkv.to(dev).view(B, S, 3, H, D)
    c, sn = cos.to(dev), sin.to(dev)
    for j, got in ((0, q), (1, k)):
        t = x[:, :, j].transpose(1, 2)
        assert torch.equal(got, t * c + _rotate_half(t) * sn)


@pytest.mark.gpu
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("M,F", [(1, 8), (19, 512), (64, 11008), (2, 16384)])
def test_swiglu_kernel(dev, dtype, M, F):
    """h = silu(gate) * up bit for bit as torch computes it on the GPU
    (F.silu then the product, both in the dtype); against the oracle on every
    element it does not flag (its exp is correctly rounded, the device's expf
    may be an ulp off)."""
    from shadowinfer_amd.execution import row_ops
    g = torch.Generator().manual_seed(M + F)
    gu = (torch.randn(M, 2 * F, generator=g) * 3).to(dtype)
    gu[0, :8] = torch.tensor([0.0, -0.0, 80.0, -80.0, 100.0, -100.0, 1e-3, -1e-3]).to(dtype)
    h, q, s = row_ops.swiglu_quant(gu.to(dev), want_h=True)
    dt = DT[dtype]
    gd = gu.to(dev)
    torch_h = torch.nn.functional.silu(gd[:, :F]) * gd[:, F:]
    assert torch.equal(h, torch_h)
    want, amb = R.swiglu(to_np(gu), dt, return_ambiguous=True)
    if dtype == torch.float32:      # no rounding to absorb the device expf's ulp
        np.testing.assert_allclose(to_np(h), want, rtol=4 * 2.0 ** -23, atol=1e-37)
    else:
        assert amb.mean() < 0.01
        np.testing.assert_array_equal(to_np(h)[~amb], want[~amb])
    qr, sr = O.int8_act_quant(to_np(h), dt)
    np.testing.assert_array_equal(to_np(q), qr)
    np.testing.assert_array_equal(to_np(s), sr)
    _, q2, s2 = row_ops.swiglu_quant(gu.to(dev), want_h=False)
    assert torch.equal(q2, q) and torch.equal(s2, s)


@pytest.mark.gpu
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_swiglu_every_gate_value(dev, dtype):
    """Every one of the 2^16 gate bit patterns (NaN and inf included) with
    up = 1 and up = -3: h equals torch's silu(gate) * up on the GPU bit for
    bit, NaN where torch gives NaN."""
    from shadowinfer_amd.execution import row_ops
    F = 8192
    gate = torch.arange(1 << 16, dtype=torch.int32).to(torch.int16).view(dtype).view(8, F)
    for up_val in (1.0, -3.0):
        up = torch.full((8, F), up_val, dtype=dtype)
        gd = torch.cat([gate, up], 1).to(dev)
        h, _, _ = row_ops.swiglu_quant(gd, want_h=True)
        want = torch.nn.functional.silu(gd[:, :F]) * gd[:, F:]
        nan = torch.isnan(want)
        assert torch.equal(torch.isnan(h), nan)
        assert torch.equal(h[~nan], want[~nan])


@pytest.mark.gpu
def test_swiglu_under_graph_capture(dev):
    """swiglu_quant captured in a HIP graph: three replays, with eager work
    and a synchronization between them, each equal to the eager call."""
    from shadowinfer_amd.execution import row_ops
    g = torch.Generator().manual_seed(7)
    gu = (torch.randn(64, 2 * 1024, generator=g) * 3).to(torch.bfloat16).to(dev)
    h0, q0, s0 = row_ops.swiglu_quant(gu, want_h=True)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        h, q, s = row_ops.swiglu_quant(gu, want_h=True)
    for _ in range(3):
        for t in (h, q, s):
            t.zero_()
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(h, h0) and torch.equal(q, q0) and torch.equal(s, s0)


@pytest.mark.gpu
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("M,V,scale", [(3, 1, 1.0), (5, 7, 1.0), (64, 32000, 0.05),
                                       (64, 32000, 4.0), (2, 50001, 1.0), (33, 1000, 0.02)])
def test_argmax_conf_kernel(dev, dtype, M, V, scale):
    """softmax(logits).max(-1) in the logits' dtype: tokens and confidences
    against torch's own softmax + max on the GPU and against the oracle, on
    every row the oracle does not flag; rows with NaN / +inf / only -inf."""
    from shadowinfer_amd.execution import argmax_confidence
    g = torch.Generator().manual_seed(M * V)
    logits = (torch.randn(M, V, generator=g) * scale).to(dtype)
    if V >= 7:
        logits[0, :] = 1.0                     # all tied: first index
        logits[1, 3] = logits[1, 5] = 1e4      # tie of two maxima
    tok, conf = argmax_confidence(logits.to(dev))
    assert conf.dtype == dtype
    rt, rc, amb = R.argmax_conf(to_np(logits), DT[dtype], return_ambiguous=True)
    assert amb.mean() < 0.05
    tc, tt = torch.softmax(logits.to(dev), dim=-1).max(dim=-1)
    for want_t, want_c in ((rt, rc), (tt.cpu().numpy(), to_np(tc))):
        np.testing.assert_array_equal(tok.cpu().numpy()[~amb], want_t[~amb])
        if dtype == torch.float32:
            np.testing.assert_allclose(to_np(conf), want_c, rtol=4 * R.SUM_REL_ERR)
        else:
            np.testing.assert_array_equal(to_np(conf)[~amb], want_c[~amb])
    bad = torch.zeros(3, 9)
    bad[0, 4] = bad[0, 6] = float("nan")
    bad[1, 2] = float("inf")
    bad[2, :] = float("-inf")
    t2, c2 = argmax_confidence(bad.to(dtype).to(dev))
    assert t2.tolist() == [0, 0, 0] and bool(torch.isnan(c2.float()).all())


def _reference_schedule(logits, masked, threshold):
    """block_decoding.py:144-165 as torch ops on the device (the reference's
    op sequence; its boolean-index assignment written as a loop over rows)."""
    probs = torch.softmax(logits, dim=-1)
    confidences, tokens = probs.max(dim=-1)
    above = masked & (confidences >= threshold)
    needs_fallback = masked.any(dim=1) & ~above.any(dim=1)
    fallback_positions = confidences.masked_fill(~masked, float("-inf")).argmax(dim=1)
    fallback_unmask = torch.zeros_like(above)
    for b in range(masked.shape[0]):
        if bool(needs_fallback[b]):
            fallback_unmask[b, fallback_positions[b]] = True
    unmask = above | fallback_unmask
    return unmask, tokens, confidences * (masked & ~unmask), needs_fallback


@pytest.mark.gpu
def test_schedule_round_matches_reference_rule(dev):
    from shadowinfer_amd.execution import schedule_round
    V = 16
    confs = [[0.95, 0.2, 0.91, 0.5], [0.3, 0.6, 0.6, 0.1], [0.99, 0.99, 0.2, 0.2]]
    toks = [[3, 4, 5, 6], [1, 2, 3, 4], [7, 8, 9, 10]]
    logits = torch.from_numpy(np.stack([np.stack([_conf_row(c, t, V) for c, t in zip(cr, tr)])
                                        for cr, tr in zip(confs, toks)]))
    masked = torch.tensor([[1, 1, 1, 1], [1, 1, 1, 0], [0, 0, 0, 0]], dtype=torch.bool)
    d = schedule_round(logits.to(dev), masked.to(dev), 0.9)
    np.testing.assert_array_equal(d.unmask.cpu().numpy(), [[1, 0, 1, 0], [0, 1, 0, 0], [0, 0, 0, 0]])
    np.testing.assert_array_equal(d.progress_fallback.cpu().numpy(), [False, True, False])
    np.testing.assert_array_equal(d.tokens.cpu().numpy(), toks)
    # random blocks, fp32 and bf16, against the reference's op sequence on the
    # GPU and the oracle's per-element rule (reference tests/test_block_decoding.py:363-384)
    for dtype in (torch.float32, torch.bfloat16):
        for b, w, v, sc in ((1, 1, 2, 1.0), (2, 5, 4, 1.0), (3, 8, 16, 1.0), (4, 64, 1000, 1.0),
                            (4, 256, 32000, 0.05), (2, 128, 64, 3.0)):
            g = torch.Generator().manual_seed(b * 100 + w * 7 + v)
            lg = (torch.randn(b, w, v, generator=g) * sc).to(dtype).to(dev)
            mk = (torch.rand(b, w, generator=g) < 0.6).to(dev)
            for thr in (0.9, 0.3, 0.2617):
                d = schedule_round(lg, mk, thr)
                ru, rt, rc, rf = _reference_schedule(lg, mk, thr)
                assert torch.equal(d.unmask, ru) and torch.equal(d.progress_fallback, rf)
                assert torch.equal(d.tokens[d.unmask], rt[d.unmask])
                if dtype == torch.float32:   # fp32 sums in another order: last bits
                    torch.testing.assert_close(d.confidences, rc, rtol=4 * R.SUM_REL_ERR, atol=0)
                else:
                    assert torch.equal(d.confidences, rc)
                _, conf = R.argmax_conf(to_np(lg), DT[dtype])
                ou, of = R.schedule(conf, mk.cpu().numpy(), thr, DT[dtype])
                np.testing.assert_array_equal(d.unmask.cpu().numpy(), ou)
                np.testing.assert_array_equal(d.progress_fallback.cpu().numpy(), of)
    with pytest.raises(ValueError):
        schedule_round(lg[0], mk, 0.9)
    with pytest.raises(ValueError):
        schedule_round(lg, mk[:, :1], 0.9)


@pytest.mark.gpu
def test_attention_token_major_layout(dev):
    from shadowinfer_amd.shadowkv import PackedKVCache, PrecisionPlan, packed_attention
    from helpers import kv_inputs, mixed_codes
    B, H, S, D = 2, 3, 80, 128
    k, v = kv_inputs(B, H, S, D, torch.bfloat16, seed=3)
    q, _ = kv_inputs(B, H, S, D, torch.bfloat16, seed=4)
    codes = mixed_codes(S, H, seed=3, probs=(1, 1, 1, 1), evicted=0.1)
    plan = PrecisionPlan.from_codes(torch.from_numpy(codes).to(dev))
    cache = PackedKVCache.pack(k.to(dev), v.to(dev), None, plan=plan)["packed_kv"]
    a = packed_attention(q.to(dev), cache, out_dtype=torch.bfloat16)
    t = packed_attention(q.to(dev), cache, out_dtype=torch.bfloat16, token_major=True)
    assert t.shape == (B, S, H, D)
    assert torch.equal(t, a.transpose(1, 2))


# ---------------------------------------------------------- whole model
SMALL = dict(num_hidden_layers=2, hidden_size=256, num_attention_heads=4, intermediate_size=512,
             vocab_size=512, mask_token_id=511)


def _model(dev, **over):
    from shadowinfer_amd.execution import DiffusionLlamaShape, PackedDiffusionLlama
    cfg = DiffusionLlamaShape(**{**SMALL, **over})
    return PackedDiffusionLlama(cfg, device=dev, seed=11)


def _plans(dev, S, H, L, seed=5):
    from shadowinfer_amd.shadowkv import PrecisionPlan
    from helpers import mixed_codes
    codes = [mixed_codes(S, H, seed=seed + i, probs=(1, 1, 2, 1), evicted=0.05) for i in range(L)]
    return codes, [PrecisionPlan.from_codes(torch.from_numpy(c).to(dev)) for c in codes]


@pytest.mark.gpu
@pytest.mark.parametrize("B,S", [(1, 96), (2, 64)])
def test_layers_stage_by_stage(dev, B, S):
    """Each stage from the GPU's own input to that stage (tests/stage_check.py)."""
    from shadowinfer_amd.execution import mask_tokens
    from stage_check import check_layer_stages, weights
    m = _model(dev)
    c = m.config
    H, D, Hd = c.num_attention_heads, c.head_dim, c.hidden_size
    codes, plans = _plans(dev, S, H, c.num_hidden_layers)
    tokens, _ = mask_tokens(B, S, 0.5, c, dev, seed=B)
    traces = {}
    logits, kv = m.forward_step(tokens, plans, traces=traces)
    cos, sin = (to_np(t) for t in m.rope_tables(S))
    dt = O.BF16
    for i in range(c.num_hidden_layers):
        assert kv[i] is traces[i]["cache"]
        check_layer_stages(traces[i], weights(m, i), codes[i], B, S, H, D, c.rms_norm_eps, cos, sin)
    fin = traces["final"]
    hn, amb = R.rmsnorm(to_np(fin["hidden"]).reshape(B * S, Hd), dt, to_np(m.norm),
                        c.rms_norm_eps, return_ambiguous=True)
    got = to_np(fin["hn"]).reshape(B * S, Hd)
    assert not ((got != hn).any(-1) & ~amb).any()
    lg = R.linear(got, dt, to_np(m.lm_head))
    assert rel_l2(f32(to_np(logits), dt).reshape(B * S, -1), f32(lg, dt)) <= 2e-3


@pytest.mark.gpu
def test_step_end_to_end(dev):
    """The whole step from the token ids, every stage from the reference's own
    previous stage: bf16 rounding differences compound over the layers, so the
    bound is relL2 <= 2e-2 on the logits (the int8 activations of the two
    chains may differ by one step where a bf16 value moved by one ulp)."""
    from shadowinfer_amd.execution import mask_tokens
    from stage_check import weights
    m = _model(dev)
    c = m.config
    B, S = 1, 64
    H, D, Hd = c.num_attention_heads, c.head_dim, c.hidden_size
    codes, plans = _plans(dev, S, H, c.num_hidden_layers, seed=9)
    tokens, _ = mask_tokens(B, S, 0.5, c, dev, seed=3)
    logits, _ = m.forward_step(tokens, plans)
    dt = O.BF16
    cos, sin = (to_np(t) for t in m.rope_tables(S))
    x = to_np(m.embed)[tokens.cpu().numpy().reshape(-1)]
    for i in range(c.num_hidden_layers):
        x = R.layer(x, dt, weights(m, i), codes[i], B, S, H, D, c.rms_norm_eps, cos, sin)["out"]
    lg = R.linear(R.rmsnorm(x, dt, to_np(m.norm), c.rms_norm_eps), dt, to_np(m.lm_head))
    assert rel_l2(f32(to_np(logits), dt).reshape(B * S, -1), f32(lg, dt)) <= 2e-2


@pytest.mark.gpu
def test_step_reuse_schedule_and_drift(dev):
    from shadowinfer_amd.execution import StepReuseConfig, StepReuseState, mask_tokens
    m = _model(dev, num_hidden_layers=3)
    c = m.config
    B, S = 1, 64
    _, plans = _plans(dev, S, c.num_attention_heads, c.num_hidden_layers)
    tokens, masked = mask_tokens(B, S, 0.5, c, dev, seed=1)
    state = StepReuseState()
    cfg = StepReuseConfig(enabled=True, threshold=float("inf"), warmup_steps=1,
                          reusable_layers={1})
    _, kv0 = m.forward_step(tokens, plans, 0, state, cfg)
    assert state.stats()["computed_layers"] == [0, 1, 2]
    rec = state.records[1]
    traces = {}
    tokens2 = tokens.clone()
    tokens2[0, :3] = 7
    _, kv1 = m.forward_step(tokens2, plans, 1, state, cfg, traces=traces)
    st = state.stats()
    assert st["reused_layers"] == [1] and st["computed_layers"] == [0, 2]
    assert st["reused_ratio"] == pytest.approx(1 / 3) and st["attention_reused"]
    assert kv1[1] is kv0[1] and kv1[0] is not kv0[0]
    # reused layer: hidden_out + (hidden - hidden_in), the two bf16 torch ops
    h_in = traces[0]["out"].view(B, S, -1)
    want = rec.hidden_out + (h_in - rec.hidden_in)
    assert torch.equal(traces[2]["x"].view(B, S, -1), want)
    # drift gate (reference step_reuse.py:71-95): the same input drifts 0 -> reuse
    state = StepReuseState()
    cfg = StepReuseConfig(enabled=True, threshold=0.05, warmup_steps=1)
    m.forward_step(tokens, plans, 0, state, cfg)
    m.forward_step(tokens, plans, 0, state, cfg)                 # warm-up step: no reuse
    assert state.stats()["reused_layers"] == []
    m.forward_step(tokens, plans, 1, state, cfg)
    assert state.stats()["reused_layers"] == [0, 1, 2]
    assert all(d == 0.0 for d in state.stats()["drifts"].values())
    other, _ = mask_tokens(B, S, 0.5, c, dev, seed=99)
    m.forward_step(other, plans, 2, state, cfg)
    assert state.stats()["computed_layers"] == [0, 1, 2]
    drifts = state.stats()["drifts"]
    assert all(d > 0.05 for d in drifts.values())
    with pytest.raises(ValueError):
        StepReuseConfig(threshold=-1.0)
    with pytest.raises(ValueError):
        StepReuseConfig(warmup_steps=-1)


@pytest.mark.gpu
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("n", [1, 7, 4096, 1 << 20, (1 << 20) + 13])
def test_reuse_kernels_match_the_torch_ops(dev, dtype, n):
    """The fused reuse output equals hidden_out + (hidden - hidden_in) in torch
    bit for bit; the drift equals the reference's
    float((hidden - hidden_in).norm() / hidden_in.norm()) in the dtype (up to
    the fp32 summation order of the two norms: one unit in the last place of
    the dtype, for fp32 a relative 1e-5); an all-zero hidden_in gives None."""
    from shadowinfer_amd.execution import StepReuseState
    from shadowinfer_amd.execution.step_reuse import LayerRecord
    g = torch.Generator().manual_seed(n)
    hin = torch.randn(n, generator=g).to(dtype).to(dev)
    h = (hin.float() + 0.05 * torch.randn(n, generator=g).to(dev)).to(dtype)
    hout = torch.randn(n, generator=g).to(dtype).to(dev)
    st = StepReuseState()
    rec = LayerRecord(hin, hout)
    got = st.reuse(0, rec, h)
    assert torch.equal(got, hout + (h - hin))
    d = st.relative_drift(rec, h)
    want = float((h - hin).norm() / hin.norm())
    if dtype == torch.float32:
        assert d == pytest.approx(want, rel=1e-5)
    else:
        assert abs(d - want) <= abs(float(torch.tensor(want, dtype=dtype).float()) * 2 ** -7)
    assert st.relative_drift(LayerRecord(torch.zeros_like(hin), hout), h) is None


@pytest.mark.gpu
def test_reuse_gate_with_infinite_threshold_keeps_the_reference_outcome(dev):
    """threshold=inf still computes the drift (execution/step_reuse.py:71-95):
    an all-zero recorded input drops the record and recomputes, a NaN drift
    refuses reuse, a finite one is logged and reused. skip_drift=True reuses
    every record of the right shape without reading the device."""
    from shadowinfer_amd.execution import StepReuseConfig, StepReuseState
    from shadowinfer_amd.execution.step_reuse import LayerRecord
    g = torch.Generator().manual_seed(5)
    h = torch.randn(2, 8, 64, generator=g).to(torch.bfloat16).to(dev)
    out = torch.randn(2, 8, 64, generator=g).to(torch.bfloat16).to(dev)
    inf = StepReuseConfig(enabled=True, threshold=float("inf"), warmup_steps=0)
    st = StepReuseState()
    st.records[0] = LayerRecord(torch.zeros_like(h), out)
    assert st.gate(0, h, 1, inf) is None and 0 not in st.records
    nan_h = h.clone()
    nan_h[0, 0, 0] = float("nan")
    st.records[0] = LayerRecord(h, out)
    assert st.gate(0, nan_h, 1, inf) is None and 0 in st.records
    assert math.isnan(st.stats()["drifts"][0])
    st.new_step()
    assert st.gate(0, h * 1.5, 1, inf) is st.records[0]
    assert st.stats()["drifts"][0] == pytest.approx(0.5, rel=2 ** -7)
    skip = StepReuseConfig(enabled=True, threshold=float("inf"), warmup_steps=0, skip_drift=True)
    st = StepReuseState()
    st.records[0] = LayerRecord(torch.zeros_like(h), out)
    assert st.gate(0, h, 1, skip) is st.records[0] and st.stats()["drifts"] == {}


@pytest.mark.gpu
def test_reuse_kernels_take_views_at_any_offset(dev):
    """A hidden state that is a view at an odd element offset (not 16-byte
    aligned) works like its contiguous copy in the drift and the reused output."""
    from shadowinfer_amd.execution import StepReuseState
    from shadowinfer_amd.execution.step_reuse import LayerRecord
    g = torch.Generator().manual_seed(6)
    base = torch.randn(3, 4104, generator=g).to(torch.bfloat16).to(dev)
    h, hin, hout = base[0, 1:4097], base[1, 3:4099], base[2, 5:4101]
    st = StepReuseState()
    rec = LayerRecord(hin, hout)
    got = st.reuse(0, rec, h)
    assert torch.equal(got, hout + (h - hin))
    assert st.relative_drift(rec, h) == st.relative_drift(LayerRecord(hin.clone(), hout), h.clone())


@pytest.mark.gpu
def test_denoise_loop_progress(dev):
    from shadowinfer_amd.execution import StepReuseConfig, StepReuseState, mask_tokens
    m = _model(dev)
    c = m.config
    B, S = 2, 64
    _, plans = _plans(dev, S, c.num_attention_heads, c.num_hidden_layers)
    tokens, masked = mask_tokens(B, S, 0.5, c, dev, seed=2)
    assert int(masked.sum()) == 64 and bool((tokens[masked] == c.mask_token_id).all())
    state = StepReuseState()
    cfg = StepReuseConfig(enabled=True, threshold=float("inf"), reusable_layers={1})
    before = masked.clone()
    for step in range(6):
        prev_masked = masked.clone()
        prev_tokens = tokens.clone()
        d, kv, _ = m.denoise_step(tokens, masked, plans, step, 0.9, state, cfg)
        assert bool((d.unmask <= prev_masked).all())
        assert bool(((prev_masked.sum(1) - masked.sum(1)) >= 1).all())
        assert torch.equal(tokens[d.unmask], d.tokens[d.unmask])
        assert torch.equal(tokens[~d.unmask], prev_tokens[~d.unmask])
        assert len(kv) == c.num_hidden_layers
    assert int(masked.sum()) <= int(before.sum()) - 12
    # generate: rounds, then the forced completion by the last logits' argmax
    tokens, masked = mask_tokens(B, S, 0.5, c, dev, seed=4)
    start_tokens, start_masked = tokens.clone(), masked.clone()
    seen = {}
    res = m.generate(tokens, masked, plans, 4, 0.9, StepReuseState(), cfg,
                     on_step=lambda st, d, kv, lg: seen.update(logits=lg, masked=masked.clone()))
    assert not bool(masked.any()) and bool(res["finite"])
    assert torch.equal(tokens[~start_masked], start_tokens[~start_masked])
    left = seen["masked"]
    assert torch.equal(res["forced"], left.sum(1))
    assert torch.equal(tokens[left], seen["logits"].argmax(-1)[left])
    assert torch.equal(res["unmasked_per_step"].sum(0) + res["forced"], start_masked.sum(1))


def test_shape_validation_without_gpu():
    from shadowinfer_amd.execution import DiffusionLlamaShape
    with pytest.raises(ValueError):
        DiffusionLlamaShape(hidden_size=4096, num_attention_heads=24)
    with pytest.raises(ValueError):
        DiffusionLlamaShape(mask_token_id=32000)
    assert DiffusionLlamaShape().head_dim == 128


@pytest.mark.gpu
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("B,S,H,D,group", [(1, 96, 4, 128, 16), (2, 67, 3, 64, 16),
                                           (1, 300, 2, 128, 32), (2, 33, 5, 64, 8),
                                           (1, 1, 1, 128, 16), (1, 2048, 32, 128, 16),
                                           (2, 1000, 32, 128, 16)])
def test_pack_projection_equals_rope_then_pack(dev, dtype, B, S, H, D, group):
    """PackedKVCache.pack_projection (K and V read from the q|k|v projection,
    K rotated in the pack kernel) writes the buckets and scales that
    rope_split followed by PackedKVCache.pack writes, bit for bit, for every
    precision including fp32 entries and evictions; rope_split with kv=False
    writes the same q."""
    from shadowinfer_amd.execution import row_ops
    from shadowinfer_amd.shadowkv import PackedKVCache, PrecisionPlan
    from helpers import mixed_codes
    g = torch.Generator().manual_seed(S * H + D)
    qkv = (torch.randn(B * S, 3 * H * D, generator=g) * 2).to(dtype).to(dev)
    qkv[:, H * D: H * D + D] *= 40  # large K rows of head 0: scales far from 1
    ang = torch.randn(S, D, generator=g) * 3
    cos, sin = ang.cos().to(dtype).to(dev), ang.sin().to(dtype).to(dev)
    codes = mixed_codes(S, H, seed=S + D, probs=(1, 1, 2, 2), sink=min(4, S), evicted=0.1)
    plan = PrecisionPlan.from_codes(torch.from_numpy(codes).to(dev))
    assert row_ops.rope_pack_supported(dtype, D, group)
    q_ref, k, v = row_ops.rope_split(qkv, cos, sin, B, S, H, D)
    ref = PackedKVCache.pack(k, v, None, group_size=group, plan=plan)["packed_kv"]
    q, none_k, none_v = row_ops.rope_split(qkv, cos, sin, B, S, H, D, kv=False)
    assert none_k is None and none_v is None and torch.equal(q, q_ref)
    got = PackedKVCache.pack_projection(qkv, cos, sin, B, S, H, D, group, plan)
    assert got.memory_bytes() == ref.memory_bytes()
    rb, gb = ref._buckets, got._buckets
    assert rb.keys() == gb.keys()
    for name in rb:
        for part in ("k", "v", "scale_k", "scale_v"):
            if rb[name][part] is None:
                assert gb[name][part] is None
            else:
                assert torch.equal(gb[name][part].view(torch.uint8),
                                   rb[name][part].view(torch.uint8)), (name, part)
    uk, uv = got.unpack()
    rk, rv = ref.unpack()
    assert torch.equal(uk, rk) and torch.equal(uv, rv)


def test_rope_pack_support_rule():
    from shadowinfer_amd.execution import row_ops
    assert row_ops.rope_pack_supported(torch.bfloat16, 128, 16)
    assert row_ops.rope_pack_supported(torch.float16, 64, 8)
    assert row_ops.rope_pack_supported(torch.bfloat16, 128, 12)  # 12 does not divide 128: one group of D
    assert not row_ops.rope_pack_supported(torch.float32, 128, 16)
    assert not row_ops.rope_pack_supported(torch.bfloat16, 96, 16)
    assert not row_ops.rope_pack_supported(torch.bfloat16, 128, 4)
    assert row_ops.rope_pack_supported(torch.bfloat16, 64, 24)  # 24 does not divide 64: one group of D
