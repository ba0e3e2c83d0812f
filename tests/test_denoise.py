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
    # bf16: the fp32 result rounded once (RNE) to bf16
    xb = O.from_f32(x, O.BF16)
    yb = R.rmsnorm(xb, O.BF16, O.from_f32(w, O.BF16), 1e-5)
    xf = O.to_f32(xb, O.BF16).astype(np.float64)
    wf = O.to_f32(O.from_f32(w, O.BF16), O.BF16).astype(np.float64)
    want = torch.from_numpy((xf / np.sqrt((xf ** 2).mean(-1, keepdims=True) + 1e-5) * wf)
                            .astype(np.float32)).to(torch.bfloat16)
    np.testing.assert_array_equal(yb, to_np(want))


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


def test_swiglu_ref_matches_library_silu():
    rng = np.random.default_rng(2)
    g = (rng.standard_normal((4, 40)) * 4).astype(np.float32)
    u = rng.standard_normal((4, 40)).astype(np.float32)
    gb, ub = O.from_f32(g, O.BF16), O.from_f32(u, O.BF16)
    h = R.swiglu(np.concatenate([gb, ub], 1), O.BF16)
    gf = O.to_f32(gb, O.BF16).astype(np.float64)
    sg = O.to_f32(O.from_f32((gf * expit(gf)).astype(np.float32), O.BF16), O.BF16).astype(np.float64)
    want = O.from_f32((sg * O.to_f32(ub, O.BF16)).astype(np.float32), O.BF16)
    assert ulp_diff(h, want).max() <= 1
    z = R.swiglu(np.zeros((1, 16), np.float32), O.F32)
    np.testing.assert_array_equal(z, 0.0)


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
    unmask, fb = R.schedule(conf, masked, 0.9)
    # row 0: both above 0.9; row 1: fallback, tie 0.6/0.6 -> smaller index;
    # row 2: nothing masked
    np.testing.assert_array_equal(unmask, [[1, 0, 1, 0], [0, 1, 0, 0], [0, 0, 0, 0]])
    np.testing.assert_array_equal(fb, [False, True, False])


# ------------------------------------------------------------------ GPU
def _need_lib():
    from shadowinfer_amd import _native
    _native.load()


@pytest.mark.gpu
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("M,K", [(1, 8), (37, 256), (64, 4096), (5, 11008), (3, 16384)])
def test_rmsnorm_kernel(dev, dtype, M, K):
    from shadowinfer_amd.execution import row_ops
    g = torch.Generator().manual_seed(M * 7 + K)
    x = (torch.randn(M, K, generator=g) * 3).to(dtype)
    w = (torch.rand(K, generator=g) + 0.5).to(dtype)
    y, q, s = row_ops.rmsnorm(x.to(dev), w.to(dev), 1e-5, want_y=True, want_q=True)
    dt = DT[dtype]
    assert_row_kernel_close(to_np(y), R.rmsnorm(to_np(x), dt, to_np(w), 1e-5), dtype)
    qr, sr = O.int8_act_quant(to_np(y), dt)      # fused quantization of the kernel's own y
    np.testing.assert_array_equal(to_np(q), qr)
    np.testing.assert_array_equal(to_np(s), sr)
    _, q2, s2 = row_ops.rmsnorm(x.to(dev), w.to(dev), 1e-5, want_y=False, want_q=True)
    assert torch.equal(q2, q) and torch.equal(s2, s)


@pytest.mark.gpu
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("B,S,H,D", [(1, 7, 3, 64), (2, 33, 4, 128), (1, 256, 32, 128)])
def test_rope_kernel(dev, dtype, B, S, H, D):
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
    for got, want in ((q, rq), (k, rk)):
        assert_row_kernel_close(to_np(got), want, dtype)
    np.testing.assert_array_equal(to_np(v), rv)


@pytest.mark.gpu
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("M,F", [(1, 8), (19, 512), (64, 11008), (2, 16384)])
def test_swiglu_kernel(dev, dtype, M, F):
    from shadowinfer_amd.execution import row_ops
    g = torch.Generator().manual_seed(M + F)
    gu = (torch.randn(M, 2 * F, generator=g) * 3).to(dtype)
    h, q, s = row_ops.swiglu_quant(gu.to(dev), want_h=True)
    dt = DT[dtype]
    # two roundings (silu, then the product): within 2 units in the last place
    assert_row_kernel_close(to_np(h), R.swiglu(to_np(gu), dt), dtype, max_ulp=2)
    qr, sr = O.int8_act_quant(to_np(h), dt)
    np.testing.assert_array_equal(to_np(q), qr)
    np.testing.assert_array_equal(to_np(s), sr)
    _, q2, s2 = row_ops.swiglu_quant(gu.to(dev), want_h=False)
    assert torch.equal(q2, q) and torch.equal(s2, s)


@pytest.mark.gpu
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("M,V", [(3, 1), (5, 7), (64, 32000), (2, 50001)])
def test_argmax_conf_kernel(dev, dtype, M, V):
    from shadowinfer_amd.execution import argmax_confidence
    g = torch.Generator().manual_seed(M * V)
    logits = (torch.randn(M, V, generator=g) * 4).to(dtype)
    if V >= 7:
        logits[0, :] = 1.0                     # all tied: first index
        logits[1, 3] = logits[1, 5] = 1e4      # tie of two maxima
    tok, conf = argmax_confidence(logits.to(dev))
    rt, rc = R.argmax_conf(to_np(logits), DT[dtype])
    np.testing.assert_array_equal(tok.cpu().numpy(), rt)
    np.testing.assert_allclose(conf.cpu().numpy(), rc, rtol=1e-5)
    nan = torch.zeros(1, 9)
    nan[0, 4] = float("nan")
    nan[0, 6] = float("nan")
    t2, c2 = argmax_confidence(nan.to(dev))
    assert int(t2[0]) == 4 and math.isnan(float(c2[0]))


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
    # random blocks against the per-element rule (reference tests/test_block_decoding.py:363-384)
    for b, w, v in ((1, 1, 2), (2, 5, 4), (3, 8, 16), (4, 64, 1000)):
        g = torch.Generator().manual_seed(b * 100 + w * 7 + v)
        lg = torch.randn(b, w, v, generator=g)
        mk = torch.rand(b, w, generator=g) < 0.6
        for thr in (0.9, 0.3):
            d = schedule_round(lg.to(dev), mk.to(dev), thr)
            _, conf = R.argmax_conf(lg.numpy(), O.F32)
            ru, rf = R.schedule(conf, mk.numpy(), thr)
            np.testing.assert_array_equal(d.unmask.cpu().numpy(), ru)
            np.testing.assert_array_equal(d.progress_fallback.cpu().numpy(), rf)
            still = (mk & ~d.unmask.cpu()).numpy()
            np.testing.assert_allclose(d.confidences.cpu().numpy()[still], conf[still], rtol=1e-5)
            assert not d.confidences.cpu().numpy()[~still].any()
    with pytest.raises(ValueError):
        schedule_round(lg.to(dev)[0], mk.to(dev), 0.9)
    with pytest.raises(ValueError):
        schedule_round(lg.to(dev), mk.to(dev)[:, :1], 0.9)


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


def _weights(model, i):
    L = model.layers[i]
    return {"ln1": to_np(L.ln1), "w_qkv": to_np(L.w_qkv), "w_o": to_np(L.w_o), "ln2": to_np(L.ln2),
            "gu_q": L.gu_q.cpu().numpy(), "gu_s": L.gu_s.cpu().numpy(),
            "dn_q": L.dn_q.cpu().numpy(), "dn_s": L.dn_s.cpu().numpy()}


@pytest.mark.gpu
@pytest.mark.parametrize("B,S", [(1, 96), (2, 64)])
def test_layers_stage_by_stage(dev, B, S):
    """Each stage from the GPU's own input to that stage."""
    from shadowinfer_amd.execution import mask_tokens
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
        t = {k: v for k, v in traces[i].items()}
        W = _weights(m, i)
        g = {k: (to_np(v) if isinstance(v, torch.Tensor) else v) for k, v in t.items()}
        d = ulp_diff(g["xn"], R.rmsnorm(g["x"], dt, W["ln1"], c.rms_norm_eps))
        assert d.max() <= 1 and (d > 0).mean() <= 1e-2
        # bf16 library GEMM (fp32 accumulation, one rounding): relL2 <= 2e-3
        assert rel_l2(f32(g["qkv"], dt), f32(R.linear(g["xn"], dt, W["w_qkv"]), dt)) <= 2e-3
        rq, rk, rv = R.rope_split(g["qkv"], dt, cos, sin, B, S, H, D)
        for got, want in ((g["q"], rq), (g["k"], rk)):
            assert ulp_diff(got, want).max() <= 1
        np.testing.assert_array_equal(g["v"], rv)
        # the packed KV: bit-exact to the oracle pack of the GPU's own K/V
        ref_cache = O.kv_pack(g["k"], g["v"], dt, codes[i], 16)
        assert_cache_equal(t["cache"], ref_cache)
        assert kv[i] is t["cache"]
        kf, vf = O.kv_unpack(ref_cache)
        att = O.attention(f32(g["q"], dt), kf, vf).transpose(0, 2, 1, 3)
        # fused dequant + attention (fp16 P/V tiles) against double precision: relL2 <= 2e-3
        assert rel_l2(f32(g["attn"], dt).reshape(B, S, H, D), att) <= 2e-3
        x1 = f32(g["x"], dt).astype(np.float64) + \
            f32(g["attn"], dt).reshape(B * S, Hd).astype(np.float64) @ f32(W["w_o"], dt).T.astype(np.float64)
        assert rel_l2(f32(g["x1"], dt), x1) <= 2e-3
        d = ulp_diff(g["y2"], R.rmsnorm(g["x1"], dt, W["ln2"], c.rms_norm_eps))
        assert d.max() <= 1
        qx, sx = O.int8_act_quant(g["y2"], dt)
        np.testing.assert_array_equal(g["qx"], qx)
        np.testing.assert_array_equal(g["sx"], sx)
        gu = O.int8_epilogue(O.gemm_i8(g["qx"], W["gu_q"].T), g["sx"], W["gu_s"], None, dt)
        np.testing.assert_array_equal(g["gu"], gu)
        assert ulp_diff(g["h"], R.swiglu(g["gu"], dt)).max() <= 2
        qh, sh = O.int8_act_quant(g["h"], dt)
        np.testing.assert_array_equal(g["qh"], qh)
        np.testing.assert_array_equal(g["sh"], sh)
        ffn = O.int8_epilogue(O.gemm_i8(g["qh"], W["dn_q"].T), g["sh"], W["dn_s"], None, dt)
        np.testing.assert_array_equal(g["ffn"], ffn)
        out = O.from_f32(f32(g["x1"], dt) + f32(g["ffn"], dt), dt)
        np.testing.assert_array_equal(g["out"], out)
    fin = traces["final"]
    hn = R.rmsnorm(to_np(fin["hidden"]).reshape(B * S, Hd), dt, to_np(m.norm), c.rms_norm_eps)
    assert ulp_diff(to_np(fin["hn"]).reshape(B * S, Hd), hn).max() <= 1
    lg = R.linear(to_np(fin["hn"]).reshape(B * S, Hd), dt, to_np(m.lm_head))
    assert rel_l2(f32(to_np(logits), dt).reshape(B * S, -1), f32(lg, dt)) <= 2e-3


@pytest.mark.gpu
def test_step_end_to_end(dev):
    """The whole step from the token ids, every stage from the reference's own
    previous stage: bf16 rounding differences compound over the layers, so the
    bound is relL2 <= 2e-2 on the logits (the int8 activations of the two
    chains may differ by one step where a bf16 value moved by one ulp)."""
    from shadowinfer_amd.execution import mask_tokens
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
        x = R.layer(x, dt, _weights(m, i), codes[i], B, S, H, D, c.rms_norm_eps, cos, sin)["out"]
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
    entry = state.entries[1]
    traces = {}
    tokens2 = tokens.clone()
    tokens2[0, :3] = 7
    _, kv1 = m.forward_step(tokens2, plans, 1, state, cfg, traces=traces)
    st = state.stats()
    assert st["reused_layers"] == [1] and st["computed_layers"] == [0, 2]
    assert st["reused_ratio"] == pytest.approx(1 / 3)
    assert kv1[1] is kv0[1] and kv1[0] is not kv0[0]
    # reused layer: hidden_out + (hidden - hidden_in), bf16 elementwise ops
    h_in = traces[0]["out"].view(B, S, -1)
    want = entry.hidden_out + (h_in - entry.hidden_in)
    assert torch.equal(traces[2]["x"].view(B, S, -1), want)
    # drift gate (reference step_reuse.py:82-95): the same input drifts 0 -> reuse
    state = StepReuseState()
    cfg = StepReuseConfig(enabled=True, threshold=0.05, warmup_steps=1)
    m.forward_step(tokens, plans, 0, state, cfg)
    m.forward_step(tokens, plans, 0, state, cfg)                 # warm-up step: no reuse
    assert state.stats()["reused_layers"] == []
    m.forward_step(tokens, plans, 1, state, cfg)
    assert state.stats()["reused_layers"] == [0, 1, 2]
    assert all(d == 0.0 for d in state.last_drifts.values())
    other, _ = mask_tokens(B, S, 0.5, c, dev, seed=99)
    m.forward_step(other, plans, 2, state, cfg)
    assert state.stats()["computed_layers"] == [0, 1, 2]
    assert all(d > 0.05 for d in state.last_drifts.values())
    with pytest.raises(ValueError):
        StepReuseConfig(threshold=-1.0)


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
        d, kv = m.denoise_step(tokens, masked, plans, step, 0.9, state, cfg)
        assert bool((d.unmask <= prev_masked).all())
        assert bool(((prev_masked.sum(1) - masked.sum(1)) >= 1).all())
        assert torch.equal(tokens[d.unmask], d.tokens[d.unmask])
        assert torch.equal(tokens[~d.unmask], prev_tokens[~d.unmask])
        assert len(kv) == c.num_hidden_layers
    assert int(masked.sum()) <= int(before.sum()) - 12


def test_shape_validation_without_gpu():
    from shadowinfer_amd.execution import DiffusionLlamaShape
    with pytest.raises(ValueError):
        DiffusionLlamaShape(hidden_size=4096, num_attention_heads=24)
    with pytest.raises(ValueError):
        DiffusionLlamaShape(mask_token_id=32000)
    assert DiffusionLlamaShape().head_dim == 128
