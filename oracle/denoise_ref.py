"""CPU reference of one denoising step of a Llama-shaped diffusion LM on the
quantized data plane (packed KV + INT8 FFN).

TEST INFRASTRUCTURE ONLY: this module is the checker for the denoising-step
kernels. Only ``tests/`` may import it; the product package never does.

Floating-point parts restate the reference's torch op chains in the model
dtype: every elementwise op is an fp32 operation rounded to the dtype, emulated
in float64 (exact for sums and products of two dtype values, correctly rounded
for quotients and square roots). Reductions (RMSNorm's mean, softmax's sum)
are taken exactly and rounded once; where the device's summation order or its
expf could round differently, the functions can flag the rows or elements
("ambiguous") instead of guessing. The quantized parts (KV pack/unpack,
INT8Linear) come from ``oracle.py``. Array conventions follow
``oracle.py`` (bf16/fp16 values as uint16 bit patterns plus a dtype code).

* ``rmsnorm``       DiffusionLlamaRMSNorm (models/diffusion_llama.py:311-321)
* ``rope_split``    q/k rotation and head split (diffusion_llama.py:362-373)
* ``swiglu``        silu(gate) * up, each op rounded (diffusion_llama.py:332-333)
* ``add``           the residual adds (diffusion_llama.py:421-423)
* ``argmax_conf``   softmax(logits).max(-1) in the logits' dtype (block_decoding.py:146-147)
* ``schedule``      per-element unmasking rule (block_decoding.py:118-158)
* ``layer``         one decoder layer over packed KV (diffusion_llama.py:407-424)
"""

from __future__ import annotations

from typing import Dict, Tuple

import numpy as np

from . import oracle as O


def _f64(x: np.ndarray, dt: int) -> np.ndarray:
    return O.to_f32(x, dt).astype(np.float64)


def _round(x64: np.ndarray, dt: int) -> np.ndarray:
    """float64 -> fp32 (RNE) -> dt (RNE): an fp32 operation's result rounded to
    dt. Exact for the sums, differences and products of two dt values (exact in
    float64); for a quotient or square root the float64 result rounded to fp32
    is the correctly rounded fp32 result (53 >= 2 * 24 + 2)."""
    return O.from_f32(x64.astype(np.float32), dt)


def _op(x64: np.ndarray, dt: int) -> np.ndarray:
    """One torch elementwise op in dtype dt: fp32 result rounded to dt, as float64."""
    return _f64(_round(x64, dt), dt)


# The GPU row kernels sum a row of K values per thread in runs of at most 64
# and combine 256 partial sums in a tree: 64 + 8 roundings, relative error
# below 72 * 2^-24 of the sum of |terms|. Results are "ambiguous" where a
# rounding to dt lies that close to a midpoint.
SUM_REL_ERR = 72.0 * 2.0 ** -24


def rmsnorm(x: np.ndarray, dt: int, w: np.ndarray, eps: float, return_ambiguous: bool = False):
    """DiffusionLlamaRMSNorm.forward (diffusion_llama.py:319-321) as its torch
    op chain in dt: ``x / sqrt(mean(x.pow(2)) + eps) * w``, each op rounded to
    dt: var = T(fp32(sum T(x^2)) * f), r = T(sqrt(T(var + eps))),
    y = T(T(x / r) * w), with f = float(M) / float(M * K), torch's mean factor.
    The fp32 sum is taken exactly; with ``return_ambiguous`` a bool per row
    also says whether a sum within SUM_REL_ERR could round var differently."""
    xf = _f64(x, dt)
    K = xf.shape[-1]
    M = xf.size // K if K else 0
    f = np.float64(np.float32(M) / np.float32(M * K)) if M else 1.0
    sq = _op(xf * xf, dt)
    ss = sq.sum(axis=-1, keepdims=True)

    def var_of(total):
        return _op(_f64(_round(total, O.F32), O.F32) * f, dt)

    var = var_of(ss)
    eps32 = np.float64(np.float32(eps))
    r = _op(np.sqrt(_op(var + eps32, dt)), dt)
    y = _round(_op(xf / r, dt) * _f64(w, dt), dt)
    if not return_ambiguous:
        return y
    amb = ((var_of(ss * (1 - SUM_REL_ERR)) != var) | (var_of(ss * (1 + SUM_REL_ERR)) != var))
    return y, amb.reshape(amb.shape[:-1])


def add(a: np.ndarray, b: np.ndarray, dt: int) -> np.ndarray:
    """``a + b`` in dt (the residual adds, diffusion_llama.py:421-423)."""
    return _round(_f64(a, dt) + _f64(b, dt), dt)


def rope_split(qkv: np.ndarray, dt: int, cos: np.ndarray, sin: np.ndarray, B: int, S: int,
               H: int, D: int) -> Tuple[np.ndarray, np.ndarray, np.ndarray]:
    """qkv [B*S, 3*H*D] -> q, k, v [B, H, S, D]; q, k = x*cos + rotate_half(x)*sin
    as torch evaluates it in dt (diffusion_llama.py:288-292, 372-373): both
    products rounded to dt, then their sum; cos/sin [S, D] in dt."""
    x = _f64(qkv, dt).reshape(B, S, 3, H, D).transpose(2, 0, 3, 1, 4)  # [3, B, H, S, D]
    c = _f64(cos, dt)[None, None]
    s = _f64(sin, dt)[None, None]

    def rot(t):
        half = D // 2
        return np.concatenate([-t[..., half:], t[..., :half]], axis=-1)

    q = _round(_op(x[0] * c, dt) + _op(rot(x[0]) * s, dt), dt)
    k = _round(_op(x[1] * c, dt) + _op(rot(x[1]) * s, dt), dt)
    v = np.ascontiguousarray(qkv.reshape(B, S, 3, H, D)[:, :, 2].transpose(0, 2, 1, 3))
    return q, k, v


def _silu32(g: np.ndarray) -> np.ndarray:
    """torch's silu in fp32 on float64 inputs: g / (1 + exp(-g)) with every op
    an fp32 operation and exp correctly rounded to fp32."""
    with np.errstate(over="ignore", invalid="ignore"):
        e = np.exp(-g).astype(np.float32).astype(np.float64)
        d = (1.0 + e).astype(np.float32).astype(np.float64)
        return (g / d).astype(np.float32).astype(np.float64)


def swiglu(gu: np.ndarray, dt: int, return_ambiguous: bool = False):
    """gu [M, 2F] (gate | up) -> T(T(silu(g)) * u) (diffusion_llama.py:333),
    silu as torch's fp32 formula. The device's expf may differ from the
    correctly rounded exp by an ulp; with ``return_ambiguous`` a bool per
    element also says whether the fp32 silu lies within 4 fp32 ulps of a dt
    rounding midpoint (only there can that ulp change the result)."""
    F2 = gu.shape[-1]
    g = _f64(gu[..., : F2 // 2], dt)
    u = _f64(gu[..., F2 // 2:], dt)
    s32 = _silu32(g)
    h = _round(_f64(_round(s32, dt), dt) * u, dt)
    if not return_ambiguous:
        return h
    with np.errstate(invalid="ignore"):
        ulp = np.abs(np.spacing(s32.astype(np.float32)).astype(np.float64))
        lo = _f64(_round(s32 - 4 * ulp, dt), dt)
        hi = _f64(_round(s32 + 4 * ulp, dt), dt)
    # an exact zero (g = 0, or exp overflowing for g << 0) has no neighbour to
    # round to; -0 and +0 compare equal above
    return h, (lo != hi) & (s32 != 0)


def argmax_conf(logits: np.ndarray, dt: int, sum_rel_err: float = SUM_REL_ERR,
                return_ambiguous: bool = False):
    """Rows of logits -> (token, confidence) of ``softmax(logits).max(-1)`` in
    dt (block_decoding.py:146-147): torch's softmax gives
    p_v = T(expf(l_v - m) / s) with m the row max and s = sum_v expf(l_v - m)
    in fp32, so confidence = T(1 / s) and token = the first v with
    p_v == confidence. A row with a NaN or +inf, or only -inf, gives NaN and
    token 0. Returns (int64 tokens, confidences as dt bit patterns / fp32).

    s is the exactly rounded fp32 sum of correctly rounded exps; with
    ``return_ambiguous`` a bool per row also says whether a sum within
    ``sum_rel_err`` of it, or an exp an ulp away, could change the result (for
    fp32 logits: the token; the fp32 confidence itself then carries that
    relative error)."""
    lf = _f64(logits, dt)
    V = lf.shape[-1]
    rows = lf.reshape(-1, V)
    tok = np.zeros(rows.shape[0], np.int64)
    conf = np.full(rows.shape[0], np.nan, np.float64)
    amb = np.zeros(rows.shape[0], bool)
    for i, r in enumerate(rows):
        if np.isnan(r).any() or np.isposinf(r).any() or np.isneginf(r).all():
            continue
        m = r.max()
        d = (r - m).astype(np.float32).astype(np.float64)           # fp32 difference
        e = np.exp(d).astype(np.float32).astype(np.float64)         # fp32 exp
        s = np.float64(np.float32(e.sum()))

        def decide(s_, e_):
            c_ = float(_f64(_round(np.array([1.0 / s_]), dt), dt)[0])
            p_ = _f64(_round(e_ / s_, dt), dt)
            return int(np.flatnonzero(p_ == c_)[0]), c_

        tok[i], conf[i] = decide(s, e)
        if return_ambiguous:
            ulp = np.abs(np.spacing(e.astype(np.float32)).astype(np.float64))
            for s_ in (s * (1 - sum_rel_err), s * (1 + sum_rel_err)):
                s_ = np.float64(np.float32(s_))
                for e_ in (e - ulp, e + ulp):
                    e_ = np.where(d == 0, 1.0, e_)   # exp(0) = 1 exactly
                    t_, c_ = decide(s_, e_)
                    # an fp32 confidence moves with any change of the sum:
                    # there only the token decision counts
                    if t_ != tok[i] or (dt != O.F32 and c_ != conf[i]):
                        amb[i] = True
    shape = logits.shape[:-1]
    conf_dt = _round(conf, dt).reshape(shape)
    if return_ambiguous:
        return tok.reshape(shape), conf_dt, amb.reshape(shape)
    return tok.reshape(shape), conf_dt


def schedule(conf: np.ndarray, masked: np.ndarray, threshold: float, dt: int
             ) -> Tuple[np.ndarray, np.ndarray]:
    """Per batch row (block_decoding.py:148-158): unmask every masked position
    whose confidence (dt values) reaches the threshold rounded to dt (torch
    compares a dt tensor with a Python float in dt); with none, the single most
    confident masked position, the smallest index on ties. Returns (unmask,
    fallback)."""
    c = _f64(conf, dt)
    thr = _f64(_round(np.array([threshold], np.float64), dt), dt)[0]
    B, W = masked.shape
    unmask = np.zeros((B, W), dtype=bool)
    fallback = np.zeros(B, dtype=bool)
    for b in range(B):
        pos = [w for w in range(W) if masked[b, w]]
        if not pos:
            continue
        above = [w for w in pos if c[b, w] >= thr]
        if above:
            unmask[b, above] = True
        else:
            best = pos[0]
            for w in pos[1:]:
                if c[b, w] > c[b, best] or (np.isnan(c[b, w]) and not np.isnan(c[b, best])):
                    best = w
            unmask[b, best] = True
            fallback[b] = True
    return unmask, fallback


def linear(x: np.ndarray, dt: int, w: np.ndarray) -> np.ndarray:
    """x [M, K] @ w[N, K]^T in float64, rounded to dt (a bf16 library GEMM
    with fp32 accumulation rounds the same value once)."""
    return _round(_f64(x, dt) @ _f64(w, dt).T, dt)


def layer(x: np.ndarray, dt: int, W: Dict[str, np.ndarray], codes: np.ndarray, B: int, S: int,
          H: int, D: int, eps: float, cos: np.ndarray, sin: np.ndarray, group: int = 16
          ) -> Dict[str, np.ndarray]:
    """One decoder layer on the packed data plane from the layer input ``x``
    [B*S, hidden] (diffusion_llama.py:415-424): every intermediate, each from
    the previous one computed here. ``W``: ln1, w_qkv [3hid, hid], w_o, ln2,
    gu_q [2F, hid] int8, gu_s [2F] fp32, dn_q, dn_s."""
    r: Dict[str, np.ndarray] = {}
    r["xn"] = rmsnorm(x, dt, W["ln1"], eps)
    r["qkv"] = linear(r["xn"], dt, W["w_qkv"])
    r["q"], r["k"], r["v"] = rope_split(r["qkv"], dt, cos, sin, B, S, H, D)
    cache = O.kv_pack(r["k"], r["v"], dt, codes, group)
    kf, vf = O.kv_unpack(cache)
    att = O.attention(O.to_f32(r["q"], dt), kf, vf)                      # [B, H, S, D]
    r["attn"] = O.from_f32(np.ascontiguousarray(att.transpose(0, 2, 1, 3)).astype(np.float32), dt)
    Hd = H * D
    r["o"] = linear(r["attn"].reshape(B * S, Hd), dt, W["w_o"])
    r["x1"] = add(x, r["o"], dt)
    r["y2"] = rmsnorm(r["x1"], dt, W["ln2"], eps)
    r["qx"], r["sx"] = O.int8_act_quant(r["y2"], dt)
    r["gu"] = O.int8_epilogue(O.gemm_i8(r["qx"], W["gu_q"].T), r["sx"], W["gu_s"], None, dt)
    r["h"] = swiglu(r["gu"], dt)
    r["qh"], r["sh"] = O.int8_act_quant(r["h"], dt)
    r["ffn"] = O.int8_epilogue(O.gemm_i8(r["qh"], W["dn_q"].T), r["sh"], W["dn_s"], None, dt)
    r["out"] = add(r["x1"], r["ffn"], dt)
    r["cache"] = cache
    return r
