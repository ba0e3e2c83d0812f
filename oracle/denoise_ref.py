"""CPU reference of one denoising step of a Llama-shaped diffusion LM on the
quantized data plane (packed KV + INT8 FFN).

TEST INFRASTRUCTURE ONLY: this module is the checker for the denoising-step
kernels. Only ``tests/`` may import it; the product package never does.

Floating-point parts are restated in float64 numpy and rounded once to the
model dtype, the arithmetic the HIP row kernels state; the quantized parts
(KV pack/unpack, INT8Linear) come from ``oracle.py``. Array conventions follow
``oracle.py`` (bf16/fp16 values as uint16 bit patterns plus a dtype code).

* ``rmsnorm``       DiffusionLlamaRMSNorm (models/diffusion_llama.py:311-321)
* ``rope_split``    q/k rotation and head split (diffusion_llama.py:362-373)
* ``swiglu``        silu(gate) * up, each op rounded (diffusion_llama.py:332-333)
* ``argmax_conf``   per-position argmax / max probability (block_decoding.py:148-151)
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
    """float64 -> fp32 (RNE) -> dt (RNE): the kernels' fp32 result rounded to dt."""
    return O.from_f32(x64.astype(np.float32), dt)


def rmsnorm(x: np.ndarray, dt: int, w: np.ndarray, eps: float) -> np.ndarray:
    """y = T(x / sqrt(mean(x^2) + eps) * w) over the last axis
    (diffusion_llama.py:319-321), float64 arithmetic, one rounding."""
    xf = _f64(x, dt)
    wf = _f64(w, dt)
    inv = 1.0 / np.sqrt((xf * xf).mean(axis=-1, keepdims=True) + eps)
    return _round(xf * inv * wf, dt)


def rope_split(qkv: np.ndarray, dt: int, cos: np.ndarray, sin: np.ndarray, B: int, S: int,
               H: int, D: int) -> Tuple[np.ndarray, np.ndarray, np.ndarray]:
    """qkv [B*S, 3*H*D] -> q, k, v [B, H, S, D]; q, k = x*cos + rotate_half(x)*sin
    (diffusion_llama.py:288-292, 372-373) with cos/sin [S, D] in dt."""
    x = _f64(qkv, dt).reshape(B, S, 3, H, D).transpose(2, 0, 3, 1, 4)  # [3, B, H, S, D]
    c = _f64(cos, dt)[None, None]
    s = _f64(sin, dt)[None, None]

    def rot(t):
        half = D // 2
        return np.concatenate([-t[..., half:], t[..., :half]], axis=-1)

    q = _round(x[0] * c + rot(x[0]) * s, dt)
    k = _round(x[1] * c + rot(x[1]) * s, dt)
    v = np.ascontiguousarray(qkv.reshape(B, S, 3, H, D)[:, :, 2].transpose(0, 2, 1, 3))
    return q, k, v


def swiglu(gu: np.ndarray, dt: int) -> np.ndarray:
    """gu [M, 2F] (gate | up) -> T(T(silu(g)) * u) (diffusion_llama.py:333)."""
    F2 = gu.shape[-1]
    g = _f64(gu[..., : F2 // 2], dt)
    u = _f64(gu[..., F2 // 2:], dt)
    sg = _f64(_round(g / (1.0 + np.exp(-g)), dt), dt)
    return _round(sg * u, dt)


def argmax_conf(logits: np.ndarray, dt: int) -> Tuple[np.ndarray, np.ndarray]:
    """Rows of logits -> (first argmax, 1 / sum exp(l - max)) in float64."""
    l = _f64(logits, dt)
    tok = l.argmax(axis=-1)
    m = l.max(axis=-1, keepdims=True)
    conf = 1.0 / np.exp(l - m).sum(axis=-1)
    return tok.astype(np.int64), conf


def schedule(conf: np.ndarray, masked: np.ndarray, threshold: float
             ) -> Tuple[np.ndarray, np.ndarray]:
    """Per batch row: unmask every masked position with conf >= threshold;
    with none, the single most confident masked position, smallest index on
    ties (block_decoding.py:148-158). Returns (unmask, fallback)."""
    B, W = masked.shape
    unmask = np.zeros((B, W), dtype=bool)
    fallback = np.zeros(B, dtype=bool)
    for b in range(B):
        pos = [w for w in range(W) if masked[b, w]]
        if not pos:
            continue
        above = [w for w in pos if conf[b, w] >= threshold]
        if above:
            unmask[b, above] = True
        else:
            best = max(pos, key=lambda w: (conf[b, w], -w))
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
    x1 = _f64(x, dt) + _f64(r["attn"].reshape(B * S, Hd), dt) @ _f64(W["w_o"], dt).T
    r["x1"] = _round(x1, dt)
    r["y2"] = rmsnorm(r["x1"], dt, W["ln2"], eps)
    r["qx"], r["sx"] = O.int8_act_quant(r["y2"], dt)
    r["gu"] = O.int8_epilogue(O.gemm_i8(r["qx"], W["gu_q"].T), r["sx"], W["gu_s"], None, dt)
    r["h"] = swiglu(r["gu"], dt)
    r["qh"], r["sh"] = O.int8_act_quant(r["h"], dt)
    r["ffn"] = O.int8_epilogue(O.gemm_i8(r["qh"], W["dn_q"].T), r["sh"], W["dn_s"], None, dt)
    r["out"] = _round(_f64(r["x1"], dt) + _f64(r["ffn"], dt), dt)
    r["cache"] = cache
    return r
