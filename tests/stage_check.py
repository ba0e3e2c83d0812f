"""Stage-by-stage check of one decoder layer of the packed-KV / INT8-FFN step
(models/diffusion_llama.py:407-424) against the oracle, each stage computed
from the GPU's own input to that stage.

* bit-exact: RoPE and the head split, the packed KV (buckets, scales, bytes),
  the residual adds, the int8 activations and scales, both INT8 GEMM outputs;
  SwiGLU also bit-exact to torch's own F.silu(gate) * up on the GPU;
* bit-exact on every row (element) the oracle does not flag: both RMSNorms,
  SwiGLU against the oracle (its exp is correctly rounded);
* relL2 <= 2e-3: the bf16 library GEMMs (q|k|v, o; fp32 accumulation) and the
  fused dequant + attention (fp16 tiles) against double precision.

``rows`` picks the rows (token positions) for the stages whose oracle costs a
GEMM (the library GEMMs, attention queries, the INT8 GEMMs); every other stage
is checked on all rows.
"""

from __future__ import annotations

from typing import Dict, Optional

import numpy as np
import torch
import torch.nn.functional as F

from helpers import assert_cache_equal, to_np
from oracle import denoise_ref as R
from oracle import oracle as O


def f32(x, dt):
    return O.to_f32(np.ascontiguousarray(x), dt)


def rel_l2(a, b):
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    return float(np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-30))


def weights(model, i) -> Dict[str, np.ndarray]:
    L = model.layers[i]
    return {"ln1": to_np(L.ln1), "w_qkv": to_np(L.w_qkv), "w_o": to_np(L.w_o), "ln2": to_np(L.ln2),
            "gu_q": L.gu_q.cpu().numpy(), "gu_s": L.gu_s.cpu().numpy(),
            "dn_q": L.dn_q.cpu().numpy(), "dn_s": L.dn_s.cpu().numpy()}


def _rows_equal(got, want, amb, what):
    assert amb.mean() < 0.05, (what, float(amb.mean()))
    bad = (got != want).reshape(got.shape[0], -1).any(-1) & ~amb
    assert not bad.any(), (what, np.flatnonzero(bad)[:8])


def check_layer_stages(trace: dict, W: Dict[str, np.ndarray], codes: np.ndarray, B: int, S: int,
                       H: int, D: int, eps: float, cos: np.ndarray, sin: np.ndarray,
                       rows: Optional[np.ndarray] = None, group: int = 16) -> None:
    dt = O.BF16
    T = B * S
    Hd = H * D
    rows = np.arange(T) if rows is None else np.asarray(rows)
    g = {k: (to_np(v) if isinstance(v, torch.Tensor) else v) for k, v in trace.items()}

    xn, amb = R.rmsnorm(g["x"], dt, W["ln1"], eps, return_ambiguous=True)
    _rows_equal(g["xn"], xn, amb, "ln1")
    assert rel_l2(f32(g["qkv"][rows], dt), f32(R.linear(g["xn"][rows], dt, W["w_qkv"]), dt)) <= 2e-3
    rq, rk, rv = R.rope_split(g["qkv"], dt, cos, sin, B, S, H, D)
    np.testing.assert_array_equal(g["q"], rq)
    np.testing.assert_array_equal(g["k"], rk)
    np.testing.assert_array_equal(g["v"], rv)
    # the packed KV: bit-exact to the oracle pack of the GPU's own K/V
    ref_cache = O.kv_pack(g["k"], g["v"], dt, codes, group)
    assert_cache_equal(trace["cache"], ref_cache)
    kf, vf = O.kv_unpack(ref_cache)
    qs = np.ascontiguousarray(f32(g["q"], dt).reshape(B, H, S, D)[:, :, np.unique(rows % S)])
    att = O.attention(qs, kf, vf).transpose(0, 2, 1, 3)                  # [B, s, H, D]
    got = f32(g["attn"], dt).reshape(B, S, H, D)[:, np.unique(rows % S)]
    assert rel_l2(got, att) <= 2e-3
    o = R.linear(g["attn"].reshape(T, Hd)[rows], dt, W["w_o"])
    assert rel_l2(f32(g["o"].reshape(T, Hd)[rows], dt), f32(o, dt)) <= 2e-3
    np.testing.assert_array_equal(g["x1"], R.add(g["x"], g["o"].reshape(T, Hd), dt))
    y2, amb = R.rmsnorm(g["x1"], dt, W["ln2"], eps, return_ambiguous=True)
    _rows_equal(g["y2"], y2, amb, "ln2")
    qx, sx = O.int8_act_quant(g["y2"], dt)
    np.testing.assert_array_equal(g["qx"], qx)
    np.testing.assert_array_equal(g["sx"], sx)
    gu = O.int8_epilogue(O.gemm_i8(g["qx"][rows], W["gu_q"].T), g["sx"][rows], W["gu_s"], None, dt)
    np.testing.assert_array_equal(g["gu"][rows], gu)
    F_ = g["gu"].shape[1] // 2
    gu_dev = trace["gu"]
    assert torch.equal(trace["h"], F.silu(gu_dev[:, :F_]) * gu_dev[:, F_:])
    h, amb = R.swiglu(g["gu"][rows], dt, return_ambiguous=True)
    assert amb.mean() < 0.01
    np.testing.assert_array_equal(g["h"][rows][~amb], h[~amb])
    qh, sh = O.int8_act_quant(g["h"], dt)
    np.testing.assert_array_equal(g["qh"], qh)
    np.testing.assert_array_equal(g["sh"], sh)
    ffn = O.int8_epilogue(O.gemm_i8(g["qh"][rows], W["dn_q"].T), g["sh"][rows], W["dn_s"], None, dt)
    np.testing.assert_array_equal(g["ffn"][rows], ffn)
    np.testing.assert_array_equal(g["out"].reshape(T, -1), R.add(g["x1"], g["ffn"], dt))
