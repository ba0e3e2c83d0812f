"""The reference's hot path as CPU torch op chains, for timing on the host.

TEST INFRASTRUCTURE ONLY: bench.py's cpu_baseline leg runs these functions to
measure what the reference's own CPU path costs on the same workload; the
product package never imports them, and parity is checked against oracle.py.

Each function performs the reference's torch operations in the reference's
order, with the Python bookkeeping that goes with them:

* ``plan_from_codes``  the grouping of PrecisionPlan.from_codes
  (shadowinfer/shadowkv/precision_plan.py:132-151): per code, ``nonzero`` of
  the flat codes, token/head split, Python index lists, ``h*S+t`` indices;
* ``pack_with_plan``   PackedKVCache._do_pack_with_plan
  (shadowinfer/shadowkv/packed_kv_cache.py:222-365) with the Quantizer op
  chains (shadowinfer/utils/quantization.py:120-178) and the int4 row packing
  (packed_kv_cache.py:367-388), including the per-entry byte offsets of the
  int4 bucket;
* ``unpack``           PackedKVCache.unpack and _dequantize_int4_bucket
  (packed_kv_cache.py:535-577, 636-656);
* ``int8_linear_forward``  INT8Linear.forward (shadowinfer/ffn_optimizer/
  int8_linear.py:88-115) with CPU ``torch._int_mm``; ``int8_weight`` is
  from_linear's quantization (:65-82).
"""

from __future__ import annotations

from typing import Dict, List, Tuple

import torch

NAMES = ("fp32", "fp16", "int8", "int4")


def plan_from_codes(codes: torch.Tensor) -> Tuple[Dict[str, list], Dict[str, torch.Tensor]]:
    S, H = codes.shape
    flat = codes.reshape(-1).to(torch.int64)
    groups: Dict[str, list] = {}
    flat_idx: Dict[str, torch.Tensor] = {}
    for code, name in enumerate(NAMES):
        sel = (flat == code).nonzero(as_tuple=False).reshape(-1)
        t = torch.div(sel, H, rounding_mode="floor")
        h = torch.remainder(sel, H)
        groups[name] = list(zip(t.tolist(), h.tolist()))
        flat_idx[name] = h * S + t
    return groups, flat_idx


def _q_int8(x: torch.Tensor):
    s = x.abs().max(dim=-1, keepdim=True)[0] / 127.0
    s = torch.where(s == 0, torch.ones_like(s), s)
    return torch.round(x / s).clamp(-128, 127).to(torch.int8), s


def _q_int4(x: torch.Tensor, g: int):
    r = x.reshape(*x.shape[:-1], x.shape[-1] // g, g)
    s = r.abs().max(dim=-1, keepdim=True)[0] / 7.0
    s = torch.where(s == 0, torch.ones_like(s), s)
    return torch.round(r / s).clamp(-8, 7).to(torch.int8), s


def _int4_rows(q: torch.Tensor) -> torch.Tensor:
    rows = q.reshape(q.shape[0], -1)
    u = (rows + 8).to(torch.uint8)
    if u.shape[1] % 2:
        u = torch.cat([u, torch.zeros(u.shape[0], 1, dtype=torch.uint8)], dim=1)
    return (u[:, 0::2] << 4) | (u[:, 1::2] & 0x0F)


def pack_with_plan(k: torch.Tensor, v: torch.Tensor, groups: Dict[str, list],
                   flat_idx: Dict[str, torch.Tensor], group_size: int = 16) -> Dict[str, dict]:
    B, H, S, D = k.shape
    kf = k.reshape(B, H * S, D)
    vf = v.reshape(B, H * S, D)
    out: Dict[str, dict] = {}
    for name in NAMES:
        entries = groups[name]
        if not entries:
            continue
        idx = flat_idx[name]
        ks = kf.index_select(1, idx).permute(1, 0, 2)
        vs = vf.index_select(1, idx).permute(1, 0, 2)
        d: dict = {"indices": list(entries)}
        if name in ("fp32", "fp16"):
            dt = torch.float32 if name == "fp32" else torch.float16
            d["k"], d["v"] = ks.to(dt), vs.to(dt)
        elif name == "int8":
            d["k"], d["scale_k"] = _q_int8(ks)
            d["v"], d["scale_v"] = _q_int8(vs)
        else:
            g = group_size if D % group_size == 0 else D
            qk, sk = _q_int4(ks, g)
            qv, sv = _q_int4(vs, g)
            rk, rv = _int4_rows(qk), _int4_rows(qv)
            rb = rk.shape[1]
            d["k"], d["v"] = rk.reshape(-1), rv.reshape(-1)
            d["scale_k"] = sk.reshape(-1, D // g, 1)
            d["scale_v"] = sv.reshape(-1, D // g, 1)
            d["byte_offsets"] = [(i * rb, (i + 1) * rb, i * rb, (i + 1) * rb)
                                 for i in range(len(entries))]
            d["group_size"], d["num_groups"] = g, D // g
        out[name] = d
    return out


def unpack(packed: Dict[str, dict], B: int, H: int, S: int, D: int
           ) -> Tuple[torch.Tensor, torch.Tensor]:
    ko = torch.zeros(B, H, S, D, dtype=torch.float32)
    vo = torch.zeros_like(ko)
    for name, d in packed.items():
        entries = d["indices"]
        heads = torch.tensor([h for _, h in entries], dtype=torch.long)
        toks = torch.tensor([t for t, _ in entries], dtype=torch.long)
        n = len(entries)
        for key, o in (("k", ko), ("v", vo)):
            if name in ("fp32", "fp16"):
                vals = d[key].float()
            elif name == "int8":
                vals = d[key].float() * d["scale_" + key]
            else:
                rows = d[key].reshape(n, -1)
                inter = torch.stack([(rows >> 4) & 0x0F, rows & 0x0F], dim=-1).reshape(n, -1)
                codes = (inter[:, : B * D].to(torch.int16) - 8).to(torch.int8)
                g, G = d["group_size"], d["num_groups"]
                vals = (codes.reshape(n, B, G, g).float()
                        * d["scale_" + key].reshape(n, B, G, 1)).reshape(n, B, D)
            o[:, heads, toks, :] = vals.permute(1, 0, 2)
    return ko, vo


def int8_weight(w: torch.Tensor) -> Tuple[torch.Tensor, torch.Tensor]:
    """[N, K] fp32 -> (qweight [K, N] int8, scale [N] fp32)."""
    w = w.to(torch.float32)
    s = (w.abs().amax(dim=1) / 127.0).clamp_min(1e-8)
    q = torch.round(w / s.unsqueeze(1)).clamp(-127, 127).to(torch.int8)
    return q.transpose(0, 1).contiguous(), s.contiguous()


def int8_linear_forward(x: torch.Tensor, qweight: torch.Tensor, scale: torch.Tensor,
                        bias: torch.Tensor = None) -> torch.Tensor:
    flat = x.reshape(-1, qweight.shape[0])
    xf = flat.to(torch.float32)
    sx = (xf.abs().amax(dim=1) / 127.0).clamp_min(1e-8)
    qx = torch.round(xf / sx.unsqueeze(1)).clamp(-127, 127).to(torch.int8)
    acc = torch._int_mm(qx, qweight)
    out = acc.to(torch.float32) * (sx.unsqueeze(1) * scale.unsqueeze(0))
    if bias is not None:
        out = out + bias.unsqueeze(0)
    return out.to(x.dtype).reshape(*x.shape[:-1], qweight.shape[1])
