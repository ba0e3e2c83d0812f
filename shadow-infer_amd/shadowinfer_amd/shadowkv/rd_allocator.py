"""Rate-distortion KV precision admission with the reference API
(shadowinfer/shadowkv/rd_allocator.py).

``kv_sensitivity`` and ``admit_codes`` run as HIP kernels (``si_kv_sensitivity``,
``si_admit_codes``): the admission ranks eligible token-heads by ascending
``importance * sensitivity`` (stable on the token-major index) and cuts the
ranking where the bytes saved cover the excess over the budget, exactly as
the reference's argsort + cumsum + searchsorted formulation
(rd_allocator.py:190-318), but with a weighted radix select on the device
instead of a sort. ``admit_budget`` keeps the dict interface
(rd_allocator.py:66-170) on top of the same kernels.

Inputs must live on a HIP device (``importance`` and ``sensitivity`` may be
anywhere: they are copied to the codes' device as fp32, the reference's
``.float()``).
"""

from __future__ import annotations

from typing import Dict, Optional, Set, Tuple

import torch

from .. import _native
from .precision_plan import CODE_PRECISIONS as _PLAN_CODE_PRECISIONS
from .precision_plan import PRECISION_CODES

EVICTED = "evicted"
DOWNGRADE_LADDER = {"fp32": "fp16", "fp16": "int8", "int8": "int4"}
CODE_PRECISIONS = dict(_PLAN_CODE_PRECISIONS)
PRECISION_CODE_DOWNGRADE = {0: 1, 1: 2, 2: 3}
EVICTED_CODE = 4


def entry_bytes(precision: str, batch: int, head_dim: int, group_size: int = 16) -> float:
    """Stored bytes of one token-head, K + V including scales (rd_allocator.py:26-44).

    Matches ``PackedKVCache.pack``: int4 uses ``group_size`` when it divides
    ``head_dim``, otherwise one group over the whole head dim.
    """
    p = precision.lower() if isinstance(precision, str) else precision
    if p == EVICTED:
        return 0.0
    if p == "int4":
        group = group_size if group_size > 0 and head_dim % group_size == 0 else head_dim
        per_tensor = batch * head_dim / 2.0 + batch * (head_dim // group) * 4
    elif p == "int8":
        per_tensor = batch * head_dim + batch * 4
    elif p == "fp32":
        per_tensor = batch * head_dim * 4
    else:
        per_tensor = batch * head_dim * 2
    return per_tensor * 2.0


def _code_costs(batch: int, head_dim: int, group_size: int) -> "ctypes.Array":
    import ctypes
    arr = (ctypes.c_int64 * 5)()
    for code in range(5):
        arr[code] = int(entry_bytes(CODE_PRECISIONS[code], batch, head_dim, group_size=group_size))
    return arr


def kv_sensitivity(k: torch.Tensor, v: torch.Tensor) -> torch.Tensor:
    """``(|k|max^2 + |v|max^2) / 2`` over batch and head_dim, ``[seq, heads]``
    in the input dtype (rd_allocator.py:47-61); each operation rounds to the
    input dtype as torch's does."""
    if k.shape != v.shape:
        raise ValueError("k and v must have identical shapes")
    if k.dim() != 4:
        raise ValueError(f"k must be [batch, heads, seq, head_dim], got {tuple(k.shape)}")
    if k.dtype != v.dtype:
        raise ValueError(f"k and v dtypes differ ({k.dtype} vs {v.dtype})")
    _native.require_device(k, "kv_sensitivity")
    if v.device != k.device:
        raise ValueError("k and v live on different devices")
    dt = _native.dtype_code(k.dtype)
    B, H, S, D = k.shape
    kc, vc = k.detach().contiguous(), v.detach().contiguous()
    out = torch.empty(S, H, dtype=k.dtype, device=k.device)
    _native.call("si_kv_sensitivity", kc.data_ptr(), vc.data_ptr(), dt, B, H, S, D,
                 out.data_ptr(), _native.stream(k.device))
    return out


def _window(t: torch.Tensor, S: int, H: int, device: torch.device) -> torch.Tensor:
    return t.detach().to(device=device, dtype=torch.float32)[:S, :H].contiguous()


def _admit(codes: torch.Tensor, importance: torch.Tensor, sensitivity: Optional[torch.Tensor],
           budget_bytes: Optional[int], batch: int, head_dim: int, sink_tokens: int,
           rd_allocation: bool, allow_eviction: bool, protected_mask: Optional[torch.Tensor],
           group_size: int) -> Tuple[torch.Tensor, int, int]:
    """Runs si_admit_codes; ``budget_bytes`` None means no budget (any int,
    negative included, is applied as given)."""
    dev = codes.device
    S, H = int(codes.shape[0]), int(codes.shape[1])
    src = codes.detach().to(torch.int8).contiguous()
    out = torch.empty_like(src)
    imp = _window(importance, S, H, dev) if importance.dim() == 2 else None
    if imp is None or tuple(imp.shape) != (S, H):
        raise ValueError(
            f"importance must cover the codes' [seq, heads] = [{S}, {H}], "
            f"got shape {tuple(importance.shape)}")
    sens = None
    if rd_allocation and sensitivity is not None and sensitivity.dim() == 2:
        sens = _window(sensitivity, S, H, dev)
        if sens.shape != imp.shape:
            sens = None  # the reference substitutes ones (rd_allocator.py:247-248)
    prot = None
    if protected_mask is not None:
        prot = protected_mask.detach().to(device=dev, dtype=torch.bool)[:S, :H]
        if tuple(prot.shape) != (S, H):
            raise ValueError(f"protected_mask must cover [{S}, {H}], got {tuple(protected_mask.shape)}")
        prot = prot.contiguous().view(torch.uint8)
    n = S * H
    ws_bytes = _native.size_query("si_admit_workspace_bytes", n)
    ws = torch.empty(ws_bytes + 256, dtype=torch.uint8, device=dev)
    base = (-ws.data_ptr()) % 256
    result = torch.empty(3, dtype=torch.int64, device=dev)
    use_budget = budget_bytes is not None
    _native.call("si_admit_codes", src.data_ptr(), out.data_ptr(), S, H, imp.data_ptr(),
                 _native.ptr(sens), _native.ptr(prot), int(sink_tokens),
                 int(budget_bytes) if use_budget else 0, 1 if use_budget else 0,
                 1 if allow_eviction else 0, _code_costs(batch, head_dim, group_size),
                 result.data_ptr(), ws.data_ptr() + base, ws_bytes, _native.stream(dev))
    predicted, evicted, bad = (int(x) for x in result.tolist())
    if bad:
        raise ValueError("codes must hold precision codes 0..4")
    return out, predicted, evicted


def predict_codes_bytes(codes: torch.Tensor, batch: int, head_dim: int, group_size: int = 16) -> int:
    """Bytes of dense ``int8 [seq, heads]`` codes (rd_allocator.py:173-188)."""
    _native.require_device(codes, "predict_codes_bytes")
    flat = codes.detach().reshape(1, -1)
    ones = torch.ones(flat.shape, dtype=torch.float32, device=codes.device)
    _, predicted, _ = _admit(flat, ones, None, None, batch, head_dim, 0, False, False, None,
                             group_size)
    return predicted


def admit_codes(
    codes: torch.Tensor,
    importance: torch.Tensor,
    sensitivity: torch.Tensor,
    budget_bytes: int,
    batch: int,
    head_dim: int,
    sink_tokens: int = 0,
    rd_allocation: bool = True,
    allow_eviction: bool = False,
    protected_mask: Optional[torch.Tensor] = None,
    group_size: int = 16,
) -> Tuple[torch.Tensor, int, int]:
    """Fit dense ``int8 [seq, heads]`` codes into ``budget_bytes``
    (rd_allocator.py:190-318). Returns ``(codes_out, predicted_bytes,
    evicted_count)``; the input is never mutated. Sink tokens and
    ``protected_mask`` entries are never touched."""
    if codes.dim() != 2:
        raise ValueError(f"codes must be 2-D [seq, heads], got shape {tuple(codes.shape)}")
    _native.require_device(codes, "admit_codes")
    budget = None if budget_bytes is None or budget_bytes < 0 else int(budget_bytes)
    return _admit(codes, importance, sensitivity, budget, batch, head_dim, sink_tokens,
                  rd_allocation, allow_eviction, protected_mask, group_size)


def admit_budget(
    importance: torch.Tensor,
    sensitivity: torch.Tensor,
    precision_map: Dict[int, Dict[int, str]],
    budget_bytes: int,
    batch: int,
    head_dim: int,
    sink_tokens: int = 0,
    rd_allocation: bool = True,
    allow_eviction: bool = False,
    protected: Optional[Set[Tuple[int, int]]] = None,
    group_size: int = 16,
    device: Optional[torch.device] = None,
) -> Tuple[Dict[int, Dict[int, str]], int, int]:
    """Dict form of the admission (rd_allocator.py:66-170), returning
    ``(map, predicted_bytes, evicted_count)``.

    The window ``[seq, heads]`` the reference ranks is turned into codes
    (missing entries rank as fp16, as the reference's ``get(h, "fp16")``)
    and admitted on the device. The reference counts bytes only for entries
    present in the map, while the codes also count the missing ones, so the
    budget is shifted by that constant difference; the ladder steps and
    eviction savings are the same in both forms. Entries the admission does
    not change keep their place (or absence) in the map. ``device`` picks the
    HIP device (default: importance's device if it is one, else cuda).
    """
    result: Dict[int, Dict[int, str]] = {
        int(token_idx): dict(head_map) for token_idx, head_map in precision_map.items()
    }

    def total(m):
        return int(sum(entry_bytes(p, batch, head_dim, group_size=group_size)
                       for head_map in m.values() for p in head_map.values()))

    if budget_bytes is None or budget_bytes < 0:
        return result, total(result), 0
    seq_len = min(int(importance.shape[0]), max(result.keys(), default=0) + 1)
    num_heads = min(
        int(importance.shape[1]) if importance.dim() > 1 else 1,
        max((len(m) for m in result.values()), default=0),
    )
    if seq_len <= 0 or num_heads <= 0:
        return result, total(result), 0
    if device is None:
        device = importance.device if importance.device.type == "cuda" else torch.device("cuda")
    codes = torch.empty(seq_len, num_heads, dtype=torch.int8)
    for t in range(seq_len):
        head_map = result.get(t, {})
        for h in range(num_heads):
            name = head_map.get(h)
            if name is None:
                codes[t, h] = PRECISION_CODES["fp16"]
            else:
                key = name.lower() if isinstance(name, str) else name
                if key not in PRECISION_CODES:
                    raise ValueError(f"Unsupported precision: {name}")
                codes[t, h] = PRECISION_CODES[key]
    costs = [int(entry_bytes(CODE_PRECISIONS[c], batch, head_dim, group_size=group_size))
             for c in range(5)]
    # The reference's running byte count starts at the map's total, the codes'
    # at the window's total (missing entries as fp16); the ladder and eviction
    # steps change both by the same amounts, so the two differ by a constant.
    codes_total = int(sum(costs[int(c)] for c in codes.reshape(-1).tolist()))
    offset = codes_total - total(result)
    prot_mask = None
    if protected:
        prot_mask = torch.zeros(seq_len, num_heads, dtype=torch.bool)
        for t, h in protected:
            if 0 <= t < seq_len and 0 <= h < num_heads:
                prot_mask[t, h] = True
    imp = importance.detach().float()[:seq_len, :num_heads]
    sens = sensitivity.detach().float()[:seq_len, :num_heads]
    if sens.shape != imp.shape:
        sens = torch.ones_like(imp)
    out, predicted, evicted = _admit(codes.to(device), imp, sens, int(budget_bytes) + offset,
                                     batch, head_dim, sink_tokens, rd_allocation,
                                     allow_eviction,
                                     None if prot_mask is None else prot_mask.to(device),
                                     group_size)
    new = out.to("cpu")
    changed = (new != codes).nonzero().tolist()
    for t, h in changed:
        result.setdefault(t, {})[h] = CODE_PRECISIONS[int(new[t, h])]
    return result, predicted - offset, evicted
