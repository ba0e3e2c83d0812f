"""Cross-step block reuse on the packed data plane (the drift-gated reuse of
shadowinfer/execution/step_reuse.py:18-134 as DiffusionTransformerBlock uses
it, models/simple_diffusion_llm.py:99-120).

A computed layer leaves a :class:`LayerRecord`: the hidden state it read, the
one it wrote and its packed KV cache (kept by reference; the step never
writes into them afterwards). On a later step the layer is skipped when the
new input is close to the recorded one, and its output becomes
``hidden_out + (hidden - hidden_in)``; its KV is the recorded cache, so a
reused layer neither packs nor attends.

The gate keeps the reference's decision: no reuse when disabled or before
``warmup_steps``; a record of another shape, or with an all-zero input, is
dropped and the layer recomputed; otherwise reuse iff
``||hidden - hidden_in|| / ||hidden_in|| <= threshold`` evaluated as torch
evaluates it in the hidden dtype (each norm an fp32 sum of squares, square
root, rounded to the dtype; the quotient rounded to the dtype).

How it runs here:

* both sums of squares come from one HIP reduction over the two tensors
  (``si_reuse_drift``); the host reads the two floats and finishes the ratio,
  so a gated layer costs one small device read;
* the reused output is one HIP pass (``si_reuse_apply``) instead of a
  subtraction and an addition over the whole hidden state;
* ``threshold=inf`` keeps the reference's outcome: the drift is still
  computed and logged, a record with an all-zero input is dropped and a NaN
  drift refuses reuse. ``skip_drift=True`` (no reference counterpart) accepts
  every record of the right shape without computing the drift: no device
  read at all, so a denoising loop stays asynchronous; ``reusable_layers``
  limits reuse to a fixed set of layers (e.g. every other block).
"""

from __future__ import annotations

import math
from dataclasses import dataclass, field
from typing import Any, Dict, FrozenSet, List, Optional

import numpy as np
import torch

from .. import _native


@dataclass(frozen=True)
class StepReuseConfig:
    """The reference's knobs (``enabled``, ``threshold``, ``warmup_steps``)
    plus ``reusable_layers`` (None: every layer may be reused) and
    ``skip_drift`` (reuse every record of the right shape without computing
    the drift; the gate then neither drops all-zero records nor refuses NaN
    drifts, and ``stats()['drifts']`` stays empty)."""

    enabled: bool = False
    threshold: float = 0.1
    warmup_steps: int = 1
    reusable_layers: Optional[FrozenSet[int]] = None
    skip_drift: bool = False

    def __post_init__(self) -> None:
        if self.threshold < 0:
            raise ValueError(f"step reuse threshold must be >= 0, got {self.threshold}")
        if self.warmup_steps < 0:
            raise ValueError(f"step reuse warmup_steps must be >= 0, got {self.warmup_steps}")
        if self.reusable_layers is not None:
            object.__setattr__(self, "reusable_layers",
                               frozenset(int(i) for i in self.reusable_layers))

    def allows(self, layer: int, step_id: int) -> bool:
        return (self.enabled and step_id >= self.warmup_steps
                and (self.reusable_layers is None or layer in self.reusable_layers))


@dataclass
class LayerRecord:
    """What one computation of a layer leaves for the next steps."""

    hidden_in: torch.Tensor
    hidden_out: torch.Tensor
    packed_kv: Any = None


@dataclass
class _StepLog:
    reused: List[int] = field(default_factory=list)
    computed: List[int] = field(default_factory=list)
    drifts: Dict[int, float] = field(default_factory=dict)


def _round_to(x: np.float32, dtype: torch.dtype) -> np.float32:
    """An fp32 value rounded to ``dtype`` (round to nearest even)."""
    return np.float32(torch.tensor(float(x), dtype=torch.float32).to(dtype).float().item())


def _aligned(t: torch.Tensor) -> torch.Tensor:
    """``t`` contiguous at a 16-byte aligned address (the reuse kernels read
    16 bytes per lane); a view at an odd offset is copied."""
    c = t.contiguous()
    return c if c.data_ptr() % 16 == 0 else c.clone(memory_format=torch.contiguous_format)


class StepReuseState:
    """Per-layer records across denoising steps and the log of the last step."""

    def __init__(self) -> None:
        self.records: Dict[int, LayerRecord] = {}
        self._log = _StepLog()
        self._scratch: Dict[torch.device, torch.Tensor] = {}

    def clear(self) -> None:
        self.records.clear()
        self._log = _StepLog()

    def new_step(self) -> None:
        self._log = _StepLog()

    # ------------------------------------------------------------- the gate
    def relative_drift(self, record: LayerRecord, hidden: torch.Tensor) -> Optional[float]:
        """``||hidden - hidden_in|| / ||hidden_in||`` in the hidden dtype's
        arithmetic; None when ``hidden_in`` is all zeros (a NaN drift, from
        non-finite states, never passes the gate)."""
        _native.require_device(hidden, "StepReuseState.relative_drift")
        a = _aligned(hidden)
        b = _aligned(record.hidden_in)
        dev = a.device
        ws_bytes = _native.size_query("si_reuse_drift_workspace_bytes", a.numel())
        buf = self._scratch.get(dev)
        if buf is None or buf.numel() < ws_bytes + 8:
            buf = torch.empty(ws_bytes + 8, dtype=torch.uint8, device=dev)
            self._scratch[dev] = buf
        sums = buf[ws_bytes:ws_bytes + 8].view(torch.float32)
        _native.call("si_reuse_drift", a.data_ptr(), b.data_ptr(), _native.dtype_code(a.dtype),
                     a.numel(), sums.data_ptr(), buf.data_ptr(), ws_bytes, _native.stream(dev))
        s_diff, s_in = sums.cpu().numpy()
        dt = a.dtype
        # torch: each norm is the fp32 square root of the fp32 sum, rounded to
        # the dtype; the quotient is taken in fp32 and rounded to the dtype
        with np.errstate(invalid="ignore", divide="ignore"):
            denom = _round_to(np.sqrt(s_in), dt)
            if denom <= 0.0:
                return None
            return float(_round_to(_round_to(np.sqrt(s_diff), dt) / denom, dt))

    def gate(self, layer: int, hidden: torch.Tensor, step_id: int,
             config: StepReuseConfig) -> Optional[LayerRecord]:
        """The record to reuse for ``layer`` this step, or None (compute it)."""
        if not config.allows(layer, step_id):
            return None
        record = self.records.get(layer)
        if record is None or record.hidden_in.shape != hidden.shape:
            self.records.pop(layer, None)
            return None
        if config.skip_drift:
            return record
        drift = self.relative_drift(record, hidden)
        if drift is None:
            self.records.pop(layer, None)
            return None
        self._log.drifts[layer] = drift
        return record if drift <= config.threshold else None

    # ------------------------------------------------------ reuse and record
    def reuse(self, layer: int, record: LayerRecord, hidden: torch.Tensor) -> torch.Tensor:
        """The reused layer's output ``hidden_out + (hidden - hidden_in)``."""
        _native.require_device(hidden, "StepReuseState.reuse")
        h = _aligned(hidden)
        hin = _aligned(record.hidden_in)
        hout = _aligned(record.hidden_out)
        out = torch.empty_like(h)
        _native.call("si_reuse_apply", h.data_ptr(), hin.data_ptr(), hout.data_ptr(),
                     _native.dtype_code(h.dtype), h.numel(), out.data_ptr(),
                     _native.stream(h.device))
        self._log.reused.append(layer)
        return out.view(hidden.shape)

    def keep(self, layer: int, hidden_in: torch.Tensor, hidden_out: torch.Tensor,
             packed_kv: Any = None) -> None:
        """Record a computed layer (the tensors are held, not copied)."""
        self.records[layer] = LayerRecord(hidden_in.detach(), hidden_out.detach(), packed_kv)
        self._log.computed.append(layer)

    # --------------------------------------------------------------- stats
    def stats(self) -> Dict[str, Any]:
        """The last step's outcome, under the keys of the reference's
        StepReuseState.stats (execution/step_reuse.py:113-125)."""
        reused = sorted(self._log.reused)
        computed = sorted(self._log.computed)
        n = len(reused) + len(computed)
        return {"reused_layers": reused, "computed_layers": computed,
                "reused_ratio": len(reused) / n if n else 0.0,
                "drifts": dict(self._log.drifts), "attention_reused": bool(reused)}
