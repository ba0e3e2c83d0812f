"""Cross-step block reuse for diffusion denoising
(shadowinfer/execution/step_reuse.py:18-134).

Same API and gate as the reference: per layer, the input and output hidden
states of the last full computation are kept; on a later step a layer is
skipped when the relative-L2 drift of its input stays within ``threshold``,
and its output becomes ``hidden_out + (hidden - hidden_in)``. In the packed
pipeline the layer's KV is the ``PackedKVCache`` of that computation
(``packed_kv``), so a reused layer neither packs nor attends.

Two additions, both off by default:

* ``reusable_layers`` restricts reuse to a set of layers (a fixed schedule,
  e.g. every other block);
* ``threshold=inf`` accepts any drift without computing it, so the decision
  needs no read of device memory and the step stays asynchronous. A zero-norm
  ``hidden_in`` (for which the reference computes no drift and recomputes the
  layer) is then reused too.
"""

from __future__ import annotations

import math
from dataclasses import dataclass, field
from typing import Any, Dict, FrozenSet, Optional, Set, Tuple

import torch


@dataclass(frozen=True)
class StepReuseConfig:
    """step_reuse.py:18-33, plus ``reusable_layers`` (None = every layer)."""

    enabled: bool = False
    threshold: float = 0.1
    warmup_steps: int = 1
    reusable_layers: Optional[FrozenSet[int]] = None

    def validate(self) -> None:
        if self.threshold < 0:
            raise ValueError(f"step reuse threshold must be >= 0, got {self.threshold}")
        if self.warmup_steps < 0:
            raise ValueError(f"step reuse warmup_steps must be >= 0, got {self.warmup_steps}")

    def __post_init__(self) -> None:
        if self.reusable_layers is not None:
            object.__setattr__(self, "reusable_layers", frozenset(int(i) for i in self.reusable_layers))
        self.validate()


@dataclass
class LayerReuseEntry:
    """step_reuse.py:36-43; ``k``/``v`` are None when the layer's KV lives
    packed in ``packed_kv``."""

    hidden_in: torch.Tensor
    hidden_out: torch.Tensor
    k: Optional[torch.Tensor] = None
    v: Optional[torch.Tensor] = None
    packed_kv: Any = None


@dataclass
class StepReuseState:
    """step_reuse.py:46-134."""

    entries: Dict[int, LayerReuseEntry] = field(default_factory=dict)
    last_attention: Optional[torch.Tensor] = None
    last_reused_layers: Set[int] = field(default_factory=set)
    last_computed_layers: Set[int] = field(default_factory=set)
    last_drifts: Dict[int, float] = field(default_factory=dict)
    attention_reused: bool = False

    def reset(self) -> None:
        self.entries.clear()
        self.last_attention = None
        self.last_reused_layers.clear()
        self.last_computed_layers.clear()
        self.last_drifts.clear()
        self.attention_reused = False

    def begin_step(self) -> None:
        self.last_reused_layers = set()
        self.last_computed_layers = set()
        self.last_drifts = {}
        self.attention_reused = False

    def drift(self, layer_id: int, hidden: torch.Tensor) -> Optional[float]:
        """||hidden - hidden_in|| / ||hidden_in|| (step_reuse.py:71-80); None
        without an entry of the same shape or for a zero-norm ``hidden_in``."""
        entry = self.entries.get(layer_id)
        if entry is None or entry.hidden_in.shape != hidden.shape:
            return None
        denom = entry.hidden_in.norm()
        if float(denom) <= 0.0:
            return None
        return float((hidden - entry.hidden_in).norm() / denom)

    def should_reuse(self, layer_id: int, hidden: torch.Tensor, step_id: int,
                     config: StepReuseConfig) -> Tuple[bool, Optional[float]]:
        """step_reuse.py:82-95."""
        if not config.enabled or step_id < config.warmup_steps:
            return False, None
        if config.reusable_layers is not None and layer_id not in config.reusable_layers:
            return False, None
        if math.isinf(config.threshold):
            entry = self.entries.get(layer_id)
            if entry is None or entry.hidden_in.shape != hidden.shape:
                self.entries.pop(layer_id, None)
                return False, None
            return True, None
        drift = self.drift(layer_id, hidden)
        if drift is None:
            self.entries.pop(layer_id, None)
            return False, None
        return drift <= config.threshold, drift

    def record(self, layer_id: int, hidden_in: torch.Tensor, hidden_out: torch.Tensor,
               k: Optional[torch.Tensor] = None, v: Optional[torch.Tensor] = None,
               packed_kv: Any = None) -> None:
        """step_reuse.py:97-111. The tensors are kept, not copied: callers
        must not modify them in place afterwards."""
        self.entries[layer_id] = LayerReuseEntry(
            hidden_in=hidden_in.detach(), hidden_out=hidden_out.detach(),
            k=None if k is None else k.detach(), v=None if v is None else v.detach(),
            packed_kv=packed_kv)

    def stats(self) -> Dict[str, Any]:
        """step_reuse.py:113-125."""
        reused = sorted(self.last_reused_layers)
        computed = sorted(self.last_computed_layers)
        total = len(reused) + len(computed)
        return {
            "reused_layers": reused,
            "computed_layers": computed,
            "reused_ratio": (len(reused) / total) if total else 0.0,
            "drifts": dict(self.last_drifts),
            "attention_reused": self.attention_reused,
        }
