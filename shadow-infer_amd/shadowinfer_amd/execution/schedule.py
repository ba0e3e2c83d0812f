"""Confidence-aware unmasking round (shadowinfer/execution/block_decoding.py:100-158)
on the device.

``schedule_round`` keeps the reference's decision rule: a masked position is
unmasked when its max softmax probability reaches the threshold; a batch row
with masked positions but none above the threshold unmasks its single most
confident masked position (the guaranteed-progress fallback). The per-position
argmax and confidence come from one HIP row kernel over the logits
(``si_row_argmax_conf``: argmax of the logits, confidence 1 / sum exp(l - max)
in fp32); the rest is a handful of [B, W] device ops with no host read, so a
denoising loop never waits for the GPU.

Differences from the reference, both in the last bits: the confidence is the
fp32 maximum probability, where the reference rounds the probabilities to the
logits' dtype before taking the maximum; and the argmax is taken over the
logits, so positions whose rounded probabilities tie keep the largest logit.
"""

from __future__ import annotations

from dataclasses import dataclass
from typing import Tuple

import torch

from .. import _native


@dataclass
class ScheduleDecision:
    """block_decoding.py:100-115."""

    unmask: torch.Tensor
    tokens: torch.Tensor
    confidences: torch.Tensor
    progress_fallback: torch.Tensor


def argmax_confidence(logits: torch.Tensor) -> Tuple[torch.Tensor, torch.Tensor]:
    """``logits [..., V]`` -> (int64 argmax ``[...]``, fp32 max probability ``[...]``)."""
    _native.require_device(logits, "argmax_confidence")
    V = logits.shape[-1]
    flat = logits.reshape(-1, V).contiguous()
    M = flat.shape[0]
    tok = torch.empty(M, dtype=torch.int64, device=flat.device)
    conf = torch.empty(M, dtype=torch.float32, device=flat.device)
    _native.call("si_row_argmax_conf", flat.data_ptr(), _native.dtype_code(flat.dtype), M, V,
                 tok.data_ptr(), conf.data_ptr(), _native.stream(flat.device))
    return tok.view(logits.shape[:-1]), conf.view(logits.shape[:-1])


def schedule_round(logits_block: torch.Tensor, masked: torch.Tensor,
                   confidence_threshold: float) -> ScheduleDecision:
    """block_decoding.py:118-158 with ``config.confidence_threshold`` passed
    directly. ``logits_block`` ``[B, W, V]``, ``masked`` bool ``[B, W]``."""
    if logits_block.dim() != 3:
        raise ValueError(f"logits_block must be 3-D [B, W, V], got dim={logits_block.dim()}")
    if masked.dim() != 2 or masked.shape != logits_block.shape[:2]:
        raise ValueError(
            f"masked must be [B, W] matching logits_block leading shape "
            f"{tuple(logits_block.shape[:2])}, got {tuple(masked.shape)}")
    if not 0.0 < confidence_threshold <= 1.0:
        raise ValueError(
            f"confidence_threshold must be within (0, 1], got {confidence_threshold}")
    tokens, confidences = argmax_confidence(logits_block)
    masked = masked.to(device=logits_block.device, dtype=torch.bool)
    above = masked & (confidences >= confidence_threshold)
    needs_fallback = masked.any(dim=1) & ~above.any(dim=1)
    masked_conf = confidences.masked_fill(~masked, float("-inf"))
    fallback_positions = masked_conf.argmax(dim=1, keepdim=True)
    fallback_unmask = torch.zeros_like(above).scatter_(1, fallback_positions,
                                                       needs_fallback.unsqueeze(1))
    unmask = above | fallback_unmask
    retained = confidences * (masked & ~unmask)
    return ScheduleDecision(unmask=unmask, tokens=tokens, confidences=retained,
                            progress_fallback=needs_fallback)
