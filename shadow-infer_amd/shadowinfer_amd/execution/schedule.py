"""Confidence-aware unmasking round (shadowinfer/execution/block_decoding.py:100-158)
on the device.

``schedule_round`` makes the reference's decisions index for index. The
reference computes ``probs = softmax(logits)`` in the logits' dtype and takes
``probs.max(-1)``; one HIP row kernel (``si_row_argmax_conf``) produces the same
two tensors without materialising the probabilities: the confidence in the
logits' dtype, and the first index whose rounded probability equals it (for
bf16 logits several near-equal logits often round to the same probability,
and the first of them wins, not the largest logit). The decision rule then
runs as the reference's own ``[B, W]`` torch ops on those tensors, so the
threshold is compared in the logits' dtype too and fallback ties go to the
smallest position. Nothing is read back to the host, so a denoising loop never
waits for the GPU.
"""

from __future__ import annotations

from dataclasses import dataclass
from typing import Tuple

import torch

from .. import _native


@dataclass
class ScheduleDecision:
    """Fields of block_decoding.py:100-115: ``unmask`` [B, W] bool,
    ``tokens`` [B, W] int64 (argmax of the rounded probabilities),
    ``confidences`` [B, W] (logits' dtype; 0 where unmasked or never masked),
    ``progress_fallback`` [B] bool."""

    unmask: torch.Tensor
    tokens: torch.Tensor
    confidences: torch.Tensor
    progress_fallback: torch.Tensor


def argmax_confidence(logits: torch.Tensor) -> Tuple[torch.Tensor, torch.Tensor]:
    """``softmax(logits, -1).max(-1)`` in the logits' dtype without the
    probability tensor: (int64 token ``[...]``, confidence ``[...]`` in
    ``logits.dtype``)."""
    _native.require_device(logits, "argmax_confidence")
    V = logits.shape[-1]
    flat = logits.reshape(-1, V).contiguous()
    M = flat.shape[0]
    tok = torch.empty(M, dtype=torch.int64, device=flat.device)
    conf = torch.empty(M, dtype=flat.dtype, device=flat.device)
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
    # a tensor in the logits' dtype against a Python float: torch compares in
    # that dtype, so the threshold is rounded to it, as in the reference
    above = masked & (confidences >= confidence_threshold)
    needs_fallback = masked.any(dim=1) & ~above.any(dim=1)
    # first position of the largest masked confidence (torch.argmax's tie rule)
    best = confidences.masked_fill(~masked, float("-inf")).argmax(dim=1, keepdim=True)
    # the reference sets fallback_unmask[b, best[b]] for rows needing it by a
    # boolean index; a scatter of the row flag onto zeros is the same tensor
    # without the host read of the index
    fallback_unmask = torch.zeros_like(above).scatter_(1, best, needs_fallback.unsqueeze(1))
    unmask = above | fallback_unmask
    retained = confidences * (masked & ~unmask)
    return ScheduleDecision(unmask=unmask, tokens=tokens, confidences=retained,
                            progress_fallback=needs_fallback)
