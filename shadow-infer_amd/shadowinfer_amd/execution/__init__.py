"""Denoising-step execution over the quantized data plane: cross-step block
reuse (shadowinfer/execution/step_reuse.py), the confidence-aware unmasking
round (shadowinfer/execution/block_decoding.py) and a Llama-shaped diffusion
LM step on packed KV + INT8 FFN."""

from .denoise import DiffusionLlamaShape, PackedDiffusionLlama, mask_tokens
from .schedule import ScheduleDecision, argmax_confidence, schedule_round
from .step_reuse import LayerRecord, StepReuseConfig, StepReuseState

__all__ = [
    "DiffusionLlamaShape",
    "LayerRecord",
    "PackedDiffusionLlama",
    "ScheduleDecision",
    "StepReuseConfig",
    "StepReuseState",
    "argmax_confidence",
    "mask_tokens",
    "schedule_round",
]
