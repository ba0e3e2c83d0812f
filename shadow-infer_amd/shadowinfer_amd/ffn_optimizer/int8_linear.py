"""Executable INT8 linear layer with the reference API
(shadowinfer/ffn_optimizer/int8_linear.py:25-216) on a gfx950 MFMA GEMM.

Weights: symmetric per output channel, ``s_w = max(amax_k|w| / 127, 1e-8)``,
``q_w = clamp(round(w / s_w), -127, 127)``. The device buffer keeps
nn.Linear's ``[N, K]`` layout (K contiguous: the MFMA fragment layout, so the
GEMM streams it without transposition); ``qweight`` is the reference's
``[K, N]`` tensor as a view of it, and the state dict reads and writes the
reference's ``qweight [K, N]`` key.
Activations: per token row, ``s_x = max(amax / 127, 1e-8)``,
``q_x = clamp(round(x / s_x), -127, 127)``. The int8 x int8 -> int32 product
runs on MFMA (exact), then ``out = T(float(acc) * (s_x * s_w) [+ bias])``.
Activation quantization, GEMM and epilogue are one C-ABI call
(``si_int8_linear_forward``). There is no float fallback: a failing kernel
raises.
"""

from __future__ import annotations

import logging
from typing import Dict, Optional

import torch
import torch.nn as nn

from .. import _native

logger = logging.getLogger("shadowinfer_amd.ffn_optimizer.int8_linear")

_ACT_SCALE_EPS = 1e-8
_WEIGHT_SCALE_EPS = 1e-8


class INT8Linear(nn.Module):
    """Linear layer with int8 weights, per-channel scales and dynamic activations."""

    def __init__(self, qweight: torch.Tensor, weight_scale: torch.Tensor,
                 bias: Optional[torch.Tensor] = None, in_features: Optional[int] = None,
                 out_features: Optional[int] = None, *,
                 _qweight_nk: Optional[torch.Tensor] = None) -> None:
        super().__init__()
        if _qweight_nk is not None:
            qweight = _qweight_nk.t()
        if qweight.dim() != 2:
            raise ValueError(f"qweight must be 2-D, got shape {tuple(qweight.shape)}")
        if qweight.dtype != torch.int8:
            raise ValueError(f"qweight must be int8, got {qweight.dtype}")
        in_features = in_features if in_features is not None else int(qweight.shape[0])
        out_features = out_features if out_features is not None else int(qweight.shape[1])
        if tuple(qweight.shape) != (in_features, out_features):
            raise ValueError(
                f"qweight shape {tuple(qweight.shape)} != ({in_features}, {out_features})")
        if weight_scale.dim() != 1 or weight_scale.numel() != out_features:
            raise ValueError(
                f"weight_scale must have {out_features} elements, got {tuple(weight_scale.shape)}")
        if bias is not None and bias.numel() != out_features:
            raise ValueError(f"bias must have {out_features} elements")
        self.in_features = int(in_features)
        self.out_features = int(out_features)
        nk = _qweight_nk if _qweight_nk is not None else qweight.t()
        self.register_buffer("qweight_nk", nk.to(torch.int8).contiguous())
        self.register_buffer("weight_scale", weight_scale.to(torch.float32).contiguous())
        if bias is None:
            self.register_buffer("bias", None)
        else:
            self.register_buffer("bias", bias.to(torch.float32).contiguous())

    @classmethod
    def from_linear(cls, linear: nn.Linear) -> "INT8Linear":
        """Quantize an ``nn.Linear`` on its HIP device (int8_linear.py:65-82)."""
        if not isinstance(linear, nn.Linear):
            raise TypeError(f"expected nn.Linear, got {type(linear).__name__}")
        weight = linear.weight.detach().to(torch.float32).contiguous()
        _native.require_device(weight, "INT8Linear.from_linear")
        N, K = weight.shape
        q_nk = torch.empty((N, K), dtype=torch.int8, device=weight.device)
        scale = torch.empty(N, dtype=torch.float32, device=weight.device)
        _native.call("si_weight_quant_i8", weight.data_ptr(), N, K, q_nk.data_ptr(),
                     scale.data_ptr(), _native.stream(weight.device))
        bias = None if linear.bias is None else linear.bias.detach().to(torch.float32).clone()
        return cls(qweight=None, weight_scale=scale, bias=bias, in_features=linear.in_features,
                   out_features=linear.out_features, _qweight_nk=q_nk)

    @property
    def qweight(self) -> torch.Tensor:
        """The reference's ``[in_features, out_features]`` int8 weight (a view)."""
        return self.qweight_nk.t()

    def _save_to_state_dict(self, destination, prefix, keep_vars):
        super()._save_to_state_dict(destination, prefix, keep_vars)
        w = destination.pop(prefix + "qweight_nk")
        destination[prefix + "qweight"] = w.t() if keep_vars else w.t().contiguous()

    def _load_from_state_dict(self, state_dict, prefix, local_metadata, strict, missing_keys,
                              unexpected_keys, error_msgs):
        key = prefix + "qweight"
        if key in state_dict:
            state_dict[prefix + "qweight_nk"] = state_dict.pop(key).t().contiguous()
        super()._load_from_state_dict(state_dict, prefix, local_metadata, strict, missing_keys,
                                      unexpected_keys, error_msgs)

    @property
    def using_int_mm(self) -> bool:
        """True when the int8 GEMM kernel is available (it is the only path)."""
        try:
            _native.load()
            return True
        except RuntimeError:
            return False

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        """int8_linear.py:88-115."""
        if x.shape[-1] != self.in_features:
            raise ValueError(f"input last dim {x.shape[-1]} != in_features {self.in_features}")
        leading_shape = x.shape[:-1]
        flat = x.reshape(-1, self.in_features)
        if flat.numel() == 0:
            return torch.empty((*leading_shape, self.out_features), dtype=x.dtype, device=x.device)
        _native.require_device(flat, "INT8Linear.forward")
        if self.qweight_nk.device != flat.device:
            raise ValueError(f"input on {flat.device} but weights on {self.qweight_nk.device}")
        dt = _native.dtype_code(flat.dtype)
        flat = flat.contiguous()
        M, K, N = flat.shape[0], self.in_features, self.out_features
        out = torch.empty((M, N), dtype=x.dtype, device=x.device)
        ws_bytes = _native.size_query("si_int8_linear_workspace_bytes", M, K, N)
        ws = torch.empty(ws_bytes, dtype=torch.uint8, device=x.device)
        _native.call("si_int8_linear_forward", flat.data_ptr(), dt, M, K, N,
                     self.qweight_nk.data_ptr(), self.weight_scale.data_ptr(),
                     _native.ptr(self.bias), out.data_ptr(), ws.data_ptr(), ws_bytes,
                     _native.stream(x.device))
        return out.reshape(*leading_shape, N)

    def memory_bytes(self) -> int:
        total = self.qweight.numel() + self.weight_scale.numel() * 4
        if self.bias is not None:
            total += self.bias.numel() * 4
        return int(total)

    def dense_equivalent_bytes(self) -> int:
        total = self.in_features * self.out_features * 4
        if self.bias is not None:
            total += self.out_features * 4
        return int(total)

    def extra_repr(self) -> str:
        return (f"in_features={self.in_features}, out_features={self.out_features}, "
                f"bias={self.bias is not None}, backend=hip")


def dequantized_weight(linear: INT8Linear) -> torch.Tensor:
    """FP32 weight for diagnostics (int8_linear.py:146-148)."""
    return linear.qweight.to(torch.float32) * linear.weight_scale.unsqueeze(0)


FFN_LINEAR_SUFFIXES = (
    "mlp.up_proj",
    "mlp.down_proj",
    "mlp.gate_proj",
    "mlp.c_fc",
    "mlp.c_proj",
)


def quantize_ffn_modules(model: nn.Module, suffixes: tuple = FFN_LINEAR_SUFFIXES,
                         keep_fp32_reference: bool = False) -> Dict[str, object]:
    """Replace matching FFN ``nn.Linear`` modules with INT8Linear
    (int8_linear.py:160-208); idempotent."""
    references = [] if keep_fp32_reference else None
    modules = 0
    weight_bytes = 0
    dense_bytes = 0
    fallback = False
    for module_name, module in list(model.named_modules()):
        if not any(module_name.endswith(suffix) for suffix in suffixes):
            continue
        if isinstance(module, INT8Linear):
            modules += 1
            weight_bytes += module.memory_bytes()
            dense_bytes += module.dense_equivalent_bytes()
            fallback = fallback or not module.using_int_mm
            continue
        if not isinstance(module, nn.Linear):
            continue
        parent_name, _, attribute = module_name.rpartition(".")
        parent = model.get_submodule(parent_name) if parent_name else model
        quantized = INT8Linear.from_linear(module)
        if references is not None:
            references.append((parent, attribute, module))
        setattr(parent, attribute, quantized)
        modules += 1
        weight_bytes += quantized.memory_bytes()
        dense_bytes += quantized.dense_equivalent_bytes()
        fallback = fallback or not quantized.using_int_mm
    if modules == 0:
        return {"supported": False}
    stats: Dict[str, object] = {"supported": True, "modules": modules,
                                "weight_bytes": weight_bytes, "dense_bytes": dense_bytes,
                                "fallback": fallback}
    if references:
        stats["_references"] = references
    return stats


__all__ = ["FFN_LINEAR_SUFFIXES", "INT8Linear", "dequantized_weight", "quantize_ffn_modules"]
