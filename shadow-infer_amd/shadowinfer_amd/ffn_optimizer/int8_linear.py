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
from typing import Dict, List, Optional, Tuple

import torch
import torch.nn as nn

from .. import _native

logger = logging.getLogger("shadowinfer_amd.ffn_optimizer.int8_linear")

_ACT_SCALE_EPS = 1e-8
_WEIGHT_SCALE_EPS = 1e-8


def _checked_layout(qweight_nk: torch.Tensor, weight_scale: torch.Tensor,
                    bias: Optional[torch.Tensor], in_features: int, out_features: int) -> None:
    """The constructor's contract (int8_linear.py:37-52), on the [N, K] weight:
    ValueError for a non-int8 or misshapen weight, scale or bias."""
    if qweight_nk.dtype != torch.int8:
        raise ValueError(f"qweight must be int8, got {qweight_nk.dtype}")
    if tuple(qweight_nk.shape) != (out_features, in_features):
        raise ValueError(f"qweight of shape {tuple(qweight_nk.t().shape)} does not match "
                         f"(in_features, out_features) = ({in_features}, {out_features})")
    if weight_scale.dim() != 1 or weight_scale.numel() != out_features:
        raise ValueError(f"weight_scale must be 1-D with {out_features} elements, got shape "
                         f"{tuple(weight_scale.shape)}")
    if bias is not None and bias.numel() != out_features:
        raise ValueError(f"bias must have {out_features} elements, got {bias.numel()}")


class INT8Linear(nn.Module):
    """Linear layer with int8 weights, per-channel scales and dynamic activations.

    Constructed like the reference's (``qweight`` int8 ``[in_features,
    out_features]``, ``weight_scale`` ``[out_features]``, optional ``bias``);
    the weight is kept as its ``[out_features, in_features]`` transpose."""

    def __init__(self, qweight: torch.Tensor, weight_scale: torch.Tensor,
                 bias: Optional[torch.Tensor] = None, in_features: Optional[int] = None,
                 out_features: Optional[int] = None) -> None:
        if qweight.dim() != 2:
            raise ValueError(f"qweight must be 2-D, got shape {tuple(qweight.shape)}")
        self._init_nk(qweight.t(), weight_scale, bias,
                      int(qweight.shape[0]) if in_features is None else int(in_features),
                      int(qweight.shape[1]) if out_features is None else int(out_features))

    def _init_nk(self, qweight_nk: torch.Tensor, weight_scale: torch.Tensor,
                 bias: Optional[torch.Tensor], in_features: int, out_features: int) -> None:
        _checked_layout(qweight_nk, weight_scale, bias, in_features, out_features)
        nn.Module.__init__(self)
        self.in_features = in_features
        self.out_features = out_features
        self.register_buffer("qweight_nk", qweight_nk.contiguous())
        self.register_buffer("weight_scale", weight_scale.to(torch.float32).contiguous())
        self.register_buffer("bias", None if bias is None
                             else bias.to(torch.float32).reshape(-1).contiguous())

    @classmethod
    def from_quantized_nk(cls, qweight_nk: torch.Tensor, weight_scale: torch.Tensor,
                          bias: Optional[torch.Tensor] = None) -> "INT8Linear":
        """A layer over an int8 weight already in nn.Linear's ``[N, K]``
        layout (no transpose copy)."""
        if qweight_nk.dim() != 2:
            raise ValueError(f"qweight_nk must be 2-D, got shape {tuple(qweight_nk.shape)}")
        layer = cls.__new__(cls)
        layer._init_nk(qweight_nk, weight_scale, bias, int(qweight_nk.shape[1]),
                       int(qweight_nk.shape[0]))
        return layer

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
        return cls.from_quantized_nk(q_nk, scale, bias)

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
        """Bytes held: the int8 weight, fp32 scales and fp32 bias
        (int8_linear.py:128-132)."""
        return sum(t.numel() * t.element_size()
                   for t in (self.qweight_nk, self.weight_scale, self.bias) if t is not None)

    def dense_equivalent_bytes(self) -> int:
        """Bytes of the fp32 layer it replaces (int8_linear.py:134-138)."""
        return 4 * self.out_features * (self.in_features + (self.bias is not None))

    def extra_repr(self) -> str:
        return (f"in_features={self.in_features}, out_features={self.out_features}, "
                f"bias={self.bias is not None}, backend=hip")


def dequantized_weight(linear: INT8Linear) -> torch.Tensor:
    """The fp32 ``[in_features, out_features]`` weight ``q * s_w`` the layer
    stands for, for diagnostics (int8_linear.py:146-148)."""
    return (linear.qweight_nk.to(torch.float32) * linear.weight_scale[:, None]).t().contiguous()


FFN_LINEAR_SUFFIXES = (
    "mlp.up_proj",
    "mlp.down_proj",
    "mlp.gate_proj",
    "mlp.c_fc",
    "mlp.c_proj",
)


def _linear_slots(model: nn.Module, suffixes: Tuple[str, ...]):
    """(owner module, attribute, child) for every submodule whose qualified
    name ends with one of ``suffixes``: a pre-order walk of the module tree in
    registration order, visiting a module registered twice only under its
    first name (the order and the sharing rule of ``named_modules``)."""
    seen = {id(model)}

    def walk(prefix: str, owner: nn.Module):
        for attr, child in owner.named_children():
            if id(child) in seen:
                continue
            seen.add(id(child))
            name = f"{prefix}.{attr}" if prefix else attr
            if name.endswith(suffixes):
                yield owner, attr, child
            yield from walk(name, child)

    yield from walk("", model)


def quantize_ffn_modules(model: nn.Module, suffixes: tuple = FFN_LINEAR_SUFFIXES,
                         keep_fp32_reference: bool = False) -> Dict[str, object]:
    """Swap the FFN projections of ``model`` (submodules whose qualified name
    ends with one of ``suffixes``) for INT8Linear, in place
    (int8_linear.py:160-208). nn.Linear layers are quantized; layers that are
    already INT8Linear are counted as they are, so a second call changes
    nothing. Returns ``{"supported": False}`` when nothing matches, else the
    layer count, int8 and dense-equivalent weight bytes, whether any layer
    lacks its int8 kernel (``fallback``), and with ``keep_fp32_reference``
    the replaced layers as ``(owner, attribute, nn.Linear)`` under
    ``_references``."""
    layers: List[INT8Linear] = []
    replaced: List[tuple] = []
    for owner, attr, child in list(_linear_slots(model, tuple(suffixes))):
        if isinstance(child, INT8Linear):
            layers.append(child)
        elif isinstance(child, nn.Linear):
            layer = INT8Linear.from_linear(child)
            setattr(owner, attr, layer)
            layers.append(layer)
            replaced.append((owner, attr, child))
    if not layers:
        return {"supported": False}
    stats: Dict[str, object] = {
        "supported": True,
        "modules": len(layers),
        "weight_bytes": sum(layer.memory_bytes() for layer in layers),
        "dense_bytes": sum(layer.dense_equivalent_bytes() for layer in layers),
        "fallback": not all(layer.using_int_mm for layer in layers),
    }
    if keep_fp32_reference and replaced:
        stats["_references"] = replaced
    return stats


__all__ = ["FFN_LINEAR_SUFFIXES", "INT8Linear", "dequantized_weight", "quantize_ffn_modules"]
