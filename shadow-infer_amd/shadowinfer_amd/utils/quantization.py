"""Quantizer with the reference API (shadowinfer/utils/quantization.py:13-318),
running its int8/int4 arithmetic and nibble packing as HIP kernels.

Semantics kept from the reference:
* int8: per last-dim row, ``scale = T(amax / 127)`` (zero -> 1),
  ``q = clamp(round_half_even(T(x / scale)), -128, 127)``; scale in the input
  dtype T, shape ``[..., 1]``.
* int4: groups of ``group_size`` along the last dim, ``scale = T(amax / 7)``,
  clamp to [-8, 7]; returns codes ``[..., G, g]`` (int8) and scales
  ``[..., G, 1]``.
* pack_int4: offset-binary nibbles ``(q + 8) & 0xF``, first value in the high
  nibble, an odd tail padded with a zero nibble.
"""

from __future__ import annotations

from typing import List, Optional, Tuple, Union

import torch

from .. import _native


def _rows(t: torch.Tensor) -> Tuple[torch.Tensor, int, int]:
    t = t.contiguous()
    D = t.shape[-1] if t.dim() else 1
    rows = t.numel() // D if D else 0
    return t, rows, D


class Quantizer:
    """FP32 / FP16 / INT8 / INT4 quantization utilities (HIP device tensors)."""

    @staticmethod
    def quantize_tensor(tensor: torch.Tensor, precision: str,
                        group_size: int = 64) -> Tuple[torch.Tensor, Optional[torch.Tensor]]:
        p = precision.lower()
        if p == "fp32":
            return tensor, None
        if p == "fp16":
            return tensor.half(), None
        if p == "int8":
            return Quantizer.quantize_int8(tensor)
        if p == "int4":
            return Quantizer.quantize_int4(tensor, group_size=group_size)
        raise ValueError(f"Unsupported precision: {precision}")

    @staticmethod
    def quantize_batch(tensor_2d: torch.Tensor, precision: str,
                       group_size: int = 64) -> Tuple[torch.Tensor, Optional[torch.Tensor]]:
        return Quantizer.quantize_tensor(tensor_2d, precision, group_size=group_size)

    @staticmethod
    def dequantize_tensor(quantized: torch.Tensor, scale: Optional[torch.Tensor],
                          precision: str) -> torch.Tensor:
        p = precision.lower()
        if p == "fp32":
            return quantized
        if p == "fp16":
            return quantized.float()
        if p == "int8":
            if scale is None:
                raise ValueError("scale is required for INT8 dequantization")
            return Quantizer.dequantize_int8(quantized, scale)
        if p == "int4":
            if scale is None:
                raise ValueError("scale is required for INT4 dequantization")
            return Quantizer.dequantize_int4(quantized, scale)
        raise ValueError(f"Unsupported precision: {precision}")

    @staticmethod
    def quantize_int8(tensor: torch.Tensor) -> Tuple[torch.Tensor, torch.Tensor]:
        """quantization.py:120-142 on the device."""
        if tensor.numel() == 0:
            scale = torch.tensor(1.0, device=tensor.device, dtype=tensor.dtype)
            return tensor.to(torch.int8), scale
        _native.require_device(tensor, "Quantizer.quantize_int8")
        dt = _native.dtype_code(tensor.dtype)
        x, rows, D = _rows(tensor)
        q = torch.empty(x.shape, dtype=torch.int8, device=x.device)
        scale = torch.empty(x.shape[:-1] + (1,), dtype=x.dtype, device=x.device)
        _native.call("si_quant_rows_i8", x.data_ptr(), dt, rows, D, q.data_ptr(),
                     scale.data_ptr(), _native.stream(x.device))
        return q, scale

    @staticmethod
    def quantize_int4(tensor: torch.Tensor,
                      group_size: int = 64) -> Tuple[torch.Tensor, torch.Tensor]:
        """quantization.py:144-178 on the device."""
        if tensor.numel() == 0:
            scale = torch.tensor(1.0, device=tensor.device, dtype=tensor.dtype)
            return tensor.to(torch.int8), scale
        last_dim = tensor.shape[-1]
        if last_dim % group_size != 0:
            raise ValueError(
                f"last dim {last_dim} must be divisible by group_size {group_size}")
        _native.require_device(tensor, "Quantizer.quantize_int4")
        dt = _native.dtype_code(tensor.dtype)
        x, rows, D = _rows(tensor)
        G = D // group_size
        q = torch.empty(x.shape[:-1] + (G, group_size), dtype=torch.int8, device=x.device)
        scale = torch.empty(x.shape[:-1] + (G, 1), dtype=x.dtype, device=x.device)
        _native.call("si_quant_rows_i4", x.data_ptr(), dt, rows, D, group_size, q.data_ptr(),
                     scale.data_ptr(), _native.stream(x.device))
        return q, scale

    @staticmethod
    def dequantize_int8(quantized: torch.Tensor, scale: torch.Tensor) -> torch.Tensor:
        """``quantized.float() * scale`` (quantization.py:180-197)."""
        return Quantizer._dequant(quantized, scale, per_group=False)

    @staticmethod
    def dequantize_int4(quantized: torch.Tensor, scale: torch.Tensor) -> torch.Tensor:
        """``(quantized.float() * scale).reshape(*quantized.shape[:-2], -1)``
        (quantization.py:199-219)."""
        out = Quantizer._dequant(quantized, scale, per_group=True)
        return out.reshape(*quantized.shape[:-2], -1)

    @staticmethod
    def _dequant(q: torch.Tensor, scale: torch.Tensor, per_group: bool) -> torch.Tensor:
        """``q.float() * scale`` with any scale that broadcasts against ``q``
        (quantization.py:180-219): per-row ``[..., 1]`` and per-group scales,
        a per-tensor or 0-d scale (what quantize_* return for an empty
        tensor), or one scale per element. Result fp32 of the broadcast shape,
        each element ``float(q) * float(scale)`` (one fp32 multiply, as torch
        computes it). Codes are int8; scales fp32/fp16/bf16 (float64 scales,
        which torch would promote to a float64 result, raise TypeError)."""
        if not torch.is_tensor(scale):
            scale = torch.tensor(float(scale), dtype=torch.float32, device=q.device)
        if q.dtype != torch.int8:
            raise ValueError(f"dequantize expects int8 codes, got {q.dtype}")
        if scale.dtype not in (torch.float32, torch.float16, torch.bfloat16):
            raise TypeError(f"dequantize supports fp32/fp16/bf16 scales, got {scale.dtype}")
        if scale.device != q.device:
            if scale.dim() != 0:
                raise ValueError(f"scale on {scale.device} but codes on {q.device}")
            scale = scale.to(q.device)  # a 0-d tensor broadcasts across devices in torch
        shape = tuple(torch.broadcast_shapes(q.shape, scale.shape))
        n = 1
        for d in shape:
            n *= d
        if n == 0:
            return torch.empty(shape, dtype=torch.float32, device=q.device)
        _native.require_device(q, "Quantizer.dequantize")
        D = shape[-1] if shape else 1
        rows = n // D
        qc = (q.expand(shape) if tuple(q.shape) != shape else q).contiguous().reshape(rows, D)
        if scale.dim() == 0 or scale.shape[-1] == 1:
            # constant along the last dim: one scale per row
            sc = scale.reshape(scale.shape[:-1] if scale.dim() else ())
            sc = sc.expand(shape[:-1]).contiguous().reshape(rows)
            group = D
        else:
            sc = scale.expand(shape).contiguous().reshape(rows, D)
            group = 1
        out = torch.empty(shape, dtype=torch.float32, device=q.device)
        _native.call("si_dequant_rows", qc.data_ptr(), sc.data_ptr(), _native.dtype_code(sc.dtype),
                     rows, D, group, out.data_ptr(), _native.stream(q.device))
        return out

    @staticmethod
    def compute_quantization_error(original: torch.Tensor, quantized: torch.Tensor) -> float:
        if original.numel() == 0:
            return 0.0
        original_norm = torch.norm(original)
        if original_norm.item() == 0:
            return 0.0
        return float(torch.norm(original - quantized) / original_norm)

    @staticmethod
    def pack_int4(int8_tensor: torch.Tensor) -> torch.Tensor:
        """quantization.py:248-277: flat int4 codes -> bytes."""
        if int8_tensor.numel() == 0:
            return torch.empty(0, dtype=torch.uint8, device=int8_tensor.device)
        from ..kernels import _pack_int4
        return _pack_int4(int8_tensor)

    @staticmethod
    def unpack_int4(packed: torch.Tensor,
                    shape_or_num_elements: Union[int, Tuple[int, ...], List[int]]) -> torch.Tensor:
        """quantization.py:279-318."""
        if isinstance(shape_or_num_elements, (tuple, list)):
            n = 1
            for d in shape_or_num_elements:
                n *= int(d)
            shape = tuple(int(d) for d in shape_or_num_elements)
        else:
            n = int(shape_or_num_elements)
            shape = None
        if packed.numel() == 0:
            return torch.empty(shape if shape is not None else (n,), dtype=torch.int8,
                               device=packed.device)
        from ..kernels import _unpack_int4
        out = _unpack_int4(packed, n)
        return out.reshape(shape) if shape is not None else out
