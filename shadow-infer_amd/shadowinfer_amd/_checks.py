"""Argument checks shared by the Python entry points of several kernels."""

from __future__ import annotations

from . import _native


def check_rope_args(qkv, cos, sin, batch, seq, heads, head_dim, what):
    """The rotate-half RoPE launches (si_rope_split, si_kv_pack_rope_flat) read
    ``qkv [B*S, 3*H*D]`` and ``cos``/``sin`` ``[S, D]`` on one GPU, all in one dtype."""
    if qkv.shape != (batch * seq, 3 * heads * head_dim):
        raise ValueError(f"qkv must be [{batch * seq}, {3 * heads * head_dim}], got {tuple(qkv.shape)}")
    if cos.shape != (seq, head_dim) or sin.shape != (seq, head_dim):
        raise ValueError(f"cos/sin must be [{seq}, {head_dim}]")
    if cos.dtype != qkv.dtype or sin.dtype != qkv.dtype:
        raise ValueError("cos/sin must have qkv's dtype")
    _native.require_device(qkv, what)
    if cos.device != qkv.device or sin.device != qkv.device:
        raise ValueError(f"cos/sin must be on qkv's device ({qkv.device}), got {cos.device} / {sin.device}")
