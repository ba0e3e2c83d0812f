"""One denoising step of a Llama-shaped diffusion LM over the quantized data
plane: INT8Linear gate/up/down projections and a per-layer packed
mixed-precision KV cache that is rebuilt every step (kv_lifecycle=replace),
with cross-step block reuse.

The reference has no single path that combines these pieces; this module
composes them the way its parts are defined:

* layer structure, RMSNorm, RoPE, bidirectional attention and SwiGLU:
  ``DiffusionLlamaDecoderLayer`` / ``DiffusionLlamaAttention`` /
  ``DiffusionLlamaMLP`` (models/diffusion_llama.py:311-468), multi-head
  (num_key_value_heads == num_attention_heads);
* gate/up/down as INT8Linear (ffn_optimizer/int8_linear.py:65-115,
  ``quantize_ffn_modules`` :151-157);
* packed KV with the replace lifecycle: every computed layer packs its
  post-RoPE K/V with the layer's PrecisionPlan and attends over the packed
  cache (core/backends/pytorch_backend.py:521-548; the fused dequant +
  attention kernel replaces unpack() + dense attention);
* block reuse: ``DiffusionTransformerBlock.forward``
  (models/simple_diffusion_llm.py:99-120) with ``StepReuseState``;
* unmasking: ``schedule_round`` (execution/block_decoding.py:118-158) over the
  full sequence.

Per computed layer the kernels are: RMSNorm (HIP) -> q|k|v projection (one
bf16 library GEMM) -> RoPE of q (HIP) -> KV pack reading K and V straight
from the projection, K rotated on the way (HIP; the dense K/V are not
written) -> packed attention writing token-major output (HIP) -> o projection (bf16 library
GEMM) -> residual add fused with the RMSNorm and the activation quantization
(HIP) -> gate|up INT8 GEMM (HIP, one GEMM over both weights) ->
SwiGLU fused with the down projection's activation quantization (HIP) ->
down INT8 GEMM with the residual add in its epilogue (HIP).

Weights are random (no checkpoints are loaded): linear weights ~ N(0, 0.02),
norms = 1, as a Llama initializer would give.
"""

from __future__ import annotations

from dataclasses import dataclass
from typing import Dict, List, Optional, Sequence, Tuple, Union

import torch
import torch.nn.functional as F

from .. import _native
from ..shadowkv.packed_attention import packed_attention
from ..shadowkv.packed_kv_cache import PackedKVCache
from ..shadowkv.precision_plan import PrecisionPlan
from . import row_ops
from .schedule import ScheduleDecision, schedule_round
from .step_reuse import StepReuseConfig, StepReuseState


@dataclass(frozen=True)
class DiffusionLlamaShape:
    """The architecture fields of DiffusionLlamaConfig
    (models/diffusion_llama.py:98-140) this step needs. Defaults: a
    Llama-7B-shaped model."""

    num_hidden_layers: int = 32
    hidden_size: int = 4096
    num_attention_heads: int = 32
    intermediate_size: int = 11008
    vocab_size: int = 32000
    rms_norm_eps: float = 1e-5
    rope_theta: float = 10000.0
    mask_token_id: int = 31999
    int4_group_size: int = 16

    @property
    def head_dim(self) -> int:
        return self.hidden_size // self.num_attention_heads

    def validate(self) -> None:
        if self.hidden_size % self.num_attention_heads:
            raise ValueError("hidden_size must be a multiple of num_attention_heads")
        if self.head_dim not in (64, 128):
            raise ValueError(f"head_dim must be 64 or 128, got {self.head_dim}")
        if self.hidden_size % 16 or self.intermediate_size % 16:
            raise ValueError("hidden_size and intermediate_size must be multiples of 16")
        if not 0 <= self.mask_token_id < self.vocab_size:
            raise ValueError("mask_token_id must be a token id")

    def __post_init__(self) -> None:
        self.validate()


class _Layer:
    __slots__ = ("ln1", "w_qkv", "w_o", "ln2", "gu_q", "gu_s", "dn_q", "dn_s")


class PackedDiffusionLlama:
    """Llama-shaped diffusion LM whose forward step runs on the packed KV /
    INT8 FFN data plane. ``forward_step`` mirrors DiffusionLlama.forward_step
    (models/diffusion_llama.py:535-593) with the packed-KV arguments of the
    backend; ``denoise_step`` adds one unmasking round."""

    def __init__(self, config: DiffusionLlamaShape, device: Union[str, torch.device] = "cuda",
                 dtype: torch.dtype = torch.bfloat16, seed: int = 0) -> None:
        if dtype not in (torch.bfloat16, torch.float16):
            raise TypeError(f"dtype must be bfloat16 or float16, got {dtype}")
        self.config = config
        self.device = torch.device(device)
        if self.device.type != "cuda":
            raise ValueError("PackedDiffusionLlama runs on a HIP device")
        _native.load()
        self.dtype = dtype
        c = config
        g = torch.Generator(device=self.device)
        g.manual_seed(seed)

        def normal(*shape):
            return torch.randn(*shape, generator=g, device=self.device, dtype=torch.float32).mul_(0.02)

        Hd, Fi = c.hidden_size, c.intermediate_size
        ones = torch.ones(Hd, dtype=dtype, device=self.device)
        self.embed = normal(c.vocab_size, Hd).to(dtype)
        self.layers: List[_Layer] = []
        for _ in range(c.num_hidden_layers):
            L = _Layer()
            L.ln1 = ones.clone()
            L.ln2 = ones.clone()
            L.w_qkv = normal(3 * Hd, Hd).to(dtype)      # q | k | v rows, nn.Linear layout
            L.w_o = normal(Hd, Hd).to(dtype)
            # gate | up rows quantized per output channel (per-row scales, so
            # the same bytes as two separate INT8Linear.from_linear calls)
            L.gu_q, L.gu_s = row_ops.weight_quant_i8(normal(2 * Fi, Hd))
            L.dn_q, L.dn_s = row_ops.weight_quant_i8(normal(Hd, Fi))
            self.layers.append(L)
        self.norm = ones.clone()
        self.lm_head = normal(c.vocab_size, Hd).to(dtype)
        self.inv_freq = 1.0 / (c.rope_theta ** (
            torch.arange(0, c.head_dim, 2, dtype=torch.float32, device=self.device) / c.head_dim))
        self._rope: Dict[int, Tuple[torch.Tensor, torch.Tensor]] = {}

    # ------------------------------------------------------------------ parts
    def rope_tables(self, seq_len: int) -> Tuple[torch.Tensor, torch.Tensor]:
        """cos/sin ``[S, D]`` in the model dtype (models/diffusion_llama.py:505-514)."""
        t = self._rope.get(seq_len)
        if t is None:
            pos = torch.arange(seq_len, device=self.device, dtype=torch.float32)
            freqs = torch.outer(pos, self.inv_freq)
            emb = torch.cat((freqs, freqs), dim=-1)
            t = (emb.cos().to(self.dtype), emb.sin().to(self.dtype))
            self._rope[seq_len] = t
        return t

    def layer_forward(self, layer_id: int, hidden: torch.Tensor, plan: PrecisionPlan,
                      cos: torch.Tensor, sin: torch.Tensor,
                      trace: Optional[dict] = None) -> Tuple[torch.Tensor, PackedKVCache]:
        """One decoder layer (models/diffusion_llama.py:407-424) on the packed
        data plane. ``hidden`` ``[B, S, hidden]``; returns the new hidden state
        (a fresh tensor) and the layer's packed KV. ``trace``, when given,
        receives every intermediate tensor (for parity tests)."""
        c = self.config
        L = self.layers[layer_id]
        B, S, Hd = hidden.shape
        H, D = c.num_attention_heads, c.head_dim
        T = B * S
        x = hidden.reshape(T, Hd)
        xn, _, _, _ = row_ops.rmsnorm(x, L.ln1, c.rms_norm_eps)
        qkv = F.linear(xn, L.w_qkv)
        if trace is None and row_ops.rope_pack_supported(qkv.dtype, D, c.int4_group_size):
            # K and V go from the projection straight into the packed cache
            q, k, v = row_ops.rope_split(qkv, cos, sin, B, S, H, D, kv=False)
            cache = PackedKVCache.pack_projection(qkv, cos, sin, B, S, H, D,
                                                  c.int4_group_size, plan)
        else:
            q, k, v = row_ops.rope_split(qkv, cos, sin, B, S, H, D)
            cache = PackedKVCache.pack(k, v, None, group_size=c.int4_group_size,
                                       plan=plan)["packed_kv"]
        attn = packed_attention(q, cache, out_dtype=self.dtype, token_major=True)
        o = F.linear(attn.view(T, Hd), L.w_o)
        y2, qx, sx, x1 = row_ops.rmsnorm(x, L.ln2, c.rms_norm_eps, want_y=trace is not None,
                                         want_q=True, residual=o)
        gu = row_ops.int8_gemm_dequant(qx, sx, L.gu_q, L.gu_s, self.dtype)
        h, qh, sh = row_ops.swiglu_quant(gu, want_h=trace is not None)
        # the down projection with the residual add in its epilogue
        out = row_ops.int8_gemm_dequant(qh, sh, L.dn_q, L.dn_s, self.dtype, residual=x1)
        ffn = None
        if trace is not None:
            ffn = row_ops.int8_gemm_dequant(qh, sh, L.dn_q, L.dn_s, self.dtype)
        if trace is not None:
            trace.update(x=x, xn=xn, qkv=qkv, q=q, k=k, v=v, cache=cache, attn=attn, o=o, x1=x1,
                         y2=y2, qx=qx, sx=sx, gu=gu, h=h, qh=qh, sh=sh, ffn=ffn, out=out)
        return out.view(B, S, Hd), cache

    # ------------------------------------------------------------------- step
    def forward_step(self, x: torch.Tensor, plans: Union[PrecisionPlan, Sequence[PrecisionPlan]],
                     step_id: int = 0, reuse_state: Optional[StepReuseState] = None,
                     reuse_config: Optional[StepReuseConfig] = None,
                     traces: Optional[Dict[int, dict]] = None
                     ) -> Tuple[torch.Tensor, Dict[int, PackedKVCache]]:
        """``x`` int64 ``[B, S]`` token ids -> (logits ``[B, S, V]`` in the
        model dtype, {layer: PackedKVCache}). ``plans``: one PrecisionPlan per
        layer (or one for all) over ``[S, heads]``. A reused layer returns the
        packed cache of its last computation."""
        c = self.config
        if x.dim() != 2 or x.dtype not in (torch.long, torch.int):
            raise ValueError("x must be [batch, seq_len] integer token ids")
        B, S = x.shape
        if isinstance(plans, PrecisionPlan):
            plans = [plans] * c.num_hidden_layers
        if len(plans) != c.num_hidden_layers:
            raise ValueError(f"need {c.num_hidden_layers} plans, got {len(plans)}")
        for p in plans:
            if p.seq_len != S or p.num_heads != c.num_attention_heads:
                raise ValueError(
                    f"PrecisionPlan shape mismatch: plan (seq_len={p.seq_len}, "
                    f"num_heads={p.num_heads}) vs (seq_len={S}, num_heads={c.num_attention_heads})")
        cos, sin = self.rope_tables(S)
        hidden = F.embedding(x.to(self.device), self.embed)
        kv: Dict[int, PackedKVCache] = {}
        gated = reuse_state is not None and reuse_config is not None
        if reuse_state is not None:
            reuse_state.new_step()
        for i in range(c.num_hidden_layers):
            record = reuse_state.gate(i, hidden, step_id, reuse_config) if gated else None
            if record is not None:
                hidden = reuse_state.reuse(i, record, hidden)
                kv[i] = record.packed_kv
                continue
            trace = None
            if traces is not None:
                trace = traces.setdefault(i, {})
            h_in = hidden
            hidden, cache = self.layer_forward(i, hidden, plans[i], cos, sin, trace)
            if reuse_state is not None:
                reuse_state.keep(i, h_in, hidden, cache)
            kv[i] = cache
        hn, _, _, _ = row_ops.rmsnorm(hidden, self.norm, c.rms_norm_eps)
        logits = F.linear(hn, self.lm_head)
        if traces is not None:
            traces["final"] = {"hidden": hidden, "hn": hn, "logits": logits}
        return logits, kv

    def denoise_step(self, tokens: torch.Tensor, masked: torch.Tensor,
                     plans: Union[PrecisionPlan, Sequence[PrecisionPlan]], step_id: int = 0,
                     confidence_threshold: float = 0.9,
                     reuse_state: Optional[StepReuseState] = None,
                     reuse_config: Optional[StepReuseConfig] = None
                     ) -> Tuple[ScheduleDecision, Dict[int, PackedKVCache], torch.Tensor]:
        """forward_step + one unmasking round (block_decoding.py:497-502 over
        the whole sequence); ``tokens`` (int64 ``[B, S]``) and ``masked`` (bool
        ``[B, S]``) are updated in place on the device. Returns the decision,
        the per-layer packed KV and the step's logits."""
        logits, kv = self.forward_step(tokens, plans, step_id, reuse_state, reuse_config)
        decision = schedule_round(logits, masked, confidence_threshold)
        tokens.copy_(torch.where(decision.unmask, decision.tokens, tokens))
        masked &= ~decision.unmask
        return decision, kv, logits

    def generate(self, tokens: torch.Tensor, masked: torch.Tensor,
                 plans: Union[PrecisionPlan, Sequence[PrecisionPlan]], steps: int,
                 confidence_threshold: float = 0.9,
                 reuse_state: Optional[StepReuseState] = None,
                 reuse_config: Optional[StepReuseConfig] = None,
                 on_step=None) -> Dict[str, torch.Tensor]:
        """``steps`` denoising steps, then the reference's forced completion
        (block_decoding.py:493-512): positions still masked after the last
        round take the argmax of that round's logits. ``tokens``/``masked``
        are updated in place; the loop never reads the device. Returns device
        tensors: ``unmasked_per_step`` int64 ``[steps, B]``, ``fallback`` bool
        ``[steps, B]``, ``forced`` int64 ``[B]`` (positions completed by the
        argmax) and ``finite`` bool (every logit of every step finite).
        ``on_step(step, decision, kv, logits)``, when given, sees each step."""
        if steps < 1:
            raise ValueError(f"steps must be >= 1, got {steps}")
        B = tokens.shape[0]
        dev = tokens.device
        unmasked = torch.zeros(steps, B, dtype=torch.int64, device=dev)
        fallback = torch.zeros(steps, B, dtype=torch.bool, device=dev)
        finite = torch.ones((), dtype=torch.bool, device=dev)
        logits = None
        for step in range(steps):
            d, kv, logits = self.denoise_step(tokens, masked, plans, step, confidence_threshold,
                                              reuse_state, reuse_config)
            unmasked[step] = d.unmask.sum(dim=1)
            fallback[step] = d.progress_fallback
            finite &= torch.isfinite(logits).all()
            if on_step is not None:
                on_step(step, d, kv, logits)
        forced = masked.sum(dim=1)
        tokens.copy_(torch.where(masked, logits.argmax(dim=-1), tokens))
        masked.zero_()
        return {"unmasked_per_step": unmasked, "fallback": fallback, "forced": forced,
                "finite": finite}


def mask_tokens(batch: int, seq_len: int, mask_fraction: float, config: DiffusionLlamaShape,
                device: Union[str, torch.device], seed: int = 0
                ) -> Tuple[torch.Tensor, torch.Tensor]:
    """Synthetic denoising input: random token ids with ``mask_fraction`` of
    the positions (seeded choice) set to the mask token. Returns (tokens
    int64 ``[B, S]``, masked bool ``[B, S]``)."""
    g = torch.Generator().manual_seed(seed)
    tokens = torch.randint(0, config.vocab_size - 1, (batch, seq_len), generator=g)
    tokens[tokens >= config.mask_token_id] += 1  # keep the mask id for masks only
    tokens.clamp_(max=config.vocab_size - 1)
    n = int(round(mask_fraction * seq_len))
    masked = torch.zeros(batch, seq_len, dtype=torch.bool)
    for b in range(batch):
        masked[b, torch.randperm(seq_len, generator=g)[:n]] = True
    tokens[masked] = config.mask_token_id
    return tokens.to(device), masked.to(device)
