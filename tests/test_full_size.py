"""The large configurations at their real sizes on the GPU.

* One Llama-7B-shaped decoder layer of the denoising step (hidden 4096, 32
  heads, head_dim 128, SwiGLU 11008, vocab 32000, S = 2048 with 50% mask
  tokens, a per-layer packed KV with the 25% fp16 / 50% int8 / 25% int4 code
  mixture and a 4-token fp16 sink), stage by stage against the oracle from the
  GPU's own input to each stage (tests/stage_check.py): bit-exact for RoPE,
  the packed KV, the residual adds, the int8 activations and both INT8 GEMMs;
  the stages whose oracle is a GEMM are checked on 48 sampled rows.
* A 32-layer, 64-step generation of that model with step reuse on every other
  layer, checked by properties: finite logits at every step, at least one
  position unmasked per row and step, every mask resolved after the forced
  completion, reuse ratio 0.5 from the first step after warm-up, and each
  layer's packed bytes equal to the byte formula of its codes
  (packed_kv_cache.py:856-863).
* apply_reuse_mask with 50% of the token-heads on a 1 x 32 x 8192 x 128 bf16
  layer (packed_kv_cache.py:753-854), from a previous cache packed with the
  same plan and with a different one: buckets, scales and stats bit-exact to
  the oracle.
* evict of 25% of the token-heads of that layer (packed_kv_cache.py:666-751),
  given as the reference's set of (t, h) pairs: the removed count, the
  compacted buckets and scales, the byte count and the unpacked K/V bit-exact
  to the oracle.
"""

import numpy as np
import pytest
import torch

from helpers import assert_cache_equal, kv_inputs, mixed_codes, oracle_pack, to_np
from oracle import denoise_ref as R
from oracle import oracle as O

MIX = (0.0, 0.25, 0.5, 0.25)


def _sample_rows(T, n=48, seed=0):
    rng = np.random.default_rng(seed)
    rows = np.unique(np.concatenate([[0, 1, 2, 3, T - 1], rng.choice(T, n, replace=False)]))
    return rows


def _packed_bytes(codes, B, D, group, scale_bytes=2):
    """Bytes of a pack of these codes (packed_kv_cache.py:856-863, bf16 scales)."""
    n = np.bincount(codes.reshape(-1).astype(np.int64), minlength=5)
    G = D // group
    per = {0: 2 * 4 * B * D, 1: 2 * 2 * B * D, 2: 2 * (B * D + B * scale_bytes),
           3: 2 * ((B * D + 1) // 2 + B * G * scale_bytes)}
    return int(sum(n[p] * per[p] for p in range(4)))


@pytest.mark.gpu
def test_config5_layer_stage_by_stage(dev):
    from shadowinfer_amd.execution import DiffusionLlamaShape, PackedDiffusionLlama, mask_tokens
    from shadowinfer_amd.shadowkv import PrecisionPlan
    from stage_check import check_layer_stages, f32, rel_l2, weights
    cfg = DiffusionLlamaShape(num_hidden_layers=1)
    m = PackedDiffusionLlama(cfg, device=dev, seed=3)
    B, S = 1, 2048
    H, D, Hd = cfg.num_attention_heads, cfg.head_dim, cfg.hidden_size
    codes = mixed_codes(S, H, seed=21, probs=MIX)
    plan = PrecisionPlan.from_codes(torch.from_numpy(codes).to(dev))
    tokens, _ = mask_tokens(B, S, 0.5, cfg, dev, seed=5)
    traces = {}
    logits, kv = m.forward_step(tokens, [plan], traces=traces)
    print(f"config-5 layer: B={B} S={S} H={H} D={D} hidden={Hd}", flush=True)
    cos, sin = (to_np(t) for t in m.rope_tables(S))
    rows = _sample_rows(B * S)
    check_layer_stages(traces[0], weights(m, 0), codes, B, S, H, D, cfg.rms_norm_eps, cos, sin,
                       rows=rows)
    assert kv[0].memory_bytes() == _packed_bytes(codes, B, D, 16)
    fin = traces["final"]
    dt = O.BF16
    hn, amb = R.rmsnorm(to_np(fin["hidden"]).reshape(B * S, Hd), dt, to_np(m.norm),
                        cfg.rms_norm_eps, return_ambiguous=True)
    got = to_np(fin["hn"]).reshape(B * S, Hd)
    assert not ((got != hn).any(-1) & ~amb).any()
    lg = R.linear(got[rows], dt, to_np(m.lm_head))
    assert rel_l2(f32(to_np(logits).reshape(B * S, -1)[rows], dt), f32(lg, dt)) <= 2e-3


@pytest.mark.gpu
def test_config5_generation_properties(dev):
    from shadowinfer_amd.execution import (DiffusionLlamaShape, PackedDiffusionLlama,
                                           StepReuseConfig, StepReuseState, mask_tokens)
    from shadowinfer_amd.shadowkv import PrecisionPlan
    cfg = DiffusionLlamaShape()
    m = PackedDiffusionLlama(cfg, device=dev, seed=7)
    B, S, steps = 1, 2048, 64
    H, D = cfg.num_attention_heads, cfg.head_dim
    codes = [mixed_codes(S, H, seed=100 + i, probs=MIX) for i in range(cfg.num_hidden_layers)]
    plans = [PrecisionPlan.from_codes(torch.from_numpy(c).to(dev)) for c in codes]
    tokens, masked = mask_tokens(B, S, 0.5, cfg, dev, seed=9)
    start_tokens, start_masked = tokens.clone(), masked.clone()
    state = StepReuseState()
    reuse = StepReuseConfig(enabled=True, threshold=float("inf"), warmup_steps=1,
                            reusable_layers=frozenset(range(1, cfg.num_hidden_layers, 2)))
    ratios, byte_ok = [], []

    def on_step(step, d, kv, logits):
        ratios.append(state.stats()["reused_ratio"])
        if step in (0, steps - 1):
            byte_ok.append(all(kv[i].memory_bytes() == _packed_bytes(codes[i], B, D, 16)
                               for i in range(cfg.num_hidden_layers)))

    print(f"config-5 generation: {cfg.num_hidden_layers} layers, S={S}, {steps} steps", flush=True)
    res = m.generate(tokens, masked, plans, steps, 0.9, state, reuse, on_step=on_step)
    torch.cuda.synchronize()
    assert bool(res["finite"])
    per_step = res["unmasked_per_step"].cpu()
    assert bool((per_step >= 1).all())
    assert not bool(masked.any())
    assert torch.equal(tokens[~start_masked], start_tokens[~start_masked])
    assert int(per_step.sum()) + int(res["forced"].sum()) == int(start_masked.sum())
    assert ratios[0] == 0.0 and all(r == 0.5 for r in ratios[1:])
    assert byte_ok == [True, True]


@pytest.mark.gpu
@pytest.mark.parametrize("same_plan", [True, False])
def test_config3_reuse_50_percent_7b_layer(dev, same_plan):
    from shadowinfer_amd.shadowkv import PackedKVCache, PrecisionPlan
    B, H, S, D = 1, 32, 8192, 128
    k, v = kv_inputs(B, H, S, D, torch.bfloat16, seed=31, outlier_frac=0.01)
    kp, vp = kv_inputs(B, H, S, D, torch.bfloat16, seed=32, outlier_frac=0.01)
    codes = mixed_codes(S, H, seed=41, probs=MIX)
    codes_prev = codes if same_plan else mixed_codes(S, H, seed=42, probs=MIX)
    rng = np.random.default_rng(43)
    mask = rng.random((S, H)) < 0.5
    plan = PrecisionPlan.from_codes(torch.from_numpy(codes).to(dev))
    plan_prev = PrecisionPlan.from_codes(torch.from_numpy(codes_prev).to(dev))
    print(f"config-3 reuse: S={S} H={H} D={D} same_plan={same_plan}", flush=True)
    cur = PackedKVCache.pack(k.to(dev), v.to(dev), None, plan=plan)["packed_kv"]
    prev = PackedKVCache.pack(kp.to(dev), vp.to(dev), None, plan=plan_prev)["packed_kv"]
    stats = cur.apply_reuse_mask(prev, torch.from_numpy(mask).to(dev), return_stats=True)
    ref = oracle_pack(k, v, codes)
    ref_prev = oracle_pack(kp, vp, codes_prev)
    t, h = np.nonzero(mask)
    rstats = O.kv_apply_reuse_mask(ref, ref_prev, {(int(a), int(b)): True for a, b in zip(t, h)})
    assert stats == rstats
    # half the entries are masked; with two independent 25/50/25 plans an entry
    # keeps its precision with probability 0.375
    share = 0.5 if same_plan else 0.5 * 0.375
    assert abs(stats["applied"] / (S * H) - share) < 0.01
    if not same_plan:
        assert abs(stats["skipped_precision"] / (S * H) - 0.5 * 0.625) < 0.01
    assert_cache_equal(cur, ref)


@pytest.mark.gpu
def test_config3_evict_25_percent_7b_layer(dev):
    from shadowinfer_amd.shadowkv import PackedKVCache, PrecisionPlan
    B, H, S, D = 1, 32, 8192, 128
    k, v = kv_inputs(B, H, S, D, torch.bfloat16, seed=51, outlier_frac=0.01)
    codes = mixed_codes(S, H, seed=52, probs=MIX)
    rng = np.random.default_rng(53)
    flat = rng.choice(S * H, S * H // 4, replace=False)
    victims = {(int(e // H), int(e % H)) for e in flat}
    print(f"config-3 evict: S={S} H={H} D={D} victims={len(victims)}", flush=True)
    plan = PrecisionPlan.from_codes(torch.from_numpy(codes).to(dev))
    cache = PackedKVCache.pack(k.to(dev), v.to(dev), None, plan=plan)["packed_kv"]
    removed = cache.evict(victims)
    ref = oracle_pack(k, v, codes)
    assert removed == O.kv_evict(ref, victims) == len(victims)
    assert_cache_equal(cache, ref)  # buckets, scales, indices and memory_bytes
    k_out, v_out = cache.unpack()
    rk, rv = O.kv_unpack(ref)
    np.testing.assert_array_equal(to_np(k_out), rk)
    np.testing.assert_array_equal(to_np(v_out), rv)
    assert cache.evict(victims) == 0  # already absent: not counted again
