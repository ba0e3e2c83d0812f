// Row kernels of one denoising step of a Llama-shaped diffusion LM
// (models/diffusion_llama.py:311-393): RMSNorm fused with the INT8Linear
// activation quantization, RoPE with the q/k/v head split, SwiGLU fused with
// the down projection's activation quantization, and the per-position argmax /
// confidence of the unmasking schedule (execution/block_decoding.py:148-151).
// Every row kernel holds its row in registers: one read of HBM per element.
#include <mutex>

#include "si_common.h"

namespace si {
namespace {

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
  return v;
}

__device__ __forceinline__ float wave_absmax(float m) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) m = amax_fold(m, __shfl_xor(m, off, 64));
  return m;
}

// Block-wide reductions over 256 threads (4 waves); every thread gets the result.
__device__ __forceinline__ float block_sum(float v, float* lds) {
  v = wave_sum(v);
  if ((threadIdx.x & 63) == 0) lds[threadIdx.x >> 6] = v;
  __syncthreads();
  const float r = (lds[0] + lds[1]) + (lds[2] + lds[3]);
  __syncthreads();
  return r;
}

__device__ __forceinline__ float block_absmax(float m, float* lds) {
  m = wave_absmax(m);
  if ((threadIdx.x & 63) == 0) lds[threadIdx.x >> 6] = m;
  __syncthreads();
  float r = lds[0];
  for (int w = 1; w < 4; ++w) r = amax_fold(r, lds[w]);
  __syncthreads();
  return r;
}

// Block-wide maximum over 256 threads (NaN-free inputs); every thread gets it.
__device__ __forceinline__ float block_max(float m, float* lds) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) m = fmaxf(m, __shfl_xor(m, off, 64));
  if ((threadIdx.x & 63) == 0) lds[threadIdx.x >> 6] = m;
  __syncthreads();
  const float r = fmaxf(fmaxf(lds[0], lds[1]), fmaxf(lds[2], lds[3]));
  __syncthreads();
  return r;
}

template <int DT>
__device__ __forceinline__ void load8(const void* p, int64_t i, float* v) {
  if constexpr (DT == SI_DT_F32) {
    const float4 lo = reinterpret_cast<const float4*>(reinterpret_cast<const float*>(p) + i)[0];
    const float4 hi = reinterpret_cast<const float4*>(reinterpret_cast<const float*>(p) + i)[1];
    v[0] = lo.x; v[1] = lo.y; v[2] = lo.z; v[3] = lo.w;
    v[4] = hi.x; v[5] = hi.y; v[6] = hi.z; v[7] = hi.w;
  } else {
    const uint4 w = *reinterpret_cast<const uint4*>(reinterpret_cast<const uint16_t*>(p) + i);
    const uint32_t ws[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      v[2 * e] = DT == SI_DT_BF16 ? bf16_bits_to_f32(ws[e] & 0xffffu) : f16_bits_to_f32(ws[e] & 0xffffu);
      v[2 * e + 1] = DT == SI_DT_BF16 ? bf16_bits_to_f32(ws[e] >> 16) : f16_bits_to_f32(ws[e] >> 16);
    }
  }
}

// Stores 8 values already rounded to DT (exact conversion).
template <int DT>
__device__ __forceinline__ void store8(void* p, int64_t i, const float* v) {
  if constexpr (DT == SI_DT_F32) {
    float* d = reinterpret_cast<float*>(p) + i;
    reinterpret_cast<float4*>(d)[0] = make_float4(v[0], v[1], v[2], v[3]);
    reinterpret_cast<float4*>(d)[1] = make_float4(v[4], v[5], v[6], v[7]);
  } else {
    uint32_t w[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const uint32_t lo = DT == SI_DT_BF16 ? f32_to_bf16_bits(v[2 * e]) : f32_to_f16_bits(v[2 * e]);
      const uint32_t hi = DT == SI_DT_BF16 ? f32_to_bf16_bits(v[2 * e + 1]) : f32_to_f16_bits(v[2 * e + 1]);
      w[e] = lo | (hi << 16);
    }
    *reinterpret_cast<uint4*>(reinterpret_cast<uint16_t*>(p) + i) = make_uint4(w[0], w[1], w[2], w[3]);
  }
}

// INT8Linear activation quantization of a row held by the block
// (int8_linear.py:96-98): s = max(amax / 127, 1e-8), q = clamp(rint(x / s), +-127)
// with the IEEE quotient, as si_act_quant_i8.
// The quotient is Markstein's: q0 = x * r with r = RN(1/s), e = x - q0 * s
// (exact, one fma), q1 = RN(q0 + e * r) = RN(x/s) for every finite x and
// normal s (s >= 1e-8 here) -- the IEEE quotient without a division per value.
template <int R>
__device__ __forceinline__ void quant_row(float (&v)[R][8], int nch, int64_t row, int K,
                                          int8_t* __restrict__ q, float* __restrict__ scale,
                                          float* lds) {
  float a = 0.0f;
#pragma unroll
  for (int r = 0; r < R; ++r)
    if ((int)threadIdx.x + r * 256 < nch)
#pragma unroll
      for (int e = 0; e < 8; ++e) a = amax_fold(a, v[r][e]);
  a = block_absmax(a, lds);
  float s = a / 127.0f;
  s = s < 1e-8f ? 1e-8f : s;  // clamp_min(1e-8); NaN passes through like torch
  if (threadIdx.x == 0) scale[row] = s;
  const float rinv = 1.0f / s;
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const int c = (int)threadIdx.x + r * 256;
    if (c >= nch) continue;
    uint32_t b[2] = {0u, 0u};
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const float q0 = v[r][e] * rinv;
      float t = rintf(__builtin_fmaf(__builtin_fmaf(-q0, s, v[r][e]), rinv, q0));
      t = fminf(fmaxf(t, -127.0f), 127.0f);
      b[e >> 2] |= ((uint32_t)(int)t & 0xffu) << (8 * (e & 3));
    }
    *reinterpret_cast<uint2*>(q + row * K + (int64_t)c * 8) = make_uint2(b[0], b[1]);
  }
}

// A value that rounds to T exactly as the IEEE quotient x / rs does. For
// T = bf16, with x and rs bf16 values, that is x * RN(1/rs): the product is
// within 1.5 fp32 ulps of x / rs, while x / rs (a ratio of two 8-bit
// significands) is either a bf16 value or at least 2^-17 (relative) away from
// every bf16 rounding midpoint, far more than the error, so both round to the
// same bf16 (checked over every pair of bf16 significands, and over the
// exponent ranges of rows of any scale, by the exhaustive quotient tests).
// fp16 and fp32 rows keep the division.
template <int DT>
__device__ __forceinline__ float div_rs(float x, float rs, float rinv) {
  if constexpr (DT == SI_DT_BF16) return x * rinv;
  else return x / rs;
}

// ---------------------------------------------------------------------------
// RMSNorm (DiffusionLlamaRMSNorm, diffusion_llama.py:311-321) over rows of K,
// following the reference's op chain in the row dtype T, every op rounded to T:
//   var = T(mean(T(x^2)))          (fp32 sum, then * factor as torch's mean)
//   r   = T(sqrt(T(var + eps)))
//   y   = T(T(x / r) * w)
// factor is torch's mean factor float(M) / float(M * K) (1/K when exact).
// With RESID, x is first replaced by T(x + resid) (the residual add of
// DiffusionLlamaDecoderLayer.forward, diffusion_llama.py:421-423), which is
// also written to xo. Optional outputs: y [M, K] in T, and the INT8Linear
// quantization of y (q int8 [M, K], scale fp32 [M]) -- the input of a quantized
// projection, bit-identical to si_act_quant_i8 on y. One block per row, the
// row in registers (K <= 2048 R).
// ---------------------------------------------------------------------------
template <int DT, int R, bool RESID>
__global__ __launch_bounds__(256) void rmsnorm_rows(const void* __restrict__ x,
                                                    const void* __restrict__ res,
                                                    const void* __restrict__ w, int64_t M, int K,
                                                    float factor, float eps,
                                                    void* __restrict__ xo, void* __restrict__ y,
                                                    int8_t* __restrict__ q,
                                                    float* __restrict__ scale) {
  __shared__ float lds[4];
  const int nch = K / 8;
  for (int64_t m = blockIdx.x; m < M; m += gridDim.x) {
    float v[R][8];
    float ss = 0.0f;
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const int c = (int)threadIdx.x + r * 256;
      if (c < nch) {
        load8<DT>(x, m * K + (int64_t)c * 8, v[r]);
        if constexpr (RESID) {
          float o[8];
          load8<DT>(res, m * K + (int64_t)c * 8, o);
#pragma unroll
          for (int e = 0; e < 8; ++e) v[r][e] = round_to(v[r][e] + o[e], DT);
          store8<DT>(xo, m * K + (int64_t)c * 8, v[r]);
        }
#pragma unroll
        for (int e = 0; e < 8; ++e) ss += round_to(v[r][e] * v[r][e], DT);
      } else {
#pragma unroll
        for (int e = 0; e < 8; ++e) v[r][e] = 0.0f;
      }
    }
    ss = block_sum(ss, lds);
    const float var = round_to(ss * factor, DT);
    const float rs = round_to(sqrtf(round_to(var + eps, DT)), DT);
    const float rinv = 1.0f / rs;
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const int c = (int)threadIdx.x + r * 256;
      if (c >= nch) continue;
      float wv[8];
      load8<DT>(w, (int64_t)c * 8, wv);
#pragma unroll
      for (int e = 0; e < 8; ++e) v[r][e] = round_to(round_to(div_rs<DT>(v[r][e], rs, rinv), DT) * wv[e], DT);
      if (y != nullptr) store8<DT>(y, m * K + (int64_t)c * 8, v[r]);
    }
    if (q != nullptr) quant_row<R>(v, nch, m, K, q, scale, lds);
  }
}

// ---------------------------------------------------------------------------
// RoPE + head split (DiffusionLlamaAttention.forward, diffusion_llama.py:362-373):
// qkv [B*S, 3*H*D] (q | k | v column blocks, each [H, D]) ->
// q, k, v [B, H, S, D], q and k rotated as the reference's
// q * cos + rotate_half(q) * sin in the row dtype T (each product rounded to
// T, then the sum rounded to T):
//   out[d]       = T(T(x[d] cos[s,d]) - T(x[d+D/2] sin[s,d]))
//   out[d+D/2]   = T(T(x[d+D/2] cos[s,d+D/2]) + T(x[d] sin[s,d+D/2]))   (d < D/2)
// with the cos/sin tables [S, D] in T (the reference's emb = cat(freqs, freqs)
// cast to the parameter dtype).
// A thread owns 8 dims of the first half and their 8 partners. With ko and vo
// NULL only q is written (K and V then go straight into a packed cache).
// ---------------------------------------------------------------------------
template <int DT, int D>
__global__ __launch_bounds__(256) void rope_split(const void* __restrict__ qkv,
                                                  const void* __restrict__ cosb,
                                                  const void* __restrict__ sinb, int64_t B,
                                                  int64_t S, int64_t H, void* __restrict__ qo,
                                                  void* __restrict__ ko, void* __restrict__ vo) {
  constexpr int HALF = D / 2;
  constexpr int TPH = HALF / 8;  // threads per head
  const int64_t total = B * S * H * TPH;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total;
       i += (int64_t)gridDim.x * blockDim.x) {
    const int j = (int)(i % TPH);
    const int64_t hs = i / TPH;       // (b*S + s)*H + h
    const int64_t h = hs % H;
    const int64_t bs = hs / H;        // b*S + s
    const int64_t s = bs % S;
    const int64_t b = bs / S;
    const int d = 8 * j;
    const int64_t in = bs * 3 * H * D + h * D + d;
    const int64_t out = ((b * H + h) * S + s) * D + d;
    float c0[8], c1[8], s0[8], s1[8];
    load8<DT>(cosb, s * D + d, c0);
    load8<DT>(cosb, s * D + d + HALF, c1);
    load8<DT>(sinb, s * D + d, s0);
    load8<DT>(sinb, s * D + d + HALF, s1);
    const int parts = ko != nullptr ? 2 : 1;
#pragma unroll
    for (int part = 0; part < 2; ++part) {
      if (part >= parts) break;
      float x0[8], x1[8], y0[8], y1[8];
      load8<DT>(qkv, in + part * H * D, x0);
      load8<DT>(qkv, in + part * H * D + HALF, x1);
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        y0[e] = round_to(round_to(x0[e] * c0[e], DT) - round_to(x1[e] * s0[e], DT), DT);
        y1[e] = round_to(round_to(x1[e] * c1[e], DT) + round_to(x0[e] * s1[e], DT), DT);
      }
      void* dst = part == 0 ? qo : ko;
      store8<DT>(dst, out, y0);
      store8<DT>(dst, out + HALF, y1);
    }
    if (vo == nullptr) continue;
    float v0[8], v1[8];
    load8<DT>(qkv, in + 2 * H * D, v0);
    load8<DT>(qkv, in + 2 * H * D + HALF, v1);
    store8<DT>(vo, out, v0);
    store8<DT>(vo, out + HALF, v1);
  }
}

// ---------------------------------------------------------------------------
// silu(g) rounded to T as torch computes it: T(g / (1 + expf(-g))) in fp32
// with IEEE division and the library expf.
// For T = bf16/fp16 a fast form f = g * rcp(1 + exp2(-g log2e)) (v_exp_f32,
// v_rcp_f32) is used when it provably rounds the same way. Its distance to the
// fp32 quotient E is below B = (|g| 2^-22 + 2^-19) |f|: the rounded constant
// and product -g log2e move the exponent by at most |g| log2e 2^-23 (a
// relative error of at most |g| 2^-23 in exp); v_exp_f32, v_rcp_f32 and the
// library expf add one ulp (2^-23) each, and the roundings of the two sums,
// the product and the quotient half an ulp each (6e-7 in all, below
// 2^-19 = 1.9e-6). If f - 2B and f + 2B round to
// the same T value, E does too; otherwise (a T rounding midpoint lies in the
// interval, about 0.2% of elements for bf16) E itself is computed. |g| >= 64,
// NaN and infinities always take the exact path.
// ---------------------------------------------------------------------------
template <int DT>
__device__ __forceinline__ float silu_rounded(float g) {
  if constexpr (DT == SI_DT_F32) {
    return g / (1.0f + expf(-g));
  } else {
    const float ex = __builtin_amdgcn_exp2f(-g * 1.44269504088896341f);
    const float f = g * __builtin_amdgcn_rcpf(1.0f + ex);
    const float b = 2.0f * fabsf(f) * (fabsf(g) * 0x1p-22f + 0x1p-19f);
    const float lo = round_to(f - b, DT);
    if (lo == round_to(f + b, DT) && fabsf(g) < 64.0f) return lo;
    return round_to(g / (1.0f + expf(-g)), DT);
  }
}

// silu_rounded<T>(x) for all 2^16 bf16 (row 0) and fp16 (row 1) bit patterns
// x, as bits of T: a 16-bit row value picks its entry instead of evaluating
// silu. Filled on a device (silu_table_fill, 65,536 threads) before its first
// use; 256 KB of module memory per device, kept until the process ends.
__device__ uint16_t silu_tab[2][65536];

__global__ __launch_bounds__(256) void silu_table_fill() {
  const uint32_t x = blockIdx.x * 256u + threadIdx.x;
  silu_tab[0][x] = (uint16_t)f32_to_bf16_bits(silu_rounded<SI_DT_BF16>(bf16_bits_to_f32(x)));
  silu_tab[1][x] = (uint16_t)f32_to_f16_bits(silu_rounded<SI_DT_F16>(f16_bits_to_f32(x)));
}

// ---------------------------------------------------------------------------
// SwiGLU + down-projection input quantization (DiffusionLlamaMLP.forward,
// diffusion_llama.py:332-333; the down INT8Linear prologue int8_linear.py:96-98):
// gu [M, 2F] holds gate | up; h = T(T(silu(g)) * u) (torch's two elementwise
// ops, each rounded to T; T(silu(g)) as silu_rounded, from silu_tab for bf16
// and fp16 rows). Writes h [M, F] (optional) and its INT8Linear quantization
// q int8 [M, F], scale fp32 [M].
// ---------------------------------------------------------------------------
template <int DT, int R>
__global__ __launch_bounds__(256) void swiglu_quant(const void* __restrict__ gu, int64_t M, int F,
                                                    void* __restrict__ h, int8_t* __restrict__ q,
                                                    float* __restrict__ scale) {
  __shared__ float lds[4];
  const int nch = F / 8;
  for (int64_t m = blockIdx.x; m < M; m += gridDim.x) {
    float v[R][8];
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const int c = (int)threadIdx.x + r * 256;
      if (c < nch) {
        float u[8];
        load8<DT>(gu, m * 2 * F + F + (int64_t)c * 8, u);
        if constexpr (DT == SI_DT_F32) {
          float g[8];
          load8<DT>(gu, m * 2 * F + (int64_t)c * 8, g);
#pragma unroll
          for (int e = 0; e < 8; ++e) v[r][e] = round_to(silu_rounded<DT>(g[e]) * u[e], DT);
        } else {
          const uint4 gw = *reinterpret_cast<const uint4*>(
              reinterpret_cast<const uint16_t*>(gu) + m * 2 * F + (int64_t)c * 8);
          const uint32_t ws[4] = {gw.x, gw.y, gw.z, gw.w};
          const uint16_t* tab = silu_tab[DT == SI_DT_BF16 ? 0 : 1];
#pragma unroll
          for (int e = 0; e < 8; ++e) {
            const uint32_t bits = (e & 1) ? ws[e >> 1] >> 16 : ws[e >> 1] & 0xffffu;
            const uint32_t sb = tab[bits];
            const float sv = DT == SI_DT_BF16 ? bf16_bits_to_f32(sb) : f16_bits_to_f32(sb);
            v[r][e] = round_to(sv * u[e], DT);
          }
        }
        if (h != nullptr) store8<DT>(h, m * F + (int64_t)c * 8, v[r]);
      } else {
#pragma unroll
        for (int e = 0; e < 8; ++e) v[r][e] = 0.0f;
      }
    }
    quant_row<R>(v, nch, m, F, q, scale, lds);
  }
}

// ---------------------------------------------------------------------------
// Per-position token and confidence of schedule_round
// (block_decoding.py:146-147): probs = softmax(logits) in the logits' dtype T,
// then (conf, tok) = probs.max(-1), which takes the first index among equal
// maxima. torch's softmax computes p_v = T(expf(l_v - m) / s) with m the row
// max and s = sum_v expf(l_v - m) in fp32, so
//   conf = T(1 / s)                                  (expf(0) = 1)
//   tok  = first v with T(expf(l_v - m) / s) == conf
// Ties after the rounding to T are common for bf16 logits, and they resolve to
// the first index, not to the largest logit. Only logits within 1/16 of m can
// tie (a tie needs expf(l_v - m) >= 1 - 2^-7 for bf16, closer for fp16/fp32).
// A row holding a NaN or +inf, or only -inf, has NaN probabilities: conf NaN,
// tok 0 (the first NaN).
// One block per row, three passes over the row (max; sum; first tie), the
// later two from L2.
// ---------------------------------------------------------------------------
template <int DT, bool VEC, typename F>
__device__ __forceinline__ void for_row(const void* __restrict__ logits, int64_t m, int64_t V,
                                        F&& f) {
  if constexpr (VEC) {
    for (int64_t c = threadIdx.x; c < V / 8; c += blockDim.x) {
      float v[8];
      load8<DT>(logits, m * V + c * 8, v);
#pragma unroll
      for (int e = 0; e < 8; ++e) f(v[e], c * 8 + e);
    }
  } else {
    for (int64_t i = threadIdx.x; i < V; i += blockDim.x) f(load_any(logits, DT, m * V + i), i);
  }
}

template <int DT, bool VEC>
__global__ __launch_bounds__(256) void row_argmax_conf(const void* __restrict__ logits,
                                                       int64_t M, int64_t V,
                                                       int64_t* __restrict__ tok,
                                                       void* __restrict__ conf) {
  __shared__ float lds[4];
  __shared__ int64_t ldi[4];
  for (int64_t m = blockIdx.x; m < M; m += gridDim.x) {
    // pass 1: the row max, and whether the softmax is NaN everywhere
    float mx = -INFINITY;
    float bad = 0.0f;
    for_row<DT, VEC>(logits, m, V, [&](float x, int64_t) {
      if (x != x || x == INFINITY) bad = 1.0f;
      mx = fmaxf(mx, x);
    });
    mx = block_max(mx, lds);
    bad = block_sum(bad, lds);
    if (bad != 0.0f || mx == -INFINITY) {
      if (threadIdx.x == 0) {
        tok[m] = 0;
        store_any(conf, DT, m, __uint_as_float(0x7fc00000u));
      }
      continue;
    }
    // pass 2: the sum of exponentials
    float s = 0.0f;
    for_row<DT, VEC>(logits, m, V, [&](float x, int64_t) { s += expf(x - mx); });
    s = block_sum(s, lds);
    const float c = round_to(1.0f / s, DT);
    // pass 3: the first index whose rounded probability equals c
    int64_t first = INT64_MAX;
    for_row<DT, VEC>(logits, m, V, [&](float x, int64_t i) {
      if (i < first && x - mx >= -0.0625f && round_to(expf(x - mx) / s, DT) == c) first = i;
    });
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) {
      const int64_t o = __shfl_xor(first, off, 64);
      first = o < first ? o : first;
    }
    if ((threadIdx.x & 63) == 0) ldi[threadIdx.x >> 6] = first;
    __syncthreads();
    if (threadIdx.x == 0) {
      int64_t r = ldi[0];
      for (int w = 1; w < 4; ++w) r = ldi[w] < r ? ldi[w] : r;
      tok[m] = r;
      store_any(conf, DT, m, c);
    }
    __syncthreads();
  }
}

// ---------------------------------------------------------------------------
// Cross-step block reuse (execution/step_reuse.py:71-95,
// models/simple_diffusion_llm.py:104): the drift gate's two sums and the
// reused hidden state.
//   reuse_partial : per block, sum T(h - h_in)^2 and sum h_in^2 in fp32 over
//                   a grid-strided share of n elements (8 per load), then
//   reuse_final   : one block adds the block partials in a fixed order.
// The result is deterministic for a given n. The caller takes the square
// roots and the ratio (torch's norm: fp32 accumulation, one rounding to T).
//   reuse_apply   : out = T(h_out + T(h - h_in)), the reference's two ops.
// ---------------------------------------------------------------------------
constexpr int kReuseBlocks = 1024;

template <int DT>
__global__ __launch_bounds__(256) void reuse_partial(const void* __restrict__ h,
                                                     const void* __restrict__ hin, int64_t n,
                                                     float* __restrict__ part) {
  __shared__ float lds[4];
  float a = 0.0f, b = 0.0f;
  const int64_t nch = n / 8;
  for (int64_t c = (int64_t)blockIdx.x * 256 + threadIdx.x; c < nch;
       c += (int64_t)gridDim.x * 256) {
    float x[8], y[8];
    load8<DT>(h, c * 8, x);
    load8<DT>(hin, c * 8, y);
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const float d = round_to(x[e] - y[e], DT);
      a += d * d;
      b += y[e] * y[e];
    }
  }
  if (blockIdx.x == 0) {
    for (int64_t i = nch * 8 + threadIdx.x; i < n; i += 256) {
      const float y = load_any(hin, DT, i);
      const float d = round_to(load_any(h, DT, i) - y, DT);
      a += d * d;
      b += y * y;
    }
  }
  a = block_sum(a, lds);
  b = block_sum(b, lds);
  if (threadIdx.x == 0) {
    part[blockIdx.x] = a;
    part[gridDim.x + blockIdx.x] = b;
  }
}

__global__ __launch_bounds__(256) void reuse_final(const float* __restrict__ part, int nb,
                                                   float* __restrict__ out) {
  __shared__ float lds[4];
  float a = 0.0f, b = 0.0f;
  for (int i = threadIdx.x; i < nb; i += 256) {
    a += part[i];
    b += part[nb + i];
  }
  a = block_sum(a, lds);
  b = block_sum(b, lds);
  if (threadIdx.x == 0) {
    out[0] = a;
    out[1] = b;
  }
}

template <int DT>
__global__ __launch_bounds__(256) void reuse_apply(const void* __restrict__ h,
                                                   const void* __restrict__ hin,
                                                   const void* __restrict__ hout, int64_t n,
                                                   void* __restrict__ out) {
  const int64_t nch = n / 8;
  for (int64_t c = (int64_t)blockIdx.x * 256 + threadIdx.x; c < nch;
       c += (int64_t)gridDim.x * 256) {
    float x[8], y[8], z[8];
    load8<DT>(h, c * 8, x);
    load8<DT>(hin, c * 8, y);
    load8<DT>(hout, c * 8, z);
#pragma unroll
    for (int e = 0; e < 8; ++e) z[e] = round_to(z[e] + round_to(x[e] - y[e], DT), DT);
    store8<DT>(out, c * 8, z);
  }
  if (blockIdx.x == 0) {
    for (int64_t i = nch * 8 + threadIdx.x; i < n; i += 256) {
      const float d = round_to(load_any(h, DT, i) - load_any(hin, DT, i), DT);
      store_any(out, DT, i, load_any(hout, DT, i) + d);
    }
  }
}

unsigned row_grid(int64_t M) { return (unsigned)(M < 262144 ? (M < 1 ? 1 : M) : 262144); }

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

template <int DT, bool RESID>
void launch_rmsnorm(const void* x, const void* res, const void* w, int64_t M, int K, float factor,
                    float eps, void* xo, void* y, int8_t* q, float* s, hipStream_t st) {
  const unsigned g = row_grid(M);
  if (K <= 2048)
    rmsnorm_rows<DT, 1, RESID><<<g, 256, 0, st>>>(x, res, w, M, K, factor, eps, xo, y, q, s);
  else if (K <= 4096)
    rmsnorm_rows<DT, 2, RESID><<<g, 256, 0, st>>>(x, res, w, M, K, factor, eps, xo, y, q, s);
  else if (K <= 8192)
    rmsnorm_rows<DT, 4, RESID><<<g, 256, 0, st>>>(x, res, w, M, K, factor, eps, xo, y, q, s);
  else
    rmsnorm_rows<DT, 8, RESID><<<g, 256, 0, st>>>(x, res, w, M, K, factor, eps, xo, y, q, s);
}

// torch's mean factor for M rows of K: float(M) / float(M * K) (ATen's
// mean_kernel_impl), equal to 1/K whenever M * K is exact in fp32.
float mean_factor(int64_t M, int64_t K) { return (float)M / (float)(M * K); }

template <bool RESID>
int rmsnorm_entry(const char* name, const void* x, const void* res, int dtype, int64_t M,
                  int64_t K, const void* weight, float eps, void* xo, void* y, int8_t* q,
                  float* scale, si_stream_t stream) {
  SI_CHECK_ARG(dtype == SI_DT_BF16 || dtype == SI_DT_F16 || dtype == SI_DT_F32,
               "%s: unsupported dtype %d", name, dtype);
  SI_CHECK_ARG(M >= 0 && K > 0 && K % 8 == 0 && K <= 16384,
               "%s: K must be a multiple of 8 in [8, 16384] (got %lld)", name, (long long)K);
  SI_CHECK_ARG((q == nullptr) == (scale == nullptr), "%s: q and scale are given together", name);
  if (M == 0) return SI_OK;
  SI_CHECK_ARG(x && weight && (y || q) && (!RESID || (res && xo)), "%s: NULL argument", name);
  SI_CHECK_ARG(aligned16(x) && aligned16(weight) && (!y || aligned16(y)) &&
                   (!RESID || (aligned16(res) && aligned16(xo))) &&
                   (!q || (reinterpret_cast<uintptr_t>(q) & 7) == 0),
               "%s: x, residual, weight, x_out and y must be 16-byte aligned, q 8-byte aligned",
               name);
  hipStream_t st = as_stream(stream);
  const float f = mean_factor(M, K);
  if (dtype == SI_DT_BF16)
    launch_rmsnorm<SI_DT_BF16, RESID>(x, res, weight, M, (int)K, f, eps, xo, y, q, scale, st);
  else if (dtype == SI_DT_F16)
    launch_rmsnorm<SI_DT_F16, RESID>(x, res, weight, M, (int)K, f, eps, xo, y, q, scale, st);
  else
    launch_rmsnorm<SI_DT_F32, RESID>(x, res, weight, M, (int)K, f, eps, xo, y, q, scale, st);
  return check_launch(name);
}

// silu_tab is filled on a device by silu_table_fill launched on the stream
// of every call until one fill is known to have finished (an event recorded
// after it has completed); from then on every stream of the device reads the
// table. Fills write identical values, so overlapping ones are harmless, and a
// call under graph capture captures its fill.
constexpr int kMaxDevices = 64;

void ensure_silu_table(hipStream_t st) {
  static std::mutex mu;
  static bool ready[kMaxDevices];
  static hipEvent_t done[kMaxDevices];
  static bool recorded[kMaxDevices];  // a never-recorded event reads as complete
  // The stream's device; -1 (fill on every call, no event) when it is not the
  // current device, where an event created here could not be recorded on st.
  hipDevice_t dev = -1;
  int cur = -1;
  if (hipStreamGetDevice(st, &dev) != hipSuccess || hipGetDevice(&cur) != hipSuccess ||
      dev != cur || dev < 0 || dev >= kMaxDevices)
    dev = -1;
  hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
  const bool capturing =
      hipStreamIsCapturing(st, &cap) != hipSuccess || cap != hipStreamCaptureStatusNone;
  std::lock_guard<std::mutex> lock(mu);
  if (dev >= 0 && ready[dev]) return;
  if (dev >= 0 && !capturing && recorded[dev] && hipEventQuery(done[dev]) == hipSuccess) {
    ready[dev] = true;
    return;
  }
  silu_table_fill<<<256, 256, 0, st>>>();
  if (dev < 0 || capturing) return;
  if (done[dev] == nullptr &&
      hipEventCreateWithFlags(&done[dev], hipEventDisableTiming) != hipSuccess)
    done[dev] = nullptr;
  if (done[dev] != nullptr && hipEventRecord(done[dev], st) == hipSuccess) recorded[dev] = true;
}

template <int DT>
void launch_swiglu(const void* gu, int64_t M, int F, void* h, int8_t* q, float* s, hipStream_t st) {
  if (DT != SI_DT_F32) ensure_silu_table(st);
  const unsigned g = row_grid(M);
  if (F <= 2048) swiglu_quant<DT, 1><<<g, 256, 0, st>>>(gu, M, F, h, q, s);
  else if (F <= 4096) swiglu_quant<DT, 2><<<g, 256, 0, st>>>(gu, M, F, h, q, s);
  else if (F <= 8192) swiglu_quant<DT, 4><<<g, 256, 0, st>>>(gu, M, F, h, q, s);
  else if (F <= 12288) swiglu_quant<DT, 6><<<g, 256, 0, st>>>(gu, M, F, h, q, s);
  else swiglu_quant<DT, 8><<<g, 256, 0, st>>>(gu, M, F, h, q, s);
}

template <int DT>
void launch_rope(const void* qkv, const void* c, const void* s, int64_t B, int64_t S, int64_t H,
                 int64_t D, void* q, void* k, void* v, hipStream_t st) {
  const int64_t total = B * S * H * (D / 16);
  const unsigned g = (unsigned)std::min<int64_t>(ceil_div(total, 256), 262144);
  if (D == 64) rope_split<DT, 64><<<g, 256, 0, st>>>(qkv, c, s, B, S, H, q, k, v);
  else rope_split<DT, 128><<<g, 256, 0, st>>>(qkv, c, s, B, S, H, q, k, v);
}


}  // namespace
}  // namespace si

using namespace si;

extern "C" int si_rmsnorm_rows(const void* x, int dtype, int64_t M, int64_t K, const void* weight,
                               float eps, void* y, int8_t* q, float* scale, si_stream_t stream) {
  clear_error();
  return rmsnorm_entry<false>("si_rmsnorm_rows", x, nullptr, dtype, M, K, weight, eps, nullptr, y,
                              q, scale, stream);
}

extern "C" int si_add_rmsnorm_rows(const void* x, const void* residual, int dtype, int64_t M,
                                   int64_t K, const void* weight, float eps, void* x_out, void* y,
                                   int8_t* q, float* scale, si_stream_t stream) {
  clear_error();
  return rmsnorm_entry<true>("si_add_rmsnorm_rows", x, residual, dtype, M, K, weight, eps, x_out,
                             y, q, scale, stream);
}

extern "C" int si_rope_split(const void* qkv, int dtype, int64_t B, int64_t S, int64_t H,
                             int64_t D, const void* cos_table, const void* sin_table, void* q,
                             void* k, void* v, si_stream_t stream) {
  clear_error();
  SI_CHECK_ARG(dtype == SI_DT_BF16 || dtype == SI_DT_F16 || dtype == SI_DT_F32,
               "si_rope_split: unsupported dtype %d", dtype);
  SI_CHECK_ARG(D == 64 || D == 128, "si_rope_split: head_dim must be 64 or 128 (got %lld)",
               (long long)D);
  SI_CHECK_ARG(B >= 0 && S >= 0 && H >= 0, "si_rope_split: bad shape");
  if (B * S * H == 0) return SI_OK;
  SI_CHECK_ARG(qkv && cos_table && sin_table && q && (k != nullptr) == (v != nullptr),
               "si_rope_split: NULL argument (k and v are both given or both NULL)");
  SI_CHECK_ARG(aligned16(qkv) && aligned16(cos_table) && aligned16(sin_table) && aligned16(q) &&
                   (k == nullptr || (aligned16(k) && aligned16(v))),
               "si_rope_split: pointers must be 16-byte aligned");
  hipStream_t st = as_stream(stream);
  if (dtype == SI_DT_BF16) launch_rope<SI_DT_BF16>(qkv, cos_table, sin_table, B, S, H, D, q, k, v, st);
  else if (dtype == SI_DT_F16) launch_rope<SI_DT_F16>(qkv, cos_table, sin_table, B, S, H, D, q, k, v, st);
  else launch_rope<SI_DT_F32>(qkv, cos_table, sin_table, B, S, H, D, q, k, v, st);
  return check_launch("si_rope_split");
}

extern "C" int si_swiglu_quant(const void* gate_up, int dtype, int64_t M, int64_t F, void* h,
                               int8_t* q, float* scale, si_stream_t stream) {
  clear_error();
  SI_CHECK_ARG(dtype == SI_DT_BF16 || dtype == SI_DT_F16 || dtype == SI_DT_F32,
               "si_swiglu_quant: unsupported dtype %d", dtype);
  SI_CHECK_ARG(M >= 0 && F > 0 && F % 8 == 0 && F <= 16384,
               "si_swiglu_quant: F must be a multiple of 8 in [8, 16384] (got %lld)", (long long)F);
  if (M == 0) return SI_OK;
  SI_CHECK_ARG(gate_up && q && scale, "si_swiglu_quant: NULL argument");
  SI_CHECK_ARG(aligned16(gate_up) && (!h || aligned16(h)) && (reinterpret_cast<uintptr_t>(q) & 7) == 0,
               "si_swiglu_quant: gate_up and h must be 16-byte aligned, q 8-byte aligned");
  hipStream_t st = as_stream(stream);
  if (dtype == SI_DT_BF16) launch_swiglu<SI_DT_BF16>(gate_up, M, (int)F, h, q, scale, st);
  else if (dtype == SI_DT_F16) launch_swiglu<SI_DT_F16>(gate_up, M, (int)F, h, q, scale, st);
  else launch_swiglu<SI_DT_F32>(gate_up, M, (int)F, h, q, scale, st);
  return check_launch("si_swiglu_quant");
}

extern "C" int si_row_argmax_conf(const void* logits, int dtype, int64_t M, int64_t V,
                                  int64_t* tokens, void* confidence, si_stream_t stream) {
  clear_error();
  SI_CHECK_ARG(dtype_ok(dtype), "si_row_argmax_conf: unsupported dtype %d", dtype);
  SI_CHECK_ARG(M >= 0 && V > 0, "si_row_argmax_conf: bad shape");
  if (M == 0) return SI_OK;
  SI_CHECK_ARG(logits && tokens && confidence, "si_row_argmax_conf: NULL argument");
  hipStream_t st = as_stream(stream);
  const unsigned g = row_grid(M);
  const bool vec = V % 8 == 0 && aligned16(logits);
  if (dtype == SI_DT_BF16) {
    if (vec) row_argmax_conf<SI_DT_BF16, true><<<g, 256, 0, st>>>(logits, M, V, tokens, confidence);
    else row_argmax_conf<SI_DT_BF16, false><<<g, 256, 0, st>>>(logits, M, V, tokens, confidence);
  } else if (dtype == SI_DT_F16) {
    if (vec) row_argmax_conf<SI_DT_F16, true><<<g, 256, 0, st>>>(logits, M, V, tokens, confidence);
    else row_argmax_conf<SI_DT_F16, false><<<g, 256, 0, st>>>(logits, M, V, tokens, confidence);
  } else {
    if (vec) row_argmax_conf<SI_DT_F32, true><<<g, 256, 0, st>>>(logits, M, V, tokens, confidence);
    else row_argmax_conf<SI_DT_F32, false><<<g, 256, 0, st>>>(logits, M, V, tokens, confidence);
  }
  return check_launch("si_row_argmax_conf");
}

extern "C" size_t si_reuse_drift_workspace_bytes(int64_t n) {
  (void)n;
  return 2 * kReuseBlocks * sizeof(float);
}

extern "C" int si_reuse_drift(const void* hidden, const void* hidden_in, int dtype, int64_t n,
                              float* out, void* workspace, size_t workspace_bytes,
                              si_stream_t stream) {
  clear_error();
  SI_CHECK_ARG(dtype_ok(dtype), "si_reuse_drift: unsupported dtype %d", dtype);
  SI_CHECK_ARG(n >= 0, "si_reuse_drift: bad size");
  SI_CHECK_ARG(out && workspace, "si_reuse_drift: NULL argument");
  SI_CHECK_ARG(workspace_bytes >= si_reuse_drift_workspace_bytes(n),
               "si_reuse_drift: workspace of %zu bytes, need %zu", workspace_bytes,
               si_reuse_drift_workspace_bytes(n));
  SI_CHECK_ARG(n == 0 || (hidden && hidden_in && aligned16(hidden) && aligned16(hidden_in)),
               "si_reuse_drift: hidden and hidden_in must be 16-byte aligned device pointers");
  hipStream_t st = as_stream(stream);
  const int nb = (int)std::min<int64_t>(kReuseBlocks, std::max<int64_t>(1, ceil_div(n / 8, 256)));
  float* part = static_cast<float*>(workspace);
  if (dtype == SI_DT_BF16) reuse_partial<SI_DT_BF16><<<nb, 256, 0, st>>>(hidden, hidden_in, n, part);
  else if (dtype == SI_DT_F16) reuse_partial<SI_DT_F16><<<nb, 256, 0, st>>>(hidden, hidden_in, n, part);
  else reuse_partial<SI_DT_F32><<<nb, 256, 0, st>>>(hidden, hidden_in, n, part);
  reuse_final<<<1, 256, 0, st>>>(part, nb, out);
  return check_launch("si_reuse_drift");
}

extern "C" int si_reuse_apply(const void* hidden, const void* hidden_in, const void* hidden_out,
                              int dtype, int64_t n, void* out, si_stream_t stream) {
  clear_error();
  SI_CHECK_ARG(dtype_ok(dtype), "si_reuse_apply: unsupported dtype %d", dtype);
  SI_CHECK_ARG(n >= 0, "si_reuse_apply: bad size");
  if (n == 0) return SI_OK;
  SI_CHECK_ARG(hidden && hidden_in && hidden_out && out, "si_reuse_apply: NULL argument");
  SI_CHECK_ARG(aligned16(hidden) && aligned16(hidden_in) && aligned16(hidden_out) && aligned16(out),
               "si_reuse_apply: pointers must be 16-byte aligned");
  hipStream_t st = as_stream(stream);
  const unsigned g = (unsigned)std::min<int64_t>(std::max<int64_t>(1, ceil_div(n / 8, 256)), 4096);
  if (dtype == SI_DT_BF16) reuse_apply<SI_DT_BF16><<<g, 256, 0, st>>>(hidden, hidden_in, hidden_out, n, out);
  else if (dtype == SI_DT_F16) reuse_apply<SI_DT_F16><<<g, 256, 0, st>>>(hidden, hidden_in, hidden_out, n, out);
  else reuse_apply<SI_DT_F32><<<g, 256, 0, st>>>(hidden, hidden_in, hidden_out, n, out);
  return check_launch("si_reuse_apply");
}
