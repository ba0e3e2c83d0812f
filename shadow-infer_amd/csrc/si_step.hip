// Row kernels of one denoising step of a Llama-shaped diffusion LM
// (models/diffusion_llama.py:311-393): RMSNorm fused with the INT8Linear
// activation quantization, RoPE with the q/k/v head split, SwiGLU fused with
// the down projection's activation quantization, and the per-position argmax /
// confidence of the unmasking schedule (execution/block_decoding.py:148-151).
// Every row kernel holds its row in registers: one read of HBM per element.
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
// (int8_linear.py:96-98): s = max(amax / 127, 1e-8), q = clamp(rint(x / s), +-127),
// IEEE division, as si_act_quant_i8.
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
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const int c = (int)threadIdx.x + r * 256;
    if (c >= nch) continue;
    uint32_t b[2] = {0u, 0u};
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      float t = rintf(v[r][e] / s);
      t = fminf(fmaxf(t, -127.0f), 127.0f);
      b[e >> 2] |= ((uint32_t)(int)t & 0xffu) << (8 * (e & 3));
    }
    *reinterpret_cast<uint2*>(q + row * K + (int64_t)c * 8) = make_uint2(b[0], b[1]);
  }
}

// ---------------------------------------------------------------------------
// RMSNorm (DiffusionLlamaRMSNorm, diffusion_llama.py:311-321) over rows of K:
//   y = T((x * (1 / sqrt(mean(x^2) + eps))) * w)
// with the mean of squares in fp32 (one rounding to T at the end). Optional
// outputs: y [M, K] in T, and the INT8Linear quantization of y (q int8 [M, K],
// scale fp32 [M]) -- the input of a quantized projection, bit-identical to
// si_act_quant_i8 on y. One block per row, the row in registers (K <= 2048 R).
// ---------------------------------------------------------------------------
template <int DT, int R>
__global__ __launch_bounds__(256) void rmsnorm_rows(const void* __restrict__ x,
                                                    const void* __restrict__ w, int64_t M, int K,
                                                    float eps, void* __restrict__ y,
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
#pragma unroll
        for (int e = 0; e < 8; ++e) ss += v[r][e] * v[r][e];
      } else {
#pragma unroll
        for (int e = 0; e < 8; ++e) v[r][e] = 0.0f;
      }
    }
    ss = block_sum(ss, lds);
    const float inv = 1.0f / sqrtf(ss / (float)K + eps);
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const int c = (int)threadIdx.x + r * 256;
      if (c >= nch) continue;
      float wv[8];
      load8<DT>(w, (int64_t)c * 8, wv);
#pragma unroll
      for (int e = 0; e < 8; ++e) v[r][e] = round_to((v[r][e] * inv) * wv[e], DT);
      if (y != nullptr) store8<DT>(y, m * K + (int64_t)c * 8, v[r]);
    }
    if (q != nullptr) quant_row<R>(v, nch, m, K, q, scale, lds);
  }
}

// ---------------------------------------------------------------------------
// RoPE + head split (DiffusionLlamaAttention.forward, diffusion_llama.py:362-373):
// qkv [B*S, 3*H*D] (q | k | v column blocks, each [H, D]) ->
// q, k, v [B, H, S, D], q and k rotated:
//   out[d]       = T(x[d] cos[s,d] - x[d+D/2] sin[s,d])
//   out[d+D/2]   = T(x[d+D/2] cos[s,d+D/2] + x[d] sin[s,d+D/2])    (d < D/2)
// with the cos/sin tables [S, D] in T (the reference's emb = cat(freqs, freqs)
// cast to the parameter dtype) and fp32 arithmetic, one rounding.
// A thread owns 8 dims of the first half and their 8 partners.
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
#pragma unroll
    for (int part = 0; part < 2; ++part) {
      float x0[8], x1[8], y0[8], y1[8];
      load8<DT>(qkv, in + part * H * D, x0);
      load8<DT>(qkv, in + part * H * D + HALF, x1);
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        y0[e] = round_to(x0[e] * c0[e] - x1[e] * s0[e], DT);
        y1[e] = round_to(x1[e] * c1[e] + x0[e] * s1[e], DT);
      }
      void* dst = part == 0 ? qo : ko;
      store8<DT>(dst, out, y0);
      store8<DT>(dst, out + HALF, y1);
    }
    float v0[8], v1[8];
    load8<DT>(qkv, in + 2 * H * D, v0);
    load8<DT>(qkv, in + 2 * H * D + HALF, v1);
    store8<DT>(vo, out, v0);
    store8<DT>(vo, out + HALF, v1);
  }
}

// ---------------------------------------------------------------------------
// SwiGLU + down-projection input quantization (DiffusionLlamaMLP.forward,
// diffusion_llama.py:332-333; the down INT8Linear prologue int8_linear.py:96-98):
// gu [M, 2F] holds gate | up; h = T(T(silu(g)) * u), silu(g) = g / (1 + exp(-g))
// in fp32 (torch's two elementwise ops, each rounded to T). Writes h [M, F]
// (optional) and its INT8Linear quantization q int8 [M, F], scale fp32 [M].
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
        float g[8], u[8];
        load8<DT>(gu, m * 2 * F + (int64_t)c * 8, g);
        load8<DT>(gu, m * 2 * F + F + (int64_t)c * 8, u);
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          float sg;
          if constexpr (DT == SI_DT_F32) {
            sg = g[e] / (1.0f + expf(-g[e]));
          } else {
            // g / (1 + exp(-g)) with v_exp_f32 and v_rcp_f32: a few fp32 ulps from
            // the correctly rounded quotient, below half a bf16/fp16 ulp, before
            // the rounding to T
            const float ex = __builtin_amdgcn_exp2f(-g[e] * 1.44269504088896341f);
            sg = round_to(g[e] * __builtin_amdgcn_rcpf(1.0f + ex), DT);
          }
          v[r][e] = round_to(sg * u[e], DT);
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
// Per-position argmax and confidence (schedule_round, block_decoding.py:148-151):
// tok[m] = the first index of the largest logit (a NaN counts as largest),
// conf[m] = max softmax probability = 1 / sum_v exp(l_v - l_max), in fp32.
// One block per row, one pass: each thread keeps its best (value, index) and
// the sum of exp(l - its running max), rescaled when the max grows; partial
// results merge by the same rule. 16-byte loads when rows allow.
// ---------------------------------------------------------------------------
__device__ __forceinline__ bool beats(float a, int64_t ia, float b, int64_t ib) {
  const bool na = a != a, nb = b != b;
  if (na || nb) return na && (!nb || ia < ib);
  return a > b || (a == b && ia < ib);
}

struct ArgSum {
  float m;     // running max (NaN once a NaN was seen)
  int64_t i;   // its first index
  float s;     // sum of exp(l - m)
};

__device__ __forceinline__ void arg_add(ArgSum& a, float x, int64_t i) {
  if (beats(x, i, a.m, a.i)) {
    if (x != a.m) a.s = a.m == -INFINITY ? 0.0f : a.s * expf(a.m - x);
    a.m = x;
    a.i = i;
  }
  a.s += x == -INFINITY ? 0.0f : expf(x - a.m);
}

__device__ __forceinline__ void arg_merge(ArgSum& a, const ArgSum& b) {
  const float m = beats(b.m, b.i, a.m, a.i) ? b.m : a.m;
  const float sa = a.m == -INFINITY ? 0.0f : a.s * expf(a.m - m);
  const float sb = b.m == -INFINITY ? 0.0f : b.s * expf(b.m - m);
  if (beats(b.m, b.i, a.m, a.i)) a.i = b.i;
  a.m = m;
  a.s = sa + sb;
}

template <int DT, bool VEC>
__global__ __launch_bounds__(256) void row_argmax_conf(const void* __restrict__ logits,
                                                       int64_t M, int64_t V,
                                                       int64_t* __restrict__ tok,
                                                       float* __restrict__ conf) {
  __shared__ float lm[4], ls[4];
  __shared__ int64_t li[4];
  for (int64_t m = blockIdx.x; m < M; m += gridDim.x) {
    ArgSum a{-INFINITY, INT64_MAX, 0.0f};
    if constexpr (VEC) {
      for (int64_t c = threadIdx.x; c < V / 8; c += blockDim.x) {
        float v[8];
        load8<DT>(logits, m * V + c * 8, v);
#pragma unroll
        for (int e = 0; e < 8; ++e) arg_add(a, v[e], c * 8 + e);
      }
    } else {
      for (int64_t v = threadIdx.x; v < V; v += blockDim.x) arg_add(a, load_any(logits, DT, m * V + v), v);
    }
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) {
      ArgSum b{__shfl_xor(a.m, off, 64), __shfl_xor(a.i, off, 64), __shfl_xor(a.s, off, 64)};
      arg_merge(a, b);
    }
    if ((threadIdx.x & 63) == 0) {
      lm[threadIdx.x >> 6] = a.m;
      li[threadIdx.x >> 6] = a.i;
      ls[threadIdx.x >> 6] = a.s;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
      ArgSum r{lm[0], li[0], ls[0]};
      for (int w = 1; w < 4; ++w) arg_merge(r, ArgSum{lm[w], li[w], ls[w]});
      tok[m] = r.i == INT64_MAX ? 0 : r.i;
      conf[m] = 1.0f / r.s;
    }
    __syncthreads();
  }
}

unsigned row_grid(int64_t M) { return (unsigned)(M < 262144 ? (M < 1 ? 1 : M) : 262144); }

template <int DT>
void launch_rmsnorm(const void* x, const void* w, int64_t M, int K, float eps, void* y, int8_t* q,
                    float* s, hipStream_t st) {
  const unsigned g = row_grid(M);
  if (K <= 2048) rmsnorm_rows<DT, 1><<<g, 256, 0, st>>>(x, w, M, K, eps, y, q, s);
  else if (K <= 4096) rmsnorm_rows<DT, 2><<<g, 256, 0, st>>>(x, w, M, K, eps, y, q, s);
  else if (K <= 8192) rmsnorm_rows<DT, 4><<<g, 256, 0, st>>>(x, w, M, K, eps, y, q, s);
  else rmsnorm_rows<DT, 8><<<g, 256, 0, st>>>(x, w, M, K, eps, y, q, s);
}

template <int DT>
void launch_swiglu(const void* gu, int64_t M, int F, void* h, int8_t* q, float* s, hipStream_t st) {
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

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

}  // namespace
}  // namespace si

using namespace si;

extern "C" int si_rmsnorm_rows(const void* x, int dtype, int64_t M, int64_t K, const void* weight,
                               float eps, void* y, int8_t* q, float* scale, si_stream_t stream) {
  clear_error();
  SI_CHECK_ARG(dtype == SI_DT_BF16 || dtype == SI_DT_F16 || dtype == SI_DT_F32,
               "si_rmsnorm_rows: unsupported dtype %d", dtype);
  SI_CHECK_ARG(M >= 0 && K > 0 && K % 8 == 0 && K <= 16384,
               "si_rmsnorm_rows: K must be a multiple of 8 in [8, 16384] (got %lld)", (long long)K);
  SI_CHECK_ARG((q == nullptr) == (scale == nullptr),
               "si_rmsnorm_rows: q and scale are given together");
  if (M == 0) return SI_OK;
  SI_CHECK_ARG(x && weight && (y || q), "si_rmsnorm_rows: NULL argument");
  SI_CHECK_ARG(aligned16(x) && aligned16(weight) && (!y || aligned16(y)) && (!q || (reinterpret_cast<uintptr_t>(q) & 7) == 0),
               "si_rmsnorm_rows: x, weight and y must be 16-byte aligned, q 8-byte aligned");
  hipStream_t st = as_stream(stream);
  if (dtype == SI_DT_BF16) launch_rmsnorm<SI_DT_BF16>(x, weight, M, (int)K, eps, y, q, scale, st);
  else if (dtype == SI_DT_F16) launch_rmsnorm<SI_DT_F16>(x, weight, M, (int)K, eps, y, q, scale, st);
  else launch_rmsnorm<SI_DT_F32>(x, weight, M, (int)K, eps, y, q, scale, st);
  return check_launch("si_rmsnorm_rows");
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
  SI_CHECK_ARG(qkv && cos_table && sin_table && q && k && v, "si_rope_split: NULL argument");
  SI_CHECK_ARG(aligned16(qkv) && aligned16(cos_table) && aligned16(sin_table) && aligned16(q) &&
                   aligned16(k) && aligned16(v),
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
                                  int64_t* tokens, float* confidence, si_stream_t stream) {
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
