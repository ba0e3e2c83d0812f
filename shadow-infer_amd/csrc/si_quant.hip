// Quantizer kernels (utils/quantization.py) and the INT8Linear quantization
// steps (ffn_optimizer/int8_linear.py) for gfx950.
#include "si_common.h"

namespace si {
namespace {

unsigned grid_for(int64_t items, int per_block, int64_t cap = 262144) {
  int64_t b = ceil_div(items, per_block);
  return (unsigned)(b < 1 ? 1 : (b > cap ? cap : b));
}

__device__ __forceinline__ float wave_amax(float m) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) m = amax_fold(m, __shfl_xor(m, off, 64));
  return m;
}

// Block-wide |max| for a 256-thread block (4 waves).
__device__ __forceinline__ float block_amax(float m, float* lds) {
  m = wave_amax(m);
  if ((threadIdx.x & 63) == 0) lds[threadIdx.x >> 6] = m;
  __syncthreads();
  float r = lds[0];
  for (int w = 1; w < 4; ++w) r = amax_fold(r, lds[w]);
  __syncthreads();
  return r;
}

// s = T(amax / div), 0 -> 1, then q = clamp(rint(T(x / s)), lo, hi).
__device__ __forceinline__ float q_scale(float amax, float div, int dt) {
  const float s = round_to(amax / div, dt);
  return s == 0.0f ? 1.0f : s;
}

__device__ __forceinline__ int8_t q_value(float x, float s, int dt, float lo, float hi) {
  float q = rintf(round_to(x / s, dt));
  q = fminf(fmaxf(q, lo), hi);
  return (int8_t)(int)q;
}

// One wavefront per row (utils/quantization.py:138-141).
__global__ __launch_bounds__(256) void quant_rows_i8_kernel(const void* __restrict__ x, int dt,
                                                            int64_t rows, int64_t D,
                                                            int8_t* __restrict__ q,
                                                            void* __restrict__ scale) {
  const int lane = threadIdx.x & 63;
  const int64_t step = (int64_t)gridDim.x * (blockDim.x / 64);
  for (int64_t r = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) / 64; r < rows; r += step) {
    float m = 0.0f;
    for (int64_t d = lane; d < D; d += 64) m = amax_fold(m, load_any(x, dt, r * D + d));
    m = wave_amax(m);
    const float s = q_scale(m, 127.0f, dt);
    if (lane == 0) store_any(scale, dt, r, s);
    for (int64_t d = lane; d < D; d += 64)
      q[r * D + d] = q_value(load_any(x, dt, r * D + d), s, dt, -128.0f, 127.0f);
  }
}

// One thread per (row, group) (utils/quantization.py:173-177).
__global__ __launch_bounds__(256) void quant_rows_i4_kernel(const void* __restrict__ x, int dt,
                                                            int64_t rows, int64_t D, int64_t g,
                                                            int8_t* __restrict__ q,
                                                            void* __restrict__ scale) {
  const int64_t G = D / g;
  const int64_t total = rows * G;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total;
       i += (int64_t)gridDim.x * blockDim.x) {
    const int64_t base = i * g;  // (row, group) blocks are contiguous
    float m = 0.0f;
    for (int64_t d = 0; d < g; ++d) m = amax_fold(m, load_any(x, dt, base + d));
    const float s = q_scale(m, 7.0f, dt);
    store_any(scale, dt, i, s);
    for (int64_t d = 0; d < g; ++d) q[base + d] = q_value(load_any(x, dt, base + d), s, dt, -8.0f, 7.0f);
  }
}

// One thread per output byte (packed_kv_cache.py:381-387).
__global__ __launch_bounds__(256) void int4_pack_kernel(const int8_t* __restrict__ q, int64_t rows,
                                                        int64_t L, uint8_t* __restrict__ out) {
  const int64_t rb = (L + 1) / 2;
  const int64_t total = rows * rb;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total;
       i += (int64_t)gridDim.x * blockDim.x) {
    const int64_t r = i / rb;
    const int64_t j = i - r * rb;
    const uint32_t hi = (uint32_t)(q[r * L + 2 * j] + 8) & 0xffu;
    const uint32_t lo = (2 * j + 1 < L) ? ((uint32_t)(q[r * L + 2 * j + 1] + 8) & 0xffu) : 0u;
    out[i] = (uint8_t)(((hi << 4) & 0xffu) | (lo & 0x0fu));
  }
}

__global__ __launch_bounds__(256) void int4_unpack_kernel(const uint8_t* __restrict__ in,
                                                          int64_t rows, int64_t rb, int64_t L,
                                                          int8_t* __restrict__ out) {
  const int64_t total = rows * L;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total;
       i += (int64_t)gridDim.x * blockDim.x) {
    const int64_t r = i / L;
    const int64_t j = i - r * L;
    const uint32_t b = in[r * rb + j / 2];
    const int nib = (j & 1) ? (int)(b & 0xfu) : (int)((b >> 4) & 0xfu);
    out[i] = (int8_t)(nib - 8);
  }
}

__global__ __launch_bounds__(256) void dequant_rows_kernel(const int8_t* __restrict__ q,
                                                           const void* __restrict__ scale, int sdt,
                                                           int64_t rows, int64_t D, int64_t g,
                                                           float* __restrict__ out) {
  const int64_t total = rows * D;
  const int64_t G = D / g;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total;
       i += (int64_t)gridDim.x * blockDim.x) {
    const int64_t r = i / D;
    const int64_t d = i - r * D;
    out[i] = (float)q[i] * load_any(scale, sdt, r * G + d / g);
  }
}

// ---------------------------------------------------------------------------
// INT8Linear: per-row activation quantization (int8_linear.py:96-98).
//   s = max(fp32(amax) / 127, 1e-8); q = clamp(rint(fp32(x) / s), -127, 127)
// One 256-thread block per row; 16-byte loads when K allows.
// ---------------------------------------------------------------------------

__global__ __launch_bounds__(256) void act_quant_kernel(const void* __restrict__ x, int dt,
                                                        int64_t M, int64_t K,
                                                        int8_t* __restrict__ q,
                                                        float* __restrict__ scale) {
  __shared__ float lds[4];
  const float eps = 1e-8f;
  for (int64_t m = blockIdx.x; m < M; m += gridDim.x) {
    float a = 0.0f;
    for (int64_t k = threadIdx.x; k < K; k += blockDim.x) a = amax_fold(a, load_any(x, dt, m * K + k));
    a = block_amax(a, lds);
    float s = a / 127.0f;
    s = s < eps ? eps : s;  // clamp_min(1e-8); NaN passes through like torch
    if (threadIdx.x == 0) scale[m] = s;
    for (int64_t k = threadIdx.x; k < K; k += blockDim.x) {
      float v = rintf(load_any(x, dt, m * K + k) / s);
      v = fminf(fmaxf(v, -127.0f), 127.0f);
      q[m * K + k] = (int8_t)(int)v;
    }
  }
}

// INT8Linear.from_linear (int8_linear.py:70-74), step 1: per-output-channel
// scale s[n] = max(amax_k |w[n,k]| / 127, 1e-8). One block per row of w.
__global__ __launch_bounds__(256) void weight_scale_kernel(const float* __restrict__ w, int64_t N,
                                                           int64_t K, float* __restrict__ scale) {
  __shared__ float lds[4];
  const float eps = 1e-8f;
  for (int64_t n = blockIdx.x; n < N; n += gridDim.x) {
    float a = 0.0f;
    for (int64_t k = threadIdx.x; k < K; k += blockDim.x) a = amax_fold(a, w[n * K + k]);
    a = block_amax(a, lds);
    if (threadIdx.x == 0) {
      const float s = a / 127.0f;
      scale[n] = s < eps ? eps : s;
    }
  }
}

// Step 2: q = clamp(rint(w / s), -127, 127) in the [N, K] layout of w.
__global__ __launch_bounds__(256) void weight_quant_kernel(const float* __restrict__ w, int64_t N,
                                                           int64_t K,
                                                           const float* __restrict__ scale,
                                                           int8_t* __restrict__ q) {
  const int64_t total = N * K;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total;
       i += (int64_t)gridDim.x * blockDim.x) {
    float r = rintf(w[i] / scale[i / K]);
    r = fminf(fmaxf(r, -127.0f), 127.0f);
    q[i] = (int8_t)(int)r;
  }
}

}  // namespace
}  // namespace si

using namespace si;

extern "C" int si_quant_rows_i8(const void* x, int dtype, int64_t rows, int64_t D, int8_t* q,
                                void* scale, si_stream_t stream) {
  clear_error();
  SI_CHECK_ARG(dtype_ok(dtype), "si_quant_rows_i8: unsupported dtype %d", dtype);
  SI_CHECK_ARG(rows >= 0 && D >= 0, "si_quant_rows_i8: bad shape");
  if (rows == 0 || D == 0) return SI_OK;
  SI_CHECK_ARG(x && q && scale, "si_quant_rows_i8: NULL argument");
  quant_rows_i8_kernel<<<grid_for(rows * 64, 256), 256, 0, as_stream(stream)>>>(x, dtype, rows, D,
                                                                               q, scale);
  return check_launch("si_quant_rows_i8");
}

extern "C" int si_quant_rows_i4(const void* x, int dtype, int64_t rows, int64_t D, int64_t group,
                                int8_t* q, void* scale, si_stream_t stream) {
  clear_error();
  SI_CHECK_ARG(dtype_ok(dtype), "si_quant_rows_i4: unsupported dtype %d", dtype);
  SI_CHECK_ARG(rows >= 0 && D >= 0, "si_quant_rows_i4: bad shape");
  SI_CHECK_ARG(group > 0 && D % group == 0,
               "si_quant_rows_i4: last dim %lld must be divisible by group_size %lld",
               (long long)D, (long long)group);
  if (rows == 0 || D == 0) return SI_OK;
  SI_CHECK_ARG(x && q && scale, "si_quant_rows_i4: NULL argument");
  quant_rows_i4_kernel<<<grid_for(rows * (D / group), 256), 256, 0, as_stream(stream)>>>(
      x, dtype, rows, D, group, q, scale);
  return check_launch("si_quant_rows_i4");
}

extern "C" int si_int4_pack_rows(const int8_t* q, int64_t rows, int64_t L, uint8_t* out,
                                 si_stream_t stream) {
  clear_error();
  SI_CHECK_ARG(rows >= 0 && L >= 0, "si_int4_pack_rows: bad shape");
  if (rows == 0 || L == 0) return SI_OK;
  SI_CHECK_ARG(q && out, "si_int4_pack_rows: NULL argument");
  int4_pack_kernel<<<grid_for(rows * ((L + 1) / 2), 256), 256, 0, as_stream(stream)>>>(q, rows, L,
                                                                                      out);
  return check_launch("si_int4_pack_rows");
}

extern "C" int si_int4_unpack_rows(const uint8_t* in, int64_t rows, int64_t row_bytes, int64_t L,
                                   int8_t* out, si_stream_t stream) {
  clear_error();
  SI_CHECK_ARG(rows >= 0 && L >= 0 && row_bytes >= 0, "si_int4_unpack_rows: bad shape");
  SI_CHECK_ARG(2 * row_bytes >= L, "si_int4_unpack_rows: %lld bytes per row hold fewer than %lld codes",
               (long long)row_bytes, (long long)L);
  if (rows == 0 || L == 0) return SI_OK;
  SI_CHECK_ARG(in && out, "si_int4_unpack_rows: NULL argument");
  int4_unpack_kernel<<<grid_for(rows * L, 256), 256, 0, as_stream(stream)>>>(in, rows, row_bytes, L,
                                                                            out);
  return check_launch("si_int4_unpack_rows");
}

extern "C" int si_dequant_rows(const int8_t* q, const void* scale, int scale_dtype, int64_t rows,
                               int64_t D, int64_t group, float* out, si_stream_t stream) {
  clear_error();
  SI_CHECK_ARG(dtype_ok(scale_dtype), "si_dequant_rows: unsupported scale dtype %d", scale_dtype);
  SI_CHECK_ARG(rows >= 0 && D >= 0, "si_dequant_rows: bad shape");
  SI_CHECK_ARG(group > 0 && (D == 0 || D % group == 0), "si_dequant_rows: group must divide D");
  if (rows == 0 || D == 0) return SI_OK;
  SI_CHECK_ARG(q && scale && out, "si_dequant_rows: NULL argument");
  dequant_rows_kernel<<<grid_for(rows * D, 256), 256, 0, as_stream(stream)>>>(
      q, scale, scale_dtype, rows, D, group, out);
  return check_launch("si_dequant_rows");
}

// Vector form of act_quant_kernel for rows of K % 8 == 0 elements (16-byte
// aligned rows, K <= 2048 * R): one block per row, the row held in registers
// (R chunks of 8 values per thread), 16-byte loads and 8-byte int8 stores.
// Same arithmetic: amax, s = max(amax / 127, 1e-8), q = clamp(rint(x / s), +-127)
// with the IEEE quotient, here Markstein's: q0 = x * RN(1/s), e = x - q0 * s
// (exact, one fma), RN(q0 + e * RN(1/s)) = RN(x / s) -- no division per value
// (checked against the division over every bf16 and fp16 row value and 10^8
// fp32 ones, tests/native/step_quotient_check.c).
template <int DT, int R>
__global__ __launch_bounds__(256) void act_quant_vec(const void* __restrict__ x, int64_t M, int K,
                                                      int8_t* __restrict__ q,
                                                      float* __restrict__ scale) {
  __shared__ float lds[4];
  const float eps = 1e-8f;
  const int nch = K / 8;
  for (int64_t m = blockIdx.x; m < M; m += gridDim.x) {
    float v[R][8];
    float a = 0.0f;
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const int c = (int)threadIdx.x + r * 256;
#pragma unroll
      for (int e = 0; e < 8; ++e) v[r][e] = 0.0f;
      if (c < nch) {
        const int64_t base = m * K + (int64_t)c * 8;
        if constexpr (DT == SI_DT_F32) {
          const float4 lo = reinterpret_cast<const float4*>(reinterpret_cast<const float*>(x) + base)[0];
          const float4 hi = reinterpret_cast<const float4*>(reinterpret_cast<const float*>(x) + base)[1];
          v[r][0] = lo.x; v[r][1] = lo.y; v[r][2] = lo.z; v[r][3] = lo.w;
          v[r][4] = hi.x; v[r][5] = hi.y; v[r][6] = hi.z; v[r][7] = hi.w;
        } else {
          const uint4 w = *reinterpret_cast<const uint4*>(reinterpret_cast<const uint16_t*>(x) + base);
          const uint32_t ws[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            if constexpr (DT == SI_DT_BF16) {
              v[r][2 * e] = bf16_bits_to_f32(ws[e] & 0xffffu);
              v[r][2 * e + 1] = bf16_bits_to_f32(ws[e] >> 16);
            } else {
              v[r][2 * e] = f16_bits_to_f32(ws[e] & 0xffffu);
              v[r][2 * e + 1] = f16_bits_to_f32(ws[e] >> 16);
            }
          }
        }
#pragma unroll
        for (int e = 0; e < 8; ++e) a = amax_fold(a, v[r][e]);
      }
    }
    a = block_amax(a, lds);
    float s = a / 127.0f;
    s = s < eps ? eps : s;  // clamp_min(1e-8); NaN passes through like torch
    if (threadIdx.x == 0) scale[m] = s;
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
      *reinterpret_cast<uint2*>(q + m * K + (int64_t)c * 8) = make_uint2(b[0], b[1]);
    }
  }
}

template <int DT>
void launch_act_quant_vec(const void* x, int64_t M, int K, int8_t* q, float* scale, unsigned grid,
                          hipStream_t st) {
  if (K <= 2048) act_quant_vec<DT, 1><<<grid, 256, 0, st>>>(x, M, K, q, scale);
  else if (K <= 4096) act_quant_vec<DT, 2><<<grid, 256, 0, st>>>(x, M, K, q, scale);
  else act_quant_vec<DT, 4><<<grid, 256, 0, st>>>(x, M, K, q, scale);
}

extern "C" int si_act_quant_i8(const void* x, int dtype, int64_t M, int64_t K, int8_t* q,
                               float* scale, si_stream_t stream) {
  clear_error();
  SI_CHECK_ARG(dtype_ok(dtype), "si_act_quant_i8: unsupported dtype %d", dtype);
  SI_CHECK_ARG(M >= 0 && K > 0, "si_act_quant_i8: bad shape");
  if (M == 0) return SI_OK;
  SI_CHECK_ARG(x && q && scale, "si_act_quant_i8: NULL argument");
  const unsigned grid = (unsigned)(M < 65536 ? M : 65536);
  const size_t esz = dtype == SI_DT_F32 ? 4 : 2;
  const bool vec = K % 8 == 0 && K <= 8192 && (reinterpret_cast<uintptr_t>(x) & 15) == 0 &&
                   (reinterpret_cast<uintptr_t>(q) & 7) == 0 && ((size_t)K * esz) % 16 == 0;
  hipStream_t st = as_stream(stream);
  if (!vec) {
    act_quant_kernel<<<grid, 256, 0, st>>>(x, dtype, M, K, q, scale);
  } else if (dtype == SI_DT_BF16) {
    launch_act_quant_vec<SI_DT_BF16>(x, M, (int)K, q, scale, grid, st);
  } else if (dtype == SI_DT_F16) {
    launch_act_quant_vec<SI_DT_F16>(x, M, (int)K, q, scale, grid, st);
  } else {
    launch_act_quant_vec<SI_DT_F32>(x, M, (int)K, q, scale, grid, st);
  }
  return check_launch("si_act_quant_i8");
}

extern "C" int si_weight_quant_i8(const float* w, int64_t N, int64_t K, int8_t* qweight,
                                  float* scale, si_stream_t stream) {
  clear_error();
  SI_CHECK_ARG(N > 0 && K > 0, "si_weight_quant_i8: bad shape");
  SI_CHECK_ARG(w && qweight && scale, "si_weight_quant_i8: NULL argument");
  hipStream_t st = as_stream(stream);
  weight_scale_kernel<<<(unsigned)(N < 65536 ? N : 65536), 256, 0, st>>>(w, N, K, scale);
  if (int rc = check_launch("si_weight_quant_i8/scale")) return rc;
  weight_quant_kernel<<<grid_for(N * K, 256), 256, 0, st>>>(w, N, K, scale, qweight);
  return check_launch("si_weight_quant_i8/quant");
}
