// Shared helpers for the gfx950 kernels of libshadowinfer_hip.so.
//
// Numerics policy: the library is compiled with -ffp-contract=off and
// correctly rounded fp32 division, so every expression rounds exactly as
// written; fused multiply-adds appear only where a kernel calls fmaf itself.
#pragma once

#include <hip/hip_runtime.h>
#include <hip/hip_fp16.h>
#include <stdint.h>
#include <stdio.h>

#include "../../include/shadowinfer_hip.h"

namespace si {

// ---- error reporting -------------------------------------------------------

void set_error(const char* fmt, ...) __attribute__((format(printf, 1, 2)));
void clear_error();

#define SI_CHECK_ARG(cond, ...)             \
  do {                                      \
    if (!(cond)) {                          \
      ::si::set_error(__VA_ARGS__);         \
      return SI_ERR_INVALID;                \
    }                                       \
  } while (0)

// Checks the launch that was just enqueued.
int check_launch(const char* what);

inline hipStream_t as_stream(si_stream_t s) { return reinterpret_cast<hipStream_t>(s); }

inline int64_t ceil_div(int64_t a, int64_t b) { return (a + b - 1) / b; }

inline bool dtype_ok(int dt) { return dt == SI_DT_F32 || dt == SI_DT_F16 || dt == SI_DT_BF16; }

inline int dtype_size(int dt) { return dt == SI_DT_F32 ? 4 : 2; }

// ---- scalar conversions (device) -------------------------------------------

// Workgroups are dispatched round-robin over the 8 XCDs (linear id b goes to
// XCD b % 8). xcd_order renumbers a grid of n workgroups so that each XCD
// receives a contiguous run of ids, in dispatch order; consecutive ids that
// read the same data then share one L2.
__device__ __forceinline__ int xcd_order(int b, int n) {
  constexpr int X = 8;
  const int per = (n + X - 1) / X;     // ids on each of the first `tall` XCDs
  const int tall = n - (per - 1) * X;  // 1..8
  const int x = b % X, j = b / X;
  return x < tall ? x * per + j : tall * per + (x - tall) * (per - 1) + j;
}

__device__ __forceinline__ float bf16_bits_to_f32(uint32_t h) {
  return __uint_as_float(h << 16);
}

// fp32 -> bf16 bits, round to nearest even; NaN -> 0x7FC0 (torch's bf16
// NaN). gfx950's v_cvt_pk_bf16_f32 rounds to nearest even exactly like the
// bit arithmetic u + 0x7FFF + ((u >> 16) & 1), >> 16 on every non-NaN fp32
// pattern (denormals and infinities included; si_check_bf16_convert compares
// all 2^32 patterns on the device); it keeps a NaN's sign and payload, so NaN
// is mapped to 0x7FC0 here.
__device__ __forceinline__ uint32_t f32_to_bf16_bits(float f) {
  const uint32_t h = (uint32_t)__builtin_bit_cast(unsigned short, (__bf16)f);
  return f != f ? 0x7fc0u : h;
}

// Two values at once, a in the low half (one v_cvt_pk_bf16_f32).
__device__ __forceinline__ uint32_t f32x2_to_bf16x2_bits(float a, float b) {
  typedef __bf16 bf2_t __attribute__((ext_vector_type(2)));
  typedef float f2_t __attribute__((ext_vector_type(2)));
  const f2_t v = {a, b};
  uint32_t w = __builtin_bit_cast(uint32_t, __builtin_convertvector(v, bf2_t));
  if (a != a) w = (w & 0xffff0000u) | 0x7fc0u;
  if (b != b) w = (w & 0x0000ffffu) | 0x7fc00000u;
  return w;
}

// Same rounding without the NaN test, for values known to be finite.
__device__ __forceinline__ float round_bf16_finite(float f) {
  const uint32_t h = (uint32_t)__builtin_bit_cast(unsigned short, (__bf16)f);
  return __uint_as_float(h << 16);
}

__device__ __forceinline__ float f16_bits_to_f32(uint32_t h) {
  return (float)__ushort_as_half((unsigned short)h);
}

// fp32 -> fp16 bits with the hardware conversion (round to nearest even).
__device__ __forceinline__ uint32_t f32_to_f16_bits(float f) {
  return (uint32_t)__half_as_ushort(__float2half_rn(f));
}

// Element access by dtype code for the generic (shape-agnostic) kernels.
__device__ __forceinline__ float load_any(const void* p, int dt, int64_t i) {
  if (dt == SI_DT_F32) return reinterpret_cast<const float*>(p)[i];
  uint32_t h = reinterpret_cast<const uint16_t*>(p)[i];
  return dt == SI_DT_F16 ? f16_bits_to_f32(h) : bf16_bits_to_f32(h);
}

__device__ __forceinline__ void store_any(void* p, int dt, int64_t i, float v) {
  if (dt == SI_DT_F32) {
    reinterpret_cast<float*>(p)[i] = v;
  } else {
    uint32_t h = dt == SI_DT_F16 ? f32_to_f16_bits(v) : f32_to_bf16_bits(v);
    reinterpret_cast<uint16_t*>(p)[i] = (uint16_t)h;
  }
}

// A pointer that is the same in every lane, read from lane 0 so that code
// built on it (a buffer descriptor) stays in scalar registers; the compiler
// cannot always prove such values uniform (a wave index from threadIdx.x), and
// a descriptor in vector registers costs a waterfall loop around every use.
// readfirstlane returns an int: each half goes through uint32_t, or a low
// half with bit 31 set would sign-extend over the high half.
__device__ __forceinline__ void* wave_uniform(const void* p) {
  const uint64_t v = reinterpret_cast<uint64_t>(p);
  const uint32_t hi = (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)(v >> 32));
  const uint32_t lo = (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)v);
  return reinterpret_cast<void*>(((uint64_t)hi << 32) | (uint64_t)lo);
}

// Round an fp32 value to dtype dt and widen back (identity for fp32).
__device__ __forceinline__ float round_to(float v, int dt) {
  if (dt == SI_DT_F32) return v;
  if (dt == SI_DT_F16) return f16_bits_to_f32(f32_to_f16_bits(v));
  return bf16_bits_to_f32(f32_to_bf16_bits(v));
}

// |v| folded into a running maximum; NaN propagates like torch's max.
__device__ __forceinline__ float amax_fold(float m, float v) {
  float a = fabsf(v);
  return (a != a || m != m) ? __uint_as_float(0x7fc00000u) : fmaxf(m, a);
}

}  // namespace si
