// Bucket access shared by the KV kernels and the fused packed attention.
#pragma once

#include "si_common.h"

namespace si {

struct Buckets {
  void* p[16];  // [4*prec + {0:k, 1:v, 2:scale_k, 3:scale_v}]
};

inline Buckets to_buckets(const void* const* p) {
  Buckets b;
  for (int i = 0; i < 16; ++i) b.p[i] = p ? const_cast<void*>(p[i]) : nullptr;
  return b;
}

template <int SDT>
__device__ __forceinline__ float load_scale(const void* p, int64_t i) {
  if (SDT == SI_DT_F32) return reinterpret_cast<const float*>(p)[i];
  const uint32_t h = reinterpret_cast<const uint16_t*>(p)[i];
  return SDT == SI_DT_F16 ? f16_bits_to_f32(h) : bf16_bits_to_f32(h);
}

// Four consecutive dequantized values (d0 .. d0+3) of batch row b of the entry
// at slot s in bucket c, tensor j (0 = k, 1 = v). Same arithmetic as
// unpack(): float(q) * float(scale) (utils/quantization.py:197, 217).
// Requires D % 4 == 0 and g % 4 == 0 (four values never straddle a group).
template <int SDT>
__device__ __forceinline__ float4 dequant4(const Buckets& bk, int j, int c, int64_t s, int64_t b,
                                           int64_t d0, int64_t B, int64_t D, int64_t g) {
  const int64_t orow = s * B + b;
  const int64_t el = orow * D + d0;
  if (c == SI_PREC_FP32) {
    return *reinterpret_cast<const float4*>(reinterpret_cast<const float*>(bk.p[j]) + el);
  }
  if (c == SI_PREC_FP16) {
    const uint2 w = *reinterpret_cast<const uint2*>(reinterpret_cast<const uint16_t*>(bk.p[4 + j]) + el);
    return make_float4(f16_bits_to_f32(w.x & 0xffffu), f16_bits_to_f32(w.x >> 16),
                       f16_bits_to_f32(w.y & 0xffffu), f16_bits_to_f32(w.y >> 16));
  }
  if (c == SI_PREC_INT8) {
    const uint32_t w = *reinterpret_cast<const uint32_t*>(reinterpret_cast<const int8_t*>(bk.p[8 + j]) + el);
    const float sc = load_scale<SDT>(bk.p[10 + j], orow);
    return make_float4((float)(int8_t)(w & 0xffu) * sc, (float)(int8_t)((w >> 8) & 0xffu) * sc,
                       (float)(int8_t)((w >> 16) & 0xffu) * sc, (float)(int8_t)(w >> 24) * sc);
  }
  const int64_t rb = B * D / 2;
  const uint32_t w = *reinterpret_cast<const uint16_t*>(
      reinterpret_cast<const uint8_t*>(bk.p[12 + j]) + s * rb + (b * D + d0) / 2);
  const float sc = load_scale<SDT>(bk.p[14 + j], orow * (D / g) + d0 / g);
  return make_float4((float)((int)((w >> 4) & 0xfu) - 8) * sc, (float)((int)(w & 0xfu) - 8) * sc,
                     (float)((int)((w >> 12) & 0xfu) - 8) * sc,
                     (float)((int)((w >> 8) & 0xfu) - 8) * sc);
}

}  // namespace si
