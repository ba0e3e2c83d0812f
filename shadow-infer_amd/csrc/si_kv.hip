// Packed KV cache kernels for gfx950: pack, unpack, reuse copy, compaction.
//
// Row geometry. An entry e = t*H + h (token-major) owns, for each batch index
// b, the input row K[b, h, t, :] of D values; in memory that is row
// r = (b*H + h)*S + t of the [B*H*S, D] view. Inside a bucket the entry sits
// at `slot` (from the plan scan), its batch rows at bucket row slot*B + b.
// int4 entries keep the reference's per-entry byte row of ceil(B*D/2) bytes
// holding the B*D nibbles in (b, d) order (packed_kv_cache.py:367-388).
//
// Fast pack path: LPR lanes of one wavefront share a row; each lane owns one
// 16-byte chunk (8 bf16/fp16 or 4 fp32 values). Row and group maxima come from
// butterfly shuffles inside the LPR lanes, so int8 (per row) and int4 (per
// group) quantize with the same instruction stream; only the final stores
// differ by precision. Reads walk K/V in memory order and are coalesced.
#include <type_traits>

#include "si_kv_common.h"

namespace si {
namespace {



// ---------------------------------------------------------------------------
// Quantization arithmetic shared by the fast and generic paths.
// ---------------------------------------------------------------------------

// Quotient round(T(x / s)) of Quantizer.quantize_int8/int4
// (utils/quantization.py:141, 177) before clamping.
//  - fp32/fp16 inputs: correctly rounded division, then rounding to T.
//  - bf16 inputs with s >= 2^-100: x * r with r = RN(1/s), corrected by one
//    fma on the exact remainder (Markstein's theorem: for r = RN(1/s) and a
//    faithful q0, q0 + (x - q0*s)*r rounds to RN(x/s)). The identity with the
//    correctly rounded path, after bf16 rounding and rint, has been checked
//    exhaustively over every bf16 x and every bf16 s >= 2^-100 on the CPU.
template <int DT>
__device__ __forceinline__ float quant_quotient(float x, float s, float r, bool fast) {
  float q;
  if (DT == SI_DT_BF16) {
    if (fast) {
      const float q0 = x * r;
      const float e = __builtin_fmaf(-q0, s, x);
      q = __builtin_fmaf(e, r, q0);
    } else {
      q = x / s;
    }
    q = bf16_bits_to_f32(f32_to_bf16_bits(q));
  } else if (DT == SI_DT_F16) {
    q = f16_bits_to_f32(f32_to_f16_bits(x / s));
  } else {
    q = x / s;
  }
  return rintf(q);
}

// s = T(amax / div); s == 0 -> 1 (utils/quantization.py:138-140, 175-176).
template <int DT>
__device__ __forceinline__ float quant_scale(float amax, float div) {
  float s = amax / div;
  if (DT == SI_DT_BF16) s = bf16_bits_to_f32(f32_to_bf16_bits(s));
  if (DT == SI_DT_F16) s = f16_bits_to_f32(f32_to_f16_bits(s));
  return s == 0.0f ? 1.0f : s;
}

template <int DT>
__device__ __forceinline__ void store_scalar(void* p, int64_t i, float v) {
  if (DT == SI_DT_F32) {
    reinterpret_cast<float*>(p)[i] = v;
  } else {
    const uint32_t h = DT == SI_DT_F16 ? f32_to_f16_bits(v) : f32_to_bf16_bits(v);
    reinterpret_cast<uint16_t*>(p)[i] = (uint16_t)h;
  }
}

__device__ __forceinline__ float clampf(float v, float lo, float hi) {
  return fminf(fmaxf(v, lo), hi);
}

// ---------------------------------------------------------------------------
// 16-byte chunk loads: EPL values of dtype DT, widened to fp32.
// ---------------------------------------------------------------------------

template <int DT>
struct Chunk {
  static constexpr int EPL = DT == SI_DT_F32 ? 4 : 8;
};

template <int DT>
__device__ __forceinline__ void load_chunk(const void* base, int64_t elem, float* out) {
  typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
  const u32x4 raw = __builtin_nontemporal_load(
      reinterpret_cast<const u32x4*>(reinterpret_cast<const char*>(base) +
                                     elem * (DT == SI_DT_F32 ? 4 : 2)));
  const uint32_t w[4] = {raw[0], raw[1], raw[2], raw[3]};
  if (DT == SI_DT_F32) {
#pragma unroll
    for (int i = 0; i < 4; ++i) out[i] = __uint_as_float(w[i]);
  } else {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      if (DT == SI_DT_BF16) {
        out[2 * i] = __uint_as_float(w[i] << 16);
        out[2 * i + 1] = __uint_as_float(w[i] & 0xffff0000u);
      } else {
        out[2 * i] = f16_bits_to_f32(w[i] & 0xffffu);
        out[2 * i + 1] = f16_bits_to_f32(w[i] >> 16);
      }
    }
  }
}

template <int N>
__device__ __forceinline__ void store_f32(float* dst, const float* v) {
#pragma unroll
  for (int i = 0; i < N; i += 4)
    *reinterpret_cast<float4*>(dst + i) = make_float4(v[i], v[i + 1], v[i + 2], v[i + 3]);
}

template <int N>
__device__ __forceinline__ void store_f16(uint16_t* dst, const float* v) {
  uint32_t w[N / 2];
#pragma unroll
  for (int i = 0; i < N / 2; ++i)
    w[i] = f32_to_f16_bits(v[2 * i]) | (f32_to_f16_bits(v[2 * i + 1]) << 16);
  if constexpr (N == 8) {
    *reinterpret_cast<uint4*>(dst) = make_uint4(w[0], w[1], w[2], w[3]);
  } else {
    *reinterpret_cast<uint2*>(dst) = make_uint2(w[0], w[1]);
  }
}

// Bytes of N int8 codes.
template <int N>
__device__ __forceinline__ void store_i8(int8_t* dst, const float* q) {
  uint32_t w[N / 4];
#pragma unroll
  for (int i = 0; i < N / 4; ++i)
    w[i] = ((uint32_t)(int)q[4 * i] & 0xffu) | (((uint32_t)(int)q[4 * i + 1] & 0xffu) << 8) |
           (((uint32_t)(int)q[4 * i + 2] & 0xffu) << 16) |
           (((uint32_t)(int)q[4 * i + 3] & 0xffu) << 24);
  if constexpr (N == 8) {
    *reinterpret_cast<uint2*>(dst) = make_uint2(w[0], w[1]);
  } else {
    *reinterpret_cast<uint32_t*>(dst) = w[0];
  }
}

// N int4 codes -> N/2 bytes, high nibble first, nibble = code + 8.
template <int N>
__device__ __forceinline__ void store_i4(uint8_t* dst, const float* q) {
  uint32_t w = 0;
#pragma unroll
  for (int i = 0; i < N / 2; ++i) {
    const uint32_t hi = (uint32_t)((int)q[2 * i] + 8) & 0xfu;
    const uint32_t lo = (uint32_t)((int)q[2 * i + 1] + 8) & 0xfu;
    w |= ((hi << 4) | lo) << (8 * i);
  }
  if constexpr (N == 8) {
    *reinterpret_cast<uint32_t*>(dst) = w;
  } else {
    *reinterpret_cast<uint16_t*>(dst) = (uint16_t)w;
  }
}

// ---------------------------------------------------------------------------
// Dense working copy the pack can write in the same pass: the k/v tensors of
// ShadowKVAgent._compress_kv_with_plan (shadowinfer/shadowkv/
// shadowkv_agent.py:1698-1809), [B, H, S, D] in the input dtype. Per entry:
// fp32 -> the input values, fp16 -> the values rounded to fp16 and back,
// int8/int4 -> the integer codes (not dequantized), other codes -> 0; entries
// flagged in `reuse` take the rows of the previous K/V instead.
// ---------------------------------------------------------------------------
// Per-precision flat index lists (h*S + t in slot order, the plan's
// flat_indices) and the block ranges of a bucket-order launch.
struct UnpackLists {
  const int64_t* flat[4];
  int64_t n[4];
  int64_t blk_end[5];
};

struct WorkCopy {
  void* k;
  void* v;
  const void* kp;  // previous K/V, read for reuse entries only
  const void* vp;
  const uint8_t* reuse;  // [S*H] (token-major) or NULL
};

// ---------------------------------------------------------------------------
// Fast pack: D = EPL * LPR, int4 group = EPL * lpg (lpg | LPR, power of two).
// Grid: blockIdx.y = b*H + h, blockIdx.x = tile of RPP*U tokens; each thread
// keeps U rows in flight (loads issued before any row is quantized).
// ---------------------------------------------------------------------------

// Working-copy values of one chunk -> the 16 bytes of the input dtype.
template <int DT>
__device__ __forceinline__ void copy_words(const float* f, uint32_t* w) {
  if constexpr (DT == SI_DT_F32) {
#pragma unroll
    for (int i = 0; i < 4; ++i) w[i] = __float_as_uint(f[i]);
  } else {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const uint32_t a = DT == SI_DT_F16 ? f32_to_f16_bits(f[2 * i]) : f32_to_bf16_bits(f[2 * i]);
      const uint32_t b = DT == SI_DT_F16 ? f32_to_f16_bits(f[2 * i + 1]) : f32_to_bf16_bits(f[2 * i + 1]);
      w[i] = a | (b << 16);
    }
  }
}

template <int DT, int LPR, bool WC>
__device__ __forceinline__ void pack_row(const float* xk, const float* xv, int c, int s, int b,
                                         int B, int lane, int lpg, const Buckets& bk,
                                         uint32_t* ck, uint32_t* cv) {
  constexpr int EPL = Chunk<DT>::EPL;
  constexpr int D = EPL * LPR;
  const int64_t orow = (int64_t)s * B + b;
  const int64_t oel = orow * D + lane * EPL;
  if (c == SI_PREC_FP32) {
    store_f32<EPL>(reinterpret_cast<float*>(bk.p[0]) + oel, xk);
    store_f32<EPL>(reinterpret_cast<float*>(bk.p[1]) + oel, xv);
    if constexpr (WC) {
      copy_words<DT>(xk, ck);
      copy_words<DT>(xv, cv);
    }
    return;
  }
  if (c == SI_PREC_FP16) {
    store_f16<EPL>(reinterpret_cast<uint16_t*>(bk.p[4]) + oel, xk);
    store_f16<EPL>(reinterpret_cast<uint16_t*>(bk.p[5]) + oel, xv);
    if constexpr (WC) {
      float fk[EPL], fv[EPL];
#pragma unroll
      for (int i = 0; i < EPL; ++i) {
        fk[i] = f16_bits_to_f32(f32_to_f16_bits(xk[i]));
        fv[i] = f16_bits_to_f32(f32_to_f16_bits(xv[i]));
      }
      copy_words<DT>(fk, ck);
      copy_words<DT>(fv, cv);
    }
    return;
  }
  // int8 (per row) or int4 (per group): shared arithmetic.
  float gk = 0.0f, gv = 0.0f;
#pragma unroll
  for (int i = 0; i < EPL; ++i) {
    gk = amax_fold(gk, xk[i]);
    gv = amax_fold(gv, xv[i]);
  }
  for (int off = 1; off < lpg; off <<= 1) {
    gk = amax_fold(gk, __shfl_xor(gk, off, 64));
    gv = amax_fold(gv, __shfl_xor(gv, off, 64));
  }
  float mk = gk, mv = gv;
#pragma unroll
  for (int off = 1; off < LPR; off <<= 1) {
    if (off >= lpg) {
      mk = amax_fold(mk, __shfl_xor(mk, off, 64));
      mv = amax_fold(mv, __shfl_xor(mv, off, 64));
    }
  }
  const bool i8 = (c == SI_PREC_INT8);
  const float sk = quant_scale<DT>(i8 ? mk : gk, i8 ? 127.0f : 7.0f);
  const float sv = quant_scale<DT>(i8 ? mv : gv, i8 ? 127.0f : 7.0f);
  const bool fk = sk >= 7.8886090522101181e-31f;  // 2^-100
  const bool fv = sv >= 7.8886090522101181e-31f;
  const float rk = 1.0f / sk;
  const float rv = 1.0f / sv;
  const float lo = i8 ? -128.0f : -8.0f;
  const float hi = i8 ? 127.0f : 7.0f;
  float qk[EPL], qv[EPL];
#pragma unroll
  for (int i = 0; i < EPL; ++i) {
    qk[i] = clampf(quant_quotient<DT>(xk[i], sk, rk, fk), lo, hi);
    qv[i] = clampf(quant_quotient<DT>(xv[i], sv, rv, fv), lo, hi);
  }
  if constexpr (WC) {
    float fk2[EPL], fv2[EPL];
#pragma unroll
    for (int i = 0; i < EPL; ++i) {
      fk2[i] = qk[i] + 0.0f;  // the integer code as a value (-0 -> +0)
      fv2[i] = qv[i] + 0.0f;
    }
    copy_words<DT>(fk2, ck);
    copy_words<DT>(fv2, cv);
  }
  if (i8) {
    store_i8<EPL>(reinterpret_cast<int8_t*>(bk.p[8]) + oel, qk);
    store_i8<EPL>(reinterpret_cast<int8_t*>(bk.p[9]) + oel, qv);
    if (lane == 0) {
      store_scalar<DT>(bk.p[10], orow, sk);
      store_scalar<DT>(bk.p[11], orow, sv);
    }
  } else {
    const int64_t rb = (int64_t)B * D / 2;  // int4 bytes per entry (D even)
    const int64_t boff = (int64_t)s * rb + ((int64_t)b * D + lane * EPL) / 2;
    store_i4<EPL>(reinterpret_cast<uint8_t*>(bk.p[12]) + boff, qk);
    store_i4<EPL>(reinterpret_cast<uint8_t*>(bk.p[13]) + boff, qv);
    if ((lane & (lpg - 1)) == 0) {
      const int64_t si = orow * (LPR / lpg) + lane / lpg;
      store_scalar<DT>(bk.p[14], si, sk);
      store_scalar<DT>(bk.p[15], si, sv);
    }
  }
}

// ---------------------------------------------------------------------------
// bf16 fast path. Same results as pack_row<SI_DT_BF16> with fewer VALU
// instructions per element (the pack kernel is VALU-bound):
//  * |x| maxima on raw bf16 bit patterns with packed 16-bit integer max (the
//    abs bit patterns order like the values; NaN patterns order above inf, so
//    a NaN still wins), butterflies inside 16-lane rows by DPP;
//  * scale = bf16(amax / d) by q0 = amax*RN(1/d) plus one fma correction, and
//    the element quotient by r = RN(1/s) plus one fma correction; both equal
//    correctly rounded division after the bf16 rounding and round-to-integer
//    that follow (checked exhaustively over all bf16 inputs by
//    tests/native/quotient_check.c);
//  * clamp, then add 1.5*2^23: the add rounds to an integer (ties to even) and
//    the low bits of the sum are the two's-complement code.
// ---------------------------------------------------------------------------

typedef unsigned short u16x2 __attribute__((ext_vector_type(2)));

__device__ __forceinline__ uint32_t max_abs_bf16x8(const uint32_t w[4]) {
  u16x2 a = __builtin_bit_cast(u16x2, w[0] & 0x7fff7fffu);
  u16x2 b = __builtin_bit_cast(u16x2, w[1] & 0x7fff7fffu);
  u16x2 c = __builtin_bit_cast(u16x2, w[2] & 0x7fff7fffu);
  u16x2 d = __builtin_bit_cast(u16x2, w[3] & 0x7fff7fffu);
  const u16x2 m = __builtin_elementwise_max(__builtin_elementwise_max(a, b),
                                            __builtin_elementwise_max(c, d));
  return (uint32_t)(m.x > m.y ? m.x : m.y);
}

// v = max(v, v of lane ^ OFF) for a butterfly inside aligned groups of lanes.
// OFF 1/2 are quad permutes; OFF 4/8 use the half-row / row mirrors, which pair
// the same groups once the previous steps made each sub-group uniform.
template <int OFF>
__device__ __forceinline__ uint32_t bfly_max(uint32_t v) {
  int o;
  if constexpr (OFF == 1) o = __builtin_amdgcn_update_dpp(0, (int)v, 0xB1, 0xF, 0xF, false);
  else if constexpr (OFF == 2) o = __builtin_amdgcn_update_dpp(0, (int)v, 0x4E, 0xF, 0xF, false);
  else if constexpr (OFF == 4) o = __builtin_amdgcn_update_dpp(0, (int)v, 0x141, 0xF, 0xF, false);
  else if constexpr (OFF == 8) o = __builtin_amdgcn_update_dpp(0, (int)v, 0x140, 0xF, 0xF, false);
  else o = __shfl_xor((int)v, OFF, 64);
  return v > (uint32_t)o ? v : (uint32_t)o;
}

// Row maximum over LPR lanes; *grp receives the maximum over groups of lpg lanes.
template <int LPR>
__device__ __forceinline__ uint32_t row_group_max(uint32_t v, int lpg, uint32_t* grp) {
  uint32_t g = v;
  if constexpr (LPR > 1) { v = bfly_max<1>(v); if (lpg == 2) g = v; }
  if constexpr (LPR > 2) { v = bfly_max<2>(v); if (lpg == 4) g = v; }
  if constexpr (LPR > 4) { v = bfly_max<4>(v); if (lpg == 8) g = v; }
  if constexpr (LPR > 8) { v = bfly_max<8>(v); if (lpg == 16) g = v; }
  if constexpr (LPR > 16) { v = bfly_max<16>(v); if (lpg == 32) g = v; }
  if constexpr (LPR > 32) { v = bfly_max<32>(v); }
  if (lpg == LPR) g = v;
  *grp = g;
  return v;
}

// bf16(amax / d) with 0 -> 1; h = abs bf16 bits of amax.
__device__ __forceinline__ float bf16_scale(uint32_t h, float d, float rd) {
  const float a = __uint_as_float(h << 16);
  float q;
  if (h < 0x7f80u) {
    const float q0 = a * rd;
    q = __builtin_fmaf(__builtin_fmaf(-q0, d, a), rd, q0);
  } else {
    q = a / d;  // inf or NaN amax
  }
  const float s = bf16_bits_to_f32(f32_to_bf16_bits(q));
  return s == 0.0f ? 1.0f : s;
}

constexpr float kMagic = 12582912.0f;  // 1.5 * 2^23

// Integer code (as the low bits of the returned word) of one bf16 value x.
__device__ __forceinline__ uint32_t quant_bf16(float x, float s, float r, bool fast, float lo,
                                               float hi) {
  float q;
  if (fast) {
    const float q0 = x * r;
    q = round_bf16_finite(__builtin_fmaf(__builtin_fmaf(-q0, s, x), r, q0));
  } else {
    q = bf16_bits_to_f32(f32_to_bf16_bits(x / s));
  }
  q = __builtin_amdgcn_fmed3f(q, lo, hi);
  return __float_as_uint(q + kMagic);
}

// Low bytes of four words -> one word.
__device__ __forceinline__ uint32_t bytes4(uint32_t a, uint32_t b, uint32_t c, uint32_t d) {
  const uint32_t lo = __builtin_amdgcn_perm(b, a, 0x0c0c0400u);
  const uint32_t hi = __builtin_amdgcn_perm(d, c, 0x0c0c0400u);
  return __builtin_amdgcn_perm(hi, lo, 0x05040100u);
}

// Two integer codes (words from quant_bf16) -> their bf16 values in one word.
__device__ __forceinline__ uint32_t codes_bf16x2(uint32_t q0, uint32_t q1) {
  const uint32_t a = __float_as_uint(__uint_as_float(q0) - kMagic) >> 16;  // exact in bf16
  const uint32_t b = __float_as_uint(__uint_as_float(q1) - kMagic) & 0xffff0000u;
  return a | b;
}

// Bucket row stores of the bf16 pack. Token order (rows of a block anywhere
// in the bucket): plain stores. Bucket order: device-scope (sc1) buffer
// stores from the block's first row, which write the lines through as they
// leave: 7B layer, headline protocol, pack 40.8 -> 39.0 us, and an unpack
// right after the pack as fast as before (55.0 us). A non-temporal store made
// the pack as fast but pushed the buckets out of the last-level cache, so an
// unpack that follows the pack took 27% longer.
template <typename T>
__device__ __forceinline__ void st_row(void* p, T v) {
  *reinterpret_cast<T*>(p) = v;
}

typedef unsigned int u32x4_t __attribute__((ext_vector_type(4)));
typedef unsigned int u32x2_t __attribute__((ext_vector_type(2)));

// Raw buffer from byte `first` of a bucket (block-uniform); `off` is the
// byte offset from there (a block's rows span a few KB).
__device__ __forceinline__ __amdgpu_buffer_rsrc_t rows_rsrc(void* bucket, int64_t first) {
  return __builtin_amdgcn_make_buffer_rsrc(wave_uniform(reinterpret_cast<char*>(bucket) + first),
                                           (short)0, -1, 0x00020000);
}
__device__ __forceinline__ void st_dev(void* bucket, int64_t first, uint32_t off, u32x4_t v) {
  __builtin_amdgcn_raw_buffer_store_b128(v, rows_rsrc(bucket, first), (int)off, 0, 16);
}
__device__ __forceinline__ void st_dev(void* bucket, int64_t first, uint32_t off, u32x2_t v) {
  __builtin_amdgcn_raw_buffer_store_b64(v, rows_rsrc(bucket, first), (int)off, 0, 16);
}
__device__ __forceinline__ void st_dev(void* bucket, int64_t first, uint32_t off, uint32_t v) {
  __builtin_amdgcn_raw_buffer_store_b32(v, rows_rsrc(bucket, first), (int)off, 0, 16);
}

// DEV: bucket rows stored with st_dev relative to bucket row `row0` (the
// block's first row; every row of the block is at most a few KB past it).
template <int LPR, bool WC, bool DEV = false>
__device__ __forceinline__ void pack_row_bf16(const uint32_t wk[4], const uint32_t wv[4], int c,
                                              int s, int b, int B, int lane, int lpg,
                                              const Buckets& bk, uint32_t* ck, uint32_t* cv,
                                              int64_t row0 = 0) {
  constexpr int D = 8 * LPR;
  const int64_t orow = (int64_t)s * B + b;
  const int64_t oel = orow * D + lane * 8;
  const uint32_t rel = (uint32_t)((orow - row0) * D + lane * 8);  // element offset from row0
  if (c == SI_PREC_FP16 || c == SI_PREC_FP32) {
    float xk[8], xv[8];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      xk[2 * i] = __uint_as_float(wk[i] << 16);
      xk[2 * i + 1] = __uint_as_float(wk[i] & 0xffff0000u);
      xv[2 * i] = __uint_as_float(wv[i] << 16);
      xv[2 * i + 1] = __uint_as_float(wv[i] & 0xffff0000u);
    }
    if (c == SI_PREC_FP16) {
      typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
      u32x4 hk, hv;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        hk[i] = f32_to_f16_bits(xk[2 * i]) | (f32_to_f16_bits(xk[2 * i + 1]) << 16);
        hv[i] = f32_to_f16_bits(xv[2 * i]) | (f32_to_f16_bits(xv[2 * i + 1]) << 16);
      }
      if constexpr (DEV) {
        st_dev(bk.p[4], row0 * D * 2, rel * 2, hk);
        st_dev(bk.p[5], row0 * D * 2, rel * 2, hv);
      } else {
        st_row(reinterpret_cast<uint16_t*>(bk.p[4]) + oel, hk);
        st_row(reinterpret_cast<uint16_t*>(bk.p[5]) + oel, hv);
      }
      if constexpr (WC) {
        float fk[8], fv[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          fk[i] = f16_bits_to_f32(f32_to_f16_bits(xk[i]));
          fv[i] = f16_bits_to_f32(f32_to_f16_bits(xv[i]));
        }
        copy_words<SI_DT_BF16>(fk, ck);
        copy_words<SI_DT_BF16>(fv, cv);
      }
    } else {
      store_f32<8>(reinterpret_cast<float*>(bk.p[0]) + oel, xk);
      store_f32<8>(reinterpret_cast<float*>(bk.p[1]) + oel, xv);
      if constexpr (WC) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          ck[i] = wk[i];
          cv[i] = wv[i];
        }
      }
    }
    return;
  }
  uint32_t gk, gv;
  const uint32_t mk = row_group_max<LPR>(max_abs_bf16x8(wk), lpg, &gk);
  const uint32_t mv = row_group_max<LPR>(max_abs_bf16x8(wv), lpg, &gv);
  const bool i8 = (c == SI_PREC_INT8);
  const float d = i8 ? 127.0f : 7.0f;
  const float rd = i8 ? 0.0078740157186985016f : 0.14285714924335480f;  // RN(1/d)
  const float sk = bf16_scale(i8 ? mk : gk, d, rd);
  const float sv = bf16_scale(i8 ? mv : gv, d, rd);
  const bool fk = sk >= 7.8886090522101181e-31f && sk < 3.0e38f;
  const bool fv = sv >= 7.8886090522101181e-31f && sv < 3.0e38f;
  const float rk = 1.0f / sk;
  const float rv = 1.0f / sv;
  const float lo = i8 ? -128.0f : -8.0f;
  const float hi = i8 ? 127.0f : 7.0f;
  uint32_t qk[8], qv[8];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    qk[2 * i] = quant_bf16(__uint_as_float(wk[i] << 16), sk, rk, fk, lo, hi);
    qk[2 * i + 1] = quant_bf16(__uint_as_float(wk[i] & 0xffff0000u), sk, rk, fk, lo, hi);
    qv[2 * i] = quant_bf16(__uint_as_float(wv[i] << 16), sv, rv, fv, lo, hi);
    qv[2 * i + 1] = quant_bf16(__uint_as_float(wv[i] & 0xffff0000u), sv, rv, fv, lo, hi);
  }
  if constexpr (WC) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      ck[i] = codes_bf16x2(qk[2 * i], qk[2 * i + 1]);
      cv[i] = codes_bf16x2(qv[2 * i], qv[2 * i + 1]);
    }
  }
  if (i8) {
    const u32x2_t k8{bytes4(qk[0], qk[1], qk[2], qk[3]), bytes4(qk[4], qk[5], qk[6], qk[7])};
    const u32x2_t v8{bytes4(qv[0], qv[1], qv[2], qv[3]), bytes4(qv[4], qv[5], qv[6], qv[7])};
    if constexpr (DEV) {
      st_dev(bk.p[8], row0 * D, rel, k8);
      st_dev(bk.p[9], row0 * D, rel, v8);
    } else {
      st_row(reinterpret_cast<int8_t*>(bk.p[8]) + oel, k8);
      st_row(reinterpret_cast<int8_t*>(bk.p[9]) + oel, v8);
    }
    if (lane == 0) {
      reinterpret_cast<uint16_t*>(bk.p[10])[orow] = (uint16_t)(__float_as_uint(sk) >> 16);
      reinterpret_cast<uint16_t*>(bk.p[11])[orow] = (uint16_t)(__float_as_uint(sv) >> 16);
    }
  } else {
    // Byte = ((q0 & 0xF) << 4 | (q1 & 0xF)) ^ 0x88: the two's-complement nibble
    // with its top bit flipped is the offset-binary nibble q + 8.
    uint32_t bkk[4], bvv[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      bkk[j] = __builtin_amdgcn_ubfe(qk[2 * j], 0, 4) << 4 | __builtin_amdgcn_ubfe(qk[2 * j + 1], 0, 4);
      bvv[j] = __builtin_amdgcn_ubfe(qv[2 * j], 0, 4) << 4 | __builtin_amdgcn_ubfe(qv[2 * j + 1], 0, 4);
    }
    const int64_t rb = (int64_t)B * D / 2;
    const int64_t boff = (int64_t)s * rb + ((int64_t)b * D + lane * 8) / 2;
    const uint32_t k4 = bytes4(bkk[0], bkk[1], bkk[2], bkk[3]) ^ 0x88888888u;
    const uint32_t v4 = bytes4(bvv[0], bvv[1], bvv[2], bvv[3]) ^ 0x88888888u;
    if constexpr (DEV) {  // D even: row r's int4 bytes start at r * D / 2
      st_dev(bk.p[12], row0 * (D / 2), rel / 2, k4);
      st_dev(bk.p[13], row0 * (D / 2), rel / 2, v4);
    } else {
      st_row(reinterpret_cast<uint8_t*>(bk.p[12]) + boff, k4);
      st_row(reinterpret_cast<uint8_t*>(bk.p[13]) + boff, v4);
    }
    if ((lane & (lpg - 1)) == 0) {
      const int64_t si = orow * (LPR / lpg) + lane / lpg;
      reinterpret_cast<uint16_t*>(bk.p[14])[si] = (uint16_t)(__float_as_uint(sk) >> 16);
      reinterpret_cast<uint16_t*>(bk.p[15])[si] = (uint16_t)(__float_as_uint(sv) >> 16);
    }
  }
}

// 16 bytes of the working copy at byte offset `off`: the computed chunk, or
// the previous K/V when the entry is reused.
template <bool WC>
__device__ __forceinline__ void store_copy(const WorkCopy& wc, int64_t off, bool reuse,
                                           uint32_t* ck, uint32_t* cv) {
  if constexpr (WC) {
    typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
    if (reuse) {
      const u32x4 a = *reinterpret_cast<const u32x4*>(reinterpret_cast<const char*>(wc.kp) + off);
      const u32x4 b = *reinterpret_cast<const u32x4*>(reinterpret_cast<const char*>(wc.vp) + off);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        ck[i] = a[i];
        cv[i] = b[i];
      }
    }
    __builtin_nontemporal_store(u32x4{ck[0], ck[1], ck[2], ck[3]},
                                reinterpret_cast<u32x4*>(reinterpret_cast<char*>(wc.k) + off));
    __builtin_nontemporal_store(u32x4{cv[0], cv[1], cv[2], cv[3]},
                                reinterpret_cast<u32x4*>(reinterpret_cast<char*>(wc.v) + off));
  }
}

template <int DT, int LPR, int U, bool WC>
__global__ __launch_bounds__(256) void kv_pack_fast(const void* __restrict__ kin,
                                                    const void* __restrict__ vin, int B, int H,
                                                    int S, int lpg, const int8_t* __restrict__ code,
                                                    const int32_t* __restrict__ slot,
                                                    Buckets bk, WorkCopy wc) {
  constexpr int EPL = Chunk<DT>::EPL;
  constexpr int D = EPL * LPR;
  constexpr int RPP = 256 / LPR;  // rows per pass of the block
  const int lane = threadIdx.x % LPR;
  const int sub = threadIdx.x / LPR;
  const int bh = blockIdx.y;
  const int h = bh % H;
  const int b = bh / H;
  const int t0 = blockIdx.x * (RPP * U) + sub;
  const int64_t row0 = (int64_t)bh * S;
  int c[U], s[U];
  bool ru[U];  // reused entry (working copy only)
  if constexpr (DT == SI_DT_BF16) {
    typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
    uint32_t wk[U][4], wv[U][4];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int t = t0 + u * RPP;
      c[u] = SI_PREC_EVICTED;
      s[u] = 0;
      ru[u] = false;
      if (t < S) {
        const int e = t * H + h;
        const int64_t off = ((row0 + t) * D + lane * EPL) * 2;
        const u32x4 a = __builtin_nontemporal_load(
            reinterpret_cast<const u32x4*>(reinterpret_cast<const char*>(kin) + off));
        const u32x4 bb = __builtin_nontemporal_load(
            reinterpret_cast<const u32x4*>(reinterpret_cast<const char*>(vin) + off));
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          wk[u][i] = a[i];
          wv[u][i] = bb[i];
        }
        c[u] = code[e];
        s[u] = slot[e];
        ru[u] = WC && wc.reuse != nullptr && wc.reuse[e] != 0;
      }
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      uint32_t ck[4] = {0u, 0u, 0u, 0u}, cv[4] = {0u, 0u, 0u, 0u};
      if (c[u] >= 0 && c[u] <= 3)
        pack_row_bf16<LPR, WC>(wk[u], wv[u], c[u], s[u], b, B, lane, lpg, bk, ck, cv);
      if (WC && t0 + u * RPP < S)
        store_copy<WC>(wc, ((row0 + t0 + u * RPP) * D + lane * EPL) * 2, ru[u], ck, cv);
    }
  } else {
    float xk[U][EPL], xv[U][EPL];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int t = t0 + u * RPP;
      c[u] = SI_PREC_EVICTED;
      s[u] = 0;
      ru[u] = false;
      if (t < S) {
        const int e = t * H + h;
        load_chunk<DT>(kin, (row0 + t) * D + lane * EPL, xk[u]);
        load_chunk<DT>(vin, (row0 + t) * D + lane * EPL, xv[u]);
        c[u] = code[e];
        s[u] = slot[e];
        ru[u] = WC && wc.reuse != nullptr && wc.reuse[e] != 0;
      }
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      uint32_t ck[4] = {0u, 0u, 0u, 0u}, cv[4] = {0u, 0u, 0u, 0u};
      if (c[u] >= 0 && c[u] <= 3)
        pack_row<DT, LPR, WC>(xk[u], xv[u], c[u], s[u], b, B, lane, lpg, bk, ck, cv);
      if (WC && t0 + u * RPP < S)
        store_copy<WC>(wc, ((row0 + t0 + u * RPP) * D + lane * EPL) * (DT == SI_DT_F32 ? 4 : 2),
                       ru[u], ck, cv);
    }
  }
}

// K/V rows taken from a q|k|v projection instead of dense [B, H, S, D]
// tensors: row (b, h, t) of K is qkv[(b*S + t), H*D + h*D .. +D] with RoPE
// applied, row (b, h, t) of V is qkv[(b*S + t), 2*H*D + h*D .. +D] as it is.
// cos/sin: [S, D] tables in the K/V dtype.
struct RopeSrc {
  const void* qkv;
  const void* cos;
  const void* sin;
  int S;
  int H;
};

// RoPE on the EPL values of this lane's chunk of a K row (the reference's
// q * cos + rotate_half(q) * sin in the row dtype T, each product rounded to
// T, then the sum; the same arithmetic as rope_split): lanes of the first
// half of the row take the partner value x[d + D/2] from lane ^ (LPR/2),
// subtract its product with sin[d]; lanes of the second half add x[d - D/2]
// times sin[d]. Every lane of the row group must call it (cross-lane reads).
template <int DT, int LPR>
__device__ __forceinline__ void rope_chunk(float* x, int64_t t, int lane, const RopeSrc& rs) {
  static_assert(DT == SI_DT_BF16 || DT == SI_DT_F16, "16-bit rows");
  constexpr int EPL = Chunk<DT>::EPL;
  constexpr int D = EPL * LPR;
  float xp[EPL], c[EPL], sn[EPL];
#pragma unroll
  for (int e = 0; e < EPL; ++e) xp[e] = __shfl_xor(x[e], LPR / 2, 64);
  // 16-byte loads of the table chunks (reused by every head: plain loads stay in L2)
  const int64_t el = t * D + lane * EPL;
  const uint4 cw = *reinterpret_cast<const uint4*>(reinterpret_cast<const uint16_t*>(rs.cos) + el);
  const uint4 sw = *reinterpret_cast<const uint4*>(reinterpret_cast<const uint16_t*>(rs.sin) + el);
  const uint32_t cws[4] = {cw.x, cw.y, cw.z, cw.w}, sws[4] = {sw.x, sw.y, sw.z, sw.w};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    c[2 * i] = DT == SI_DT_BF16 ? bf16_bits_to_f32(cws[i] & 0xffffu) : f16_bits_to_f32(cws[i] & 0xffffu);
    c[2 * i + 1] = DT == SI_DT_BF16 ? bf16_bits_to_f32(cws[i] >> 16) : f16_bits_to_f32(cws[i] >> 16);
    sn[2 * i] = DT == SI_DT_BF16 ? bf16_bits_to_f32(sws[i] & 0xffffu) : f16_bits_to_f32(sws[i] & 0xffffu);
    sn[2 * i + 1] = DT == SI_DT_BF16 ? bf16_bits_to_f32(sws[i] >> 16) : f16_bits_to_f32(sws[i] >> 16);
  }
  const bool first = lane < LPR / 2;
#pragma unroll
  for (int e = 0; e < EPL; ++e) {
    const float a = round_to(x[e] * c[e], DT);
    const float b = round_to(xp[e] * sn[e], DT);
    x[e] = round_to(first ? a - b : a + b, DT);
  }
}

// Pack in bucket order: block x takes RPP*U consecutive rows (entry, b) of
// one precision's bucket (the flat index lists give each row's dense row
// b*H*S + h*S + t), so every wave quantizes a single precision and the bucket
// rows are written contiguously. blk_end[p]: first block after precision p's.
// Element offsets of this lane's K and V chunks of row (bb, flat = h*S + t):
// dense [B, H, S, D] tensors, or the q|k|v projection rows with ROPE (t is
// then returned for the cos/sin tables).
template <bool ROPE, int D, int EPL>
__device__ __forceinline__ void row_offsets(int64_t bb, int64_t flat, int64_t HS, int lane,
                                            const RopeSrc& rs, int64_t& koff, int64_t& voff,
                                            int64_t& t) {
  if constexpr (ROPE) {
    const int64_t h = flat / rs.S;
    t = flat - h * rs.S;
    koff = ((bb * rs.S + t) * 3 * rs.H + rs.H + h) * D + lane * EPL;
    voff = koff + (int64_t)rs.H * D;
  } else {
    koff = voff = (bb * HS + flat) * D + lane * EPL;
    t = 0;
  }
}

template <int DT, int LPR, int U, int P, int NT, bool ROPE>
__device__ __forceinline__ void pack_bucket_rows(const void* __restrict__ kin,
                                                 const void* __restrict__ vin,
                                                 const UnpackLists& L, int64_t lb, int B,
                                                 int64_t HS, int lpg, const Buckets& bk,
                                                 const RopeSrc& rs) {
  constexpr int EPL = Chunk<DT>::EPL;
  constexpr int D = EPL * LPR;
  constexpr int RPP = NT / LPR;
  const int lane = threadIdx.x % LPR;
  const int64_t rows = L.n[P] * B;
  const int64_t r0 = lb * (RPP * U) + threadIdx.x / LPR;
  if (ROPE) {
    kin = rs.qkv;
    vin = rs.qkv;
  }
  if constexpr (DT == SI_DT_BF16) {
    typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
    uint32_t wk[U][4], wv[U][4];
    int64_t sl[U], bb[U], tk[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int64_t r = r0 + u * RPP;
      sl[u] = -1;
      tk[u] = 0;
      if constexpr (ROPE) {  // rows past the end still take part in the lane exchange
#pragma unroll
        for (int i = 0; i < 4; ++i) wk[u][i] = wv[u][i] = 0u;
      }
      if (r < rows) {
        sl[u] = r / B;
        bb[u] = r - sl[u] * B;
        int64_t ko, vo;
        row_offsets<ROPE, D, EPL>(bb[u], L.flat[P][sl[u]], HS, lane, rs, ko, vo, tk[u]);
        const u32x4 a = __builtin_nontemporal_load(
            reinterpret_cast<const u32x4*>(reinterpret_cast<const char*>(kin) + ko * 2));
        const u32x4 b = __builtin_nontemporal_load(
            reinterpret_cast<const u32x4*>(reinterpret_cast<const char*>(vin) + vo * 2));
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          wk[u][i] = a[i];
          wv[u][i] = b[i];
        }
      }
    }
    if constexpr (ROPE) {
#pragma unroll
      for (int u = 0; u < U; ++u) {
        float x[8];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          x[2 * i] = bf16_bits_to_f32(wk[u][i] & 0xffffu);
          x[2 * i + 1] = bf16_bits_to_f32(wk[u][i] >> 16);
        }
        rope_chunk<DT, LPR>(x, tk[u], lane, rs);
#pragma unroll
        for (int i = 0; i < 4; ++i)
          wk[u][i] = f32x2_to_bf16x2_bits(x[2 * i], x[2 * i + 1]);
      }
    }
#pragma unroll
    for (int u = 0; u < U; ++u)
      if (sl[u] >= 0)
        pack_row_bf16<LPR, false, true>(wk[u], wv[u], P, (int)sl[u], (int)bb[u], B, lane, lpg, bk,
                                        nullptr, nullptr, lb * (RPP * U));
  } else {
    float xk[U][EPL], xv[U][EPL];
    int64_t sl[U], bb[U], tk[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int64_t r = r0 + u * RPP;
      sl[u] = -1;
      tk[u] = 0;
      if constexpr (ROPE) {
#pragma unroll
        for (int e = 0; e < EPL; ++e) xk[u][e] = xv[u][e] = 0.0f;
      }
      if (r < rows) {
        sl[u] = r / B;
        bb[u] = r - sl[u] * B;
        int64_t ko, vo;
        row_offsets<ROPE, D, EPL>(bb[u], L.flat[P][sl[u]], HS, lane, rs, ko, vo, tk[u]);
        load_chunk<DT>(kin, ko, xk[u]);
        load_chunk<DT>(vin, vo, xv[u]);
      }
    }
    if constexpr (ROPE) {
#pragma unroll
      for (int u = 0; u < U; ++u) rope_chunk<DT, LPR>(xk[u], tk[u], lane, rs);
    }
#pragma unroll
    for (int u = 0; u < U; ++u)
      if (sl[u] >= 0)
        pack_row<DT, LPR, false>(xk[u], xv[u], P, (int)sl[u], (int)bb[u], B, lane, lpg, bk,
                                 nullptr, nullptr);
  }
}

template <int DT, int LPR, int U, int NT, bool ROPE = false>
__global__ __launch_bounds__(NT) void kv_pack_lists(const void* __restrict__ kin,
                                                     const void* __restrict__ vin, UnpackLists L,
                                                     int B, int H, int S, int lpg, Buckets bk,
                                                     RopeSrc rs = RopeSrc{}) {
  const int64_t blk = blockIdx.x;
  const int64_t HS = (int64_t)H * S;
  if (blk < L.blk_end[0]) {
    pack_bucket_rows<DT, LPR, U, SI_PREC_FP32, NT, ROPE>(kin, vin, L, blk, B, HS, lpg, bk, rs);
  } else if (blk < L.blk_end[1]) {
    pack_bucket_rows<DT, LPR, U, SI_PREC_FP16, NT, ROPE>(kin, vin, L, blk - L.blk_end[0], B, HS,
                                                         lpg, bk, rs);
  } else if (blk < L.blk_end[2]) {
    pack_bucket_rows<DT, LPR, U, SI_PREC_INT8, NT, ROPE>(kin, vin, L, blk - L.blk_end[1], B, HS,
                                                         lpg, bk, rs);
  } else {
    pack_bucket_rows<DT, LPR, U, SI_PREC_INT4, NT, ROPE>(kin, vin, L, blk - L.blk_end[2], B, HS,
                                                         lpg, bk, rs);
  }
}

// ---------------------------------------------------------------------------
// Generic pack: one thread per entry, any B, D, group (odd sizes included).
// ---------------------------------------------------------------------------

template <int DT>
__device__ void pack_entry_generic(const void* in, int64_t B, int64_t H, int64_t S, int64_t D,
                                   int64_t g, int64_t t, int64_t h, int c, int64_t s,
                                   void* data, void* scale, void* copy) {
  const int64_t L = B * D;
  const int64_t rb = (L + 1) / 2;
  const int64_t G = D / g;
  uint32_t pending = 0;
  for (int64_t b = 0; b < B; ++b) {
    const int64_t src = ((b * H + h) * S + t) * D;
    const int64_t orow = s * B + b;
    if (c == SI_PREC_FP32 || c == SI_PREC_FP16) {
      for (int64_t d = 0; d < D; ++d) {
        const float x = load_any(in, DT, src + d);
        store_any(data, c == SI_PREC_FP32 ? SI_DT_F32 : SI_DT_F16, orow * D + d, x);
        if (copy != nullptr)
          store_any(copy, DT, src + d, c == SI_PREC_FP32 ? x : f16_bits_to_f32(f32_to_f16_bits(x)));
      }
      continue;
    }
    const bool i8 = (c == SI_PREC_INT8);
    const int64_t gs = i8 ? D : g;
    for (int64_t g0 = 0; g0 < D; g0 += gs) {
      float m = 0.0f;
      for (int64_t d = 0; d < gs; ++d) m = amax_fold(m, load_any(in, DT, src + g0 + d));
      const float sc = quant_scale<DT>(m, i8 ? 127.0f : 7.0f);
      store_scalar<DT>(scale, i8 ? orow : orow * G + g0 / g, sc);
      for (int64_t d = 0; d < gs; ++d) {
        const float x = load_any(in, DT, src + g0 + d);
        const float q = clampf(quant_quotient<DT>(x, sc, 0.0f, false), i8 ? -128.0f : -8.0f,
                               i8 ? 127.0f : 7.0f);
        if (copy != nullptr) store_any(copy, DT, src + g0 + d, q + 0.0f);
        if (i8) {
          reinterpret_cast<int8_t*>(data)[orow * D + g0 + d] = (int8_t)(int)q;
        } else {
          const int64_t j = b * D + g0 + d;  // nibble index in the entry row
          const uint32_t nib = (uint32_t)((int)q + 8) & 0xfu;
          if ((j & 1) == 0) {
            pending = nib << 4;
          } else {
            reinterpret_cast<uint8_t*>(data)[s * rb + j / 2] = (uint8_t)(pending | nib);
          }
        }
      }
    }
  }
  if (c == SI_PREC_INT4 && (L & 1)) reinterpret_cast<uint8_t*>(data)[s * rb + L / 2] =
      (uint8_t)pending;
}

template <int DT>
__global__ __launch_bounds__(256) void kv_pack_generic(const void* __restrict__ kin,
                                                       const void* __restrict__ vin, int64_t B,
                                                       int64_t H, int64_t S, int64_t D,
                                                       int64_t g, const int8_t* __restrict__ code,
                                                       const int32_t* __restrict__ slot,
                                                       Buckets bk, WorkCopy wc) {
  const int64_t n = S * H;
  for (int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; e < n;
       e += (int64_t)gridDim.x * blockDim.x) {
    const int c = code[e];
    const int64_t t = e / H;
    const int64_t h = e - t * H;
    const bool packed = c >= 0 && c <= 3;
    if (packed) {
      const int64_t s = slot[e];
      pack_entry_generic<DT>(kin, B, H, S, D, g, t, h, c, s, bk.p[4 * c + 0], bk.p[4 * c + 2],
                             wc.k);
      pack_entry_generic<DT>(vin, B, H, S, D, g, t, h, c, s, bk.p[4 * c + 1], bk.p[4 * c + 3],
                             wc.v);
    }
    if (wc.k == nullptr) continue;
    const bool reuse = wc.reuse != nullptr && wc.reuse[e] != 0;
    if (!reuse && packed) continue;
    // Working copy of a reused (previous K/V) or unpacked (zero) entry.
    for (int64_t b = 0; b < B; ++b) {
      const int64_t src = ((b * H + h) * S + t) * D;
      for (int64_t d = 0; d < D; ++d) {
        store_any(wc.k, DT, src + d, reuse ? load_any(wc.kp, DT, src + d) : 0.0f);
        store_any(wc.v, DT, src + d, reuse ? load_any(wc.vp, DT, src + d) : 0.0f);
      }
    }
  }
}

// ---------------------------------------------------------------------------
// Unpack (packed_kv_cache.py:535-577): every output element is written.
// ---------------------------------------------------------------------------

// Dequantized value d of batch row b of the entry at `s` in bucket c.
__device__ __forceinline__ float dequant_one(const Buckets& bk, int j, int c, int64_t s,
                                             int64_t b, int64_t d, int64_t B, int64_t D,
                                             int64_t g, int sdt) {
  const int64_t orow = s * B + b;
  if (c == SI_PREC_FP32) return reinterpret_cast<const float*>(bk.p[j])[orow * D + d];
  if (c == SI_PREC_FP16)
    return f16_bits_to_f32(reinterpret_cast<const uint16_t*>(bk.p[4 + j])[orow * D + d]);
  if (c == SI_PREC_INT8)
    return (float)reinterpret_cast<const int8_t*>(bk.p[8 + j])[orow * D + d] *
           load_any(bk.p[10 + j], sdt, orow);
  const int64_t rb = (B * D + 1) / 2;
  const int64_t nib_idx = b * D + d;
  const uint32_t byte = reinterpret_cast<const uint8_t*>(bk.p[12 + j])[s * rb + nib_idx / 2];
  const int nib = (nib_idx & 1) ? (int)(byte & 0xfu) : (int)((byte >> 4) & 0xfu);
  return (float)(nib - 8) * load_any(bk.p[14 + j], sdt, orow * (D / g) + d / g);
}

__global__ __launch_bounds__(256) void kv_unpack_generic(const int8_t* __restrict__ code,
                                                         const int32_t* __restrict__ slot,
                                                         Buckets bk, int sdt, int64_t B, int64_t H,
                                                         int64_t S, int64_t D, int64_t g,
                                                         float* __restrict__ ok,
                                                         float* __restrict__ ov) {
  const int64_t total = B * H * S * D;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total;
       i += (int64_t)gridDim.x * blockDim.x) {
    const int64_t d = i % D;
    const int64_t row = i / D;
    const int64_t t = row % S;
    const int64_t bh = row / S;
    const int64_t h = bh % H;
    const int64_t b = bh / H;
    const int64_t e = t * H + h;
    const int c = code[e];
    float vk = 0.0f, vv = 0.0f;
    if (c >= 0 && c <= 3) {
      const int64_t s = slot[e];
      vk = dequant_one(bk, 0, c, s, b, d, B, D, g, sdt);
      vv = dequant_one(bk, 1, c, s, b, d, B, D, g, sdt);
    }
    ok[i] = vk;
    ov[i] = vv;
  }
}

// Unpack for D in {64, 128}: blockIdx.y = b*H + h, blockIdx.x = tile of
// RPP*U tokens; each thread dequantizes one 4-value chunk of U rows (all loads
// issued before the stores) and writes 16-byte non-temporal stores.
// Unpack of a 64-token tile of one (b, h), rows sorted by precision in LDS:
// the tile's codes and slots are loaded once, one wave ranks the tokens per
// code with ballots, and the block then decodes the rows in that order, so
// runs of one precision share a wave while the tile's output (64 rows of D
// floats, contiguous) is written with 16-byte stores.
template <int D, int SDT, int U>
__global__ __launch_bounds__(256) void kv_unpack_sorted(const int8_t* __restrict__ code,
                                                        const int32_t* __restrict__ slot,
                                                        Buckets bk, int B, int H, int S, int g,
                                                        float* __restrict__ ok,
                                                        float* __restrict__ ov) {
  constexpr int TT = 64;
  constexpr int CPR = D / 4;      // 16-byte chunks per row
  constexpr int RPP = 256 / CPR;  // rows per pass
  __shared__ int s_tok[TT];
  __shared__ int s_code[TT];
  __shared__ int s_slot[TT];
  const int bh = blockIdx.y;
  const int h = bh % H;
  const int b = bh / H;
  const int t0 = blockIdx.x * TT;
  const int nt = min(TT, S - t0);
  if (threadIdx.x < 64) {
    const int lane = threadIdx.x;
    int c = SI_PREC_EVICTED, sl = 0;
    if (lane < nt) {
      const int e = (t0 + lane) * H + h;
      c = code[e];
      if (c < 0 || c > 3) c = SI_PREC_EVICTED;
      else sl = slot[e];
    }
    const uint64_t below = (1ull << lane) - 1ull;
    int base = 0, pos = 0;
#pragma unroll
    for (int p = 0; p <= SI_PREC_EVICTED; ++p) {
      const uint64_t m = __ballot(lane < nt && c == p);
      if (c == p) pos = base + __popcll(m & below);
      base += __popcll(m);
    }
    if (lane < nt) {
      s_tok[pos] = lane;
      s_code[pos] = c;
      s_slot[pos] = sl;
    }
  }
  __syncthreads();
  const int ch = threadIdx.x % CPR;
  const int sub = threadIdx.x / CPR;
  const int64_t row0 = (int64_t)bh * S + t0;
  typedef float f32x4 __attribute__((ext_vector_type(4)));
  for (int i0 = 0; i0 < nt; i0 += RPP * U) {
    float4 rk[U], rv[U];
    int tk[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int i = i0 + u * RPP + sub;
      tk[u] = -1;
      rk[u] = make_float4(0.f, 0.f, 0.f, 0.f);
      rv[u] = rk[u];
      if (i < nt) {
        tk[u] = s_tok[i];
        const int c = s_code[i];
        const int sl = s_slot[i];
        if (c == SI_PREC_FP16) {
          rk[u] = dequant4<SDT>(bk, 0, SI_PREC_FP16, sl, b, ch * 4, B, D, g);
          rv[u] = dequant4<SDT>(bk, 1, SI_PREC_FP16, sl, b, ch * 4, B, D, g);
        } else if (c == SI_PREC_INT8) {
          rk[u] = dequant4<SDT>(bk, 0, SI_PREC_INT8, sl, b, ch * 4, B, D, g);
          rv[u] = dequant4<SDT>(bk, 1, SI_PREC_INT8, sl, b, ch * 4, B, D, g);
        } else if (c == SI_PREC_INT4) {
          rk[u] = dequant4<SDT>(bk, 0, SI_PREC_INT4, sl, b, ch * 4, B, D, g);
          rv[u] = dequant4<SDT>(bk, 1, SI_PREC_INT4, sl, b, ch * 4, B, D, g);
        } else if (c == SI_PREC_FP32) {
          rk[u] = dequant4<SDT>(bk, 0, SI_PREC_FP32, sl, b, ch * 4, B, D, g);
          rv[u] = dequant4<SDT>(bk, 1, SI_PREC_FP32, sl, b, ch * 4, B, D, g);
        }
      }
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      if (tk[u] >= 0) {
        const int64_t off = (row0 + tk[u]) * D + ch * 4;
        __builtin_nontemporal_store(f32x4{rk[u].x, rk[u].y, rk[u].z, rk[u].w},
                                    reinterpret_cast<f32x4*>(ok + off));
        __builtin_nontemporal_store(f32x4{rv[u].x, rv[u].y, rv[u].z, rv[u].w},
                                    reinterpret_cast<f32x4*>(ov + off));
      }
    }
  }
}

// Unpack in bucket order (the order the buckets are stored in): block x
// takes RPB consecutive rows (entry, b) of one precision's bucket, so every
// wave decodes a single precision and reads the bucket contiguously; each
// row goes to out row b*H*S + flat, flat = h*S + t from that precision's
// flat index list (PrecisionPlan.flat_indices, precision_plan.py:144-151).
// Blocks past the buckets zero the rows of entries whose code is outside
// 0..3 (evicted or absent). blk_end[p]: first block after precision p's.

template <int D, int SDT, int U, int P, int NT>
__device__ __forceinline__ void unpack_bucket_rows(const UnpackLists& L, const Buckets& bk,
                                                   int64_t lb, int B, int64_t HS, int g,
                                                   float* __restrict__ ok, float* __restrict__ ov) {
  constexpr int CPR = D / 4;
  constexpr int RPP = NT / CPR;
  const int ch = threadIdx.x % CPR;
  const int64_t rows = L.n[P] * B;
  const int64_t r0 = lb * (RPP * U) + threadIdx.x / CPR;
  float4 rk[U], rv[U];
  int64_t off[U];
#pragma unroll
  for (int u = 0; u < U; ++u) {
    const int64_t r = r0 + u * RPP;
    off[u] = -1;
    if (r < rows) {
      const int64_t sl = r / B;
      const int64_t b = r - sl * B;
      off[u] = (b * HS + L.flat[P][sl]) * D + ch * 4;
      rk[u] = dequant4<SDT>(bk, 0, P, sl, b, ch * 4, B, D, g);
      rv[u] = dequant4<SDT>(bk, 1, P, sl, b, ch * 4, B, D, g);
    }
  }
  typedef float f32x4 __attribute__((ext_vector_type(4)));
#pragma unroll
  for (int u = 0; u < U; ++u) {
    if (off[u] >= 0) {
      __builtin_nontemporal_store(f32x4{rk[u].x, rk[u].y, rk[u].z, rk[u].w},
                                  reinterpret_cast<f32x4*>(ok + off[u]));
      __builtin_nontemporal_store(f32x4{rv[u].x, rv[u].y, rv[u].z, rv[u].w},
                                  reinterpret_cast<f32x4*>(ov + off[u]));
    }
  }
}

template <int D, int SDT, int U, int NT>
__global__ __launch_bounds__(NT) void kv_unpack_lists(UnpackLists L,
                                                       const int8_t* __restrict__ code,
                                                       Buckets bk, int B, int H, int S, int g,
                                                       float* __restrict__ ok,
                                                       float* __restrict__ ov) {
  const int64_t blk = blockIdx.x;
  const int64_t HS = (int64_t)H * S;
  if (blk < L.blk_end[3]) {
    if (blk < L.blk_end[0]) {
      unpack_bucket_rows<D, SDT, U, SI_PREC_FP32, NT>(L, bk, blk, B, HS, g, ok, ov);
    } else if (blk < L.blk_end[1]) {
      unpack_bucket_rows<D, SDT, U, SI_PREC_FP16, NT>(L, bk, blk - L.blk_end[0], B, HS, g, ok, ov);
    } else if (blk < L.blk_end[2]) {
      unpack_bucket_rows<D, SDT, U, SI_PREC_INT8, NT>(L, bk, blk - L.blk_end[1], B, HS, g, ok, ov);
    } else {
      unpack_bucket_rows<D, SDT, U, SI_PREC_INT4, NT>(L, bk, blk - L.blk_end[2], B, HS, g, ok, ov);
    }
    return;
  }
  // zero rows: entries e = t*H + h with a code outside 0..3
  constexpr int CPR = D / 4;
  constexpr int RPP = NT / CPR;
  const int ch = threadIdx.x % CPR;
  const int64_t e0 = (blk - L.blk_end[3]) * (RPP * U) + threadIdx.x / CPR;
  typedef float f32x4 __attribute__((ext_vector_type(4)));
#pragma unroll
  for (int u = 0; u < U; ++u) {
    const int64_t e = e0 + u * RPP;
    if (e >= HS) break;
    const int c = code[e];
    if (c >= 0 && c <= 3) continue;
    const int64_t t = e / H;
    const int64_t h = e - t * H;
    for (int b = 0; b < B; ++b) {
      const int64_t o = (b * HS + h * S + t) * D + ch * 4;
      __builtin_nontemporal_store(f32x4{0.f, 0.f, 0.f, 0.f}, reinterpret_cast<f32x4*>(ok + o));
      __builtin_nontemporal_store(f32x4{0.f, 0.f, 0.f, 0.f}, reinterpret_cast<f32x4*>(ov + o));
    }
  }
}

template <int SDT>
__global__ __launch_bounds__(256) void kv_unpack_vec4(const int8_t* __restrict__ code,
                                                      const int32_t* __restrict__ slot, Buckets bk,
                                                      int64_t B, int64_t H, int64_t S, int64_t D,
                                                      int64_t g, float* __restrict__ ok,
                                                      float* __restrict__ ov) {
  const int64_t cpr = D / 4;
  const int64_t total = B * H * S * cpr;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total;
       i += (int64_t)gridDim.x * blockDim.x) {
    const int64_t ch = i % cpr;
    const int64_t row = i / cpr;
    const int64_t t = row % S;
    const int64_t bh = row / S;
    const int64_t h = bh % H;
    const int64_t b = bh / H;
    const int64_t e = t * H + h;
    const int c = code[e];
    float4 vk = make_float4(0.f, 0.f, 0.f, 0.f), vv = vk;
    if (c >= 0 && c <= 3) {
      const int64_t s = slot[e];
      vk = dequant4<SDT>(bk, 0, c, s, b, ch * 4, B, D, g);
      vv = dequant4<SDT>(bk, 1, c, s, b, ch * 4, B, D, g);
    }
    typedef float f32x4 __attribute__((ext_vector_type(4)));
    __builtin_nontemporal_store(f32x4{vk.x, vk.y, vk.z, vk.w},
                                reinterpret_cast<f32x4*>(ok + row * D + ch * 4));
    __builtin_nontemporal_store(f32x4{vv.x, vv.y, vv.z, vv.w},
                                reinterpret_cast<f32x4*>(ov + row * D + ch * 4));
  }
}

// ---------------------------------------------------------------------------
// Row copies for reuse and compaction.
// ---------------------------------------------------------------------------

struct RowGeom {
  int64_t data_bytes[4];   // per entry, per precision
  int64_t scale_bytes[4];  // per entry, per precision (0 for fp32/fp16)
};

__host__ RowGeom make_geom(int64_t B, int64_t D, int64_t g, int sdt) {
  RowGeom r;
  const int64_t ssz = dtype_size(sdt);
  r.data_bytes[0] = B * D * 4;
  r.data_bytes[1] = B * D * 2;
  r.data_bytes[2] = B * D;
  r.data_bytes[3] = (B * D + 1) / 2;
  r.scale_bytes[0] = 0;
  r.scale_bytes[1] = 0;
  r.scale_bytes[2] = B * ssz;
  r.scale_bytes[3] = (g > 0 ? B * (D / g) : 0) * ssz;
  return r;
}

// Copy n bytes with `lanes` cooperating lanes (lane index `lane`).
__device__ __forceinline__ void copy_bytes(uint8_t* dst, const uint8_t* src, int64_t n, int lane,
                                           int lanes) {
  const uintptr_t mis = (reinterpret_cast<uintptr_t>(dst) | reinterpret_cast<uintptr_t>(src) |
                         (uintptr_t)n);
  if ((mis & 15) == 0) {
    for (int64_t i = lane; i < n / 16; i += lanes)
      reinterpret_cast<uint4*>(dst)[i] = reinterpret_cast<const uint4*>(src)[i];
  } else if ((mis & 3) == 0) {
    for (int64_t i = lane; i < n / 4; i += lanes)
      reinterpret_cast<uint32_t*>(dst)[i] = reinterpret_cast<const uint32_t*>(src)[i];
  } else {
    for (int64_t i = lane; i < n; i += lanes) dst[i] = src[i];
  }
}

__device__ __forceinline__ void copy_entry(const Buckets& dst, int64_t dslot, const Buckets& src,
                                           int64_t sslot, int c, const RowGeom& geo, int lane,
                                           int lanes) {
  if (dst.p[4 * c] == nullptr) return;  // bucket not being rewritten
  const int64_t db = geo.data_bytes[c];
  const int64_t sb = geo.scale_bytes[c];
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    copy_bytes(reinterpret_cast<uint8_t*>(dst.p[4 * c + j]) + dslot * db,
               reinterpret_cast<const uint8_t*>(src.p[4 * c + j]) + sslot * db, db, lane, lanes);
    if (sb)
      copy_bytes(reinterpret_cast<uint8_t*>(dst.p[4 * c + 2 + j]) + dslot * sb,
                 reinterpret_cast<const uint8_t*>(src.p[4 * c + 2 + j]) + sslot * sb, sb, lane,
                 lanes);
  }
}

constexpr int kCopyLanes = 16;

__global__ __launch_bounds__(256) void kv_compact_kernel(
    const int8_t* __restrict__ old_code, const int32_t* __restrict__ old_slot, Buckets oldb,
    const int8_t* __restrict__ new_code, const int32_t* __restrict__ new_slot, Buckets newb,
    int64_t n, RowGeom geo) {
  const int lane = threadIdx.x % kCopyLanes;
  const int64_t step = (int64_t)gridDim.x * (blockDim.x / kCopyLanes);
  for (int64_t e = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) / kCopyLanes; e < n;
       e += step) {
    const int c = new_code[e];
    if (c < 0 || c > 3) continue;
    copy_entry(newb, new_slot[e], oldb, old_slot[e], c, geo, lane, kCopyLanes);
  }
}

// ---------------------------------------------------------------------------
// Bucket-order entry copies for reuse and compaction. Each block owns kListRows
// consecutive destination slots of one precision (the destination plan's
// per-precision h*S + t lists, in slot order), resolves every row's source
// slot once into LDS, then copies the K and V rows and their scales with
// consecutive threads on consecutive units of the rows: contiguous destination
// rows, no divergence between precisions.
// ---------------------------------------------------------------------------

#ifndef SI_LIST_ROWS
#define SI_LIST_ROWS 128
#endif
constexpr int kListRows = SI_LIST_ROWS;
// 16-byte units each thread loads before it stores them
#ifndef SI_COPY_UNR
#define SI_COPY_UNR 1
#endif
// reuse: pack the copied rows to the front of the block's list
#ifndef SI_REUSE_COMPACT
#define SI_REUSE_COMPACT 1
#endif

// The unit indices of one block's rows need 64 bits only when kListRows fp32
// rows of B * D values reach 2^32 bytes.
inline bool list_rows_wide(int64_t B, int64_t D) { return B * D * 4 * kListRows >= ((int64_t)1 << 32); }

struct CopyLists {
  const int64_t* flat[4];  // destination slot order: h*S + t
  int64_t n[4];
  int64_t blk_end[4];
};

// WIDE: 64-bit unit indices (rows * row_bytes may exceed 2^32). Row r of the
// list goes from row srcs[r] of src to row s0 + (drows ? drows[r] : r) of dst
// (skipped where srcs[r] < 0). Each thread loads four units before it stores
// them, so four reads per lane are in flight.
template <int U, bool WIDE, int UNR = SI_COPY_UNR>
__device__ __forceinline__ void copy_units(uint8_t* __restrict__ dst, const uint8_t* __restrict__ src,
                                           int64_t row_bytes, int64_t s0, int rows,
                                           const int64_t* srcs, const int32_t* drows) {
  // a clang vector type (HIP's uint4 is a class, and an array of it is kept
  // in scratch memory instead of registers)
  typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
  typedef typename std::conditional<U == 16, u32x4,
          typename std::conditional<U == 4, uint32_t,
          typename std::conditional<U == 2, uint16_t, uint8_t>::type>::type>::type T;
  typedef typename std::conditional<WIDE, int64_t, unsigned>::type I;
  const I cpr = (I)(row_bytes / U);
  const I total = (I)rows * cpr;
  for (I i0 = threadIdx.x; i0 < total; i0 += UNR * blockDim.x) {
    T v[UNR];
    int64_t doff[UNR];
    bool ok[UNR];
#pragma unroll
    for (int u = 0; u < UNR; ++u) {
      const I i = i0 + (I)(u * blockDim.x);
      ok[u] = i < total;
      doff[u] = 0;
      if (ok[u]) {
        const I r = i / cpr;
        const I c = i - r * cpr;
        const int64_t ss = srcs[r];
        ok[u] = ss >= 0;
        doff[u] = (s0 + (drows != nullptr ? (int64_t)drows[r] : (int64_t)r)) * row_bytes + (int64_t)c * U;
        if (ok[u]) v[u] = *reinterpret_cast<const T*>(src + ss * row_bytes + (int64_t)c * U);
      }
    }
#pragma unroll
    for (int u = 0; u < UNR; ++u)
      if (ok[u]) *reinterpret_cast<T*>(dst + doff[u]) = v[u];
  }
}

// List rows 0 .. rows-1: dst row s0 + (drows ? drows[r] : r) <- src row srcs[r].
template <bool WIDE, int UNR = SI_COPY_UNR>
__device__ __forceinline__ void copy_rows(void* dst, const void* src, int64_t row_bytes, int64_t s0,
                                          int rows, const int64_t* srcs, const int32_t* drows) {
  if (dst == nullptr || src == nullptr || row_bytes == 0) return;
  uint8_t* d = reinterpret_cast<uint8_t*>(dst);
  const uint8_t* sp = reinterpret_cast<const uint8_t*>(src);
  const uintptr_t mis = reinterpret_cast<uintptr_t>(d) | reinterpret_cast<uintptr_t>(sp) |
                        (uintptr_t)row_bytes;
  if ((mis & 15) == 0) copy_units<16, WIDE, UNR>(d, sp, row_bytes, s0, rows, srcs, drows);
  else if ((mis & 3) == 0) copy_units<4, WIDE, UNR>(d, sp, row_bytes, s0, rows, srcs, drows);
  else if ((mis & 1) == 0) copy_units<2, WIDE, UNR>(d, sp, row_bytes, s0, rows, srcs, drows);
  else copy_units<1, WIDE, UNR>(d, sp, row_bytes, s0, rows, srcs, drows);
}

// REUSE: destination = current cache, source = previous cache (same H, so the
// same token-major entry id); a row is copied when mask[e] is set, t < S_src
// and the previous code equals the row's precision (apply_reuse_mask,
// packed_kv_cache.py:791-852). Otherwise (compaction, :698-737): every row is
// copied from src_slot[e] of the old buckets.
template <bool REUSE, bool WIDE>
__global__ __launch_bounds__(256) void kv_copy_lists(CopyLists L, Buckets dst, Buckets src,
                                                     const int8_t* __restrict__ src_code,
                                                     const int32_t* __restrict__ src_slot,
                                                     const uint8_t* __restrict__ mask, int64_t S,
                                                     int64_t H, int64_t S_src, RowGeom geo,
                                                     unsigned long long* __restrict__ stats) {
  static_assert(kListRows <= 256, "one thread resolves each row");
  __shared__ int64_t srcs[kListRows];
  __shared__ int32_t drows[kListRows];
  __shared__ unsigned wave_n[4];
  __shared__ unsigned cnt[2];
  const int64_t blk = blockIdx.x;
  int p = 0;
  while (p < 3 && blk >= L.blk_end[p]) ++p;
  const int64_t s0 = (blk - (p > 0 ? L.blk_end[p - 1] : 0)) * kListRows;
  const int rows = (int)min<int64_t>(kListRows, L.n[p] - s0);
  if (threadIdx.x < 2) cnt[threadIdx.x] = 0u;
  __syncthreads();
  int64_t ss = -1;
  if ((int)threadIdx.x < rows) {
    const int64_t f = L.flat[p][s0 + threadIdx.x];
    const int64_t t = f % S;
    const int64_t e = t * H + f / S;
    if constexpr (REUSE) {
      // mask, previous code and previous slot in one round of loads (entry e
      // of the previous cache exists when t < S_src)
      const bool inside = t < S_src;
      const int mk = mask[e];
      const int pc = inside ? (int)src_code[e] : 4;
      const int64_t ps = inside ? (int64_t)src_slot[e] : -1;
      if (mk != 0 && inside) {
        if (pc == p) {
          ss = ps;
          atomicAdd(&cnt[0], 1u);
        } else if (pc >= 0 && pc <= 3) {
          atomicAdd(&cnt[1], 1u);
        }
      }
    } else {
      ss = src_slot[e];
    }
  }
  int n_rows = rows;
  const int32_t* dr = nullptr;
  if constexpr (REUSE && SI_REUSE_COMPACT) {
    // Only the reused rows are copied: pack them to the front of the list
    // (in slot order), so no lane of the copy loop idles on a skipped row.
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    const bool act = ss >= 0;
    const unsigned long long bal = __ballot(act);
    if (lane == 0) wave_n[w] = (unsigned)__popcll(bal);
    __syncthreads();
    unsigned off = 0, tot = 0;
#pragma unroll
    for (int x = 0; x < 4; ++x) {
      off += x < w ? wave_n[x] : 0u;
      tot += wave_n[x];
    }
    if (act) {
      const unsigned k = off + (unsigned)__popcll(bal & ((1ull << lane) - 1ull));
      srcs[k] = ss;
      drows[k] = (int32_t)threadIdx.x;
    }
    n_rows = (int)tot;
    dr = drows;
  } else {
    if ((int)threadIdx.x < rows) srcs[threadIdx.x] = ss;
  }
  __syncthreads();
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    copy_rows<WIDE>(dst.p[4 * p + j], src.p[4 * p + j], geo.data_bytes[p], s0, n_rows, srcs, dr);
    if (geo.scale_bytes[p] > 0)
      copy_rows<WIDE>(dst.p[4 * p + 2 + j], src.p[4 * p + 2 + j], geo.scale_bytes[p], s0, n_rows,
                      srcs, dr);
  }
  if (REUSE && stats != nullptr && threadIdx.x == 0 && (cnt[0] | cnt[1])) {
    atomicAdd(stats, (unsigned long long)cnt[0]);
    atomicAdd(stats + 1, (unsigned long long)cnt[1]);
  }
}

// Block counts of a CopyLists launch; 0 for precisions with no destination bucket.
int64_t copy_lists_setup(CopyLists& L, const int64_t* const* flat, const int64_t* counts,
                         const Buckets& dst) {
  int64_t acc = 0;
  for (int p = 0; p < 4; ++p) {
    L.flat[p] = flat[p];
    L.n[p] = dst.p[4 * p] != nullptr ? counts[p] : 0;
    acc += ceil_div(L.n[p], kListRows);
    L.blk_end[p] = acc;
  }
  return acc;
}

// ---------------------------------------------------------------------------
// Evict over the old grouping's lists (si_kv_evict_count + si_kv_evict_flat).
// Chunk j of the chunk space covers kEvictRows consecutive old slots of one
// precision (precisions in order 0..3, as the lists). Pass 1 counts the
// survivors of every chunk and writes the new code of every entry, and slot
// -1 for the entries that leave or were absent. Pass 2 gives each survivor
// the new slot
//   (survivors in the earlier chunks of its precision) + (its rank in the chunk)
// - the stable in-bucket compaction of packed_kv_cache.py:698-737 - and
// writes that slot, the new flat list entry and the entry's K/V rows and
// scales (source rows: consecutive old slots; destination rows: consecutive
// new slots). No token-order rescan of the codes is needed.
// ---------------------------------------------------------------------------
#ifndef SI_EVICT_ROWS
#define SI_EVICT_ROWS 128
#endif
constexpr int kEvictRows = SI_EVICT_ROWS;
constexpr int kEvictWords = kEvictRows / 64;  // survivor bit words per chunk
#ifndef SI_EVICT_THREADS
#define SI_EVICT_THREADS 256
#endif
// threads of a pass-2 block: threads past kEvictRows only help with the copy
constexpr int kEvictThreads = SI_EVICT_THREADS;
static_assert(kEvictThreads >= kEvictRows && kEvictThreads % 64 == 0, "one thread per row at least");
constexpr int kEvictFixEntries = 16;          // absent entries: 16 codes per thread
static_assert(kEvictRows == 128 || kEvictRows == 256, "chunks of 2 or 4 waves");

struct EvictLists {
  const int64_t* flat[4];  // old grouping: h*S + t per old slot
  int64_t n[4];            // old bucket sizes
  int64_t blk_end[4];      // end of each precision's chunks in the chunk space
};

struct NewLists {
  int64_t* flat[4];  // new grouping's lists (null: not written)
  int64_t n[4];      // new bucket sizes
};

__host__ int64_t evict_lists_setup(EvictLists& L, const int64_t* const* flat, const int64_t* counts) {
  int64_t acc = 0;
  for (int p = 0; p < 4; ++p) {
    L.flat[p] = flat[p];
    L.n[p] = counts[p];
    acc += ceil_div(counts[p], kEvictRows);
    L.blk_end[p] = acc;
  }
  return acc;
}

// Precision, first old slot and row count of chunk `blk`.
__device__ __forceinline__ int evict_chunk(const EvictLists& L, int64_t blk, int64_t* s0, int* rows) {
  int p = 0;
  while (p < 3 && blk >= L.blk_end[p]) ++p;
  *s0 = (blk - (p > 0 ? L.blk_end[p - 1] : 0)) * kEvictRows;
  *rows = (int)min<int64_t>(kEvictRows, L.n[p] - *s0);
  return p;
}

// Blocks [0, chunks): one thread per old slot. Blocks from `chunks` on: the
// entries that are in no list (code outside 0..3) get code 4 and slot -1.
__global__ __launch_bounds__(kEvictRows) void kv_evict_count(EvictLists L, int64_t chunks,
                                                             const int8_t* __restrict__ old_code,
                                                             const uint8_t* __restrict__ mask,
                                                             int64_t S, int64_t H,
                                                             int8_t* __restrict__ new_code,
                                                             int32_t* __restrict__ new_slot,
                                                             int32_t* __restrict__ chunk_count,
                                                             unsigned long long* __restrict__ chunk_bits) {
  const int64_t blk = blockIdx.x;
  if (blk >= chunks) {
    const int64_t n = S * H;
    const int64_t e0 = ((blk - chunks) * kEvictRows + threadIdx.x) * kEvictFixEntries;
    if (e0 >= n) return;
    int8_t c[kEvictFixEntries];
    if (e0 + kEvictFixEntries <= n && (reinterpret_cast<uintptr_t>(old_code + e0) & 15) == 0) {
      const uint4 w = *reinterpret_cast<const uint4*>(old_code + e0);
      const uint32_t ws[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
      for (int i = 0; i < kEvictFixEntries; ++i) c[i] = (int8_t)(ws[i / 4] >> (8 * (i % 4)));
    } else {
#pragma unroll
      for (int i = 0; i < kEvictFixEntries; ++i) c[i] = e0 + i < n ? old_code[e0 + i] : (int8_t)0;
    }
#pragma unroll
    for (int i = 0; i < kEvictFixEntries; ++i) {
      if (e0 + i < n && (c[i] < 0 || c[i] > 3)) {
        new_code[e0 + i] = 4;
        new_slot[e0 + i] = -1;
      }
    }
    return;
  }
  __shared__ unsigned wave_n[kEvictRows / 64];
  int64_t s0;
  int rows;
  const int p = evict_chunk(L, blk, &s0, &rows);
  bool keep = false;
  if ((int)threadIdx.x < rows) {
    const int64_t f = L.flat[p][s0 + threadIdx.x];
    const uint32_t fu = (uint32_t)f, su = (uint32_t)S;  // S * H < 2^31
    const int64_t e = (int64_t)(fu % su) * H + (fu / su);
    keep = mask[e] == 0;
    new_code[e] = keep ? (int8_t)p : (int8_t)4;
    if (!keep) new_slot[e] = -1;
  }
  const unsigned long long bal = __ballot(keep);
  if ((threadIdx.x & 63) == 0) {
    wave_n[threadIdx.x >> 6] = (unsigned)__popcll(bal);
    chunk_bits[blk * kEvictWords + (threadIdx.x >> 6)] = bal;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    unsigned tot = 0;
#pragma unroll
    for (int w = 0; w < kEvictWords; ++w) tot += wave_n[w];
    chunk_count[blk] = (int32_t)tot;
  }
}

// One block per chunk, a thread per old slot (and more threads for the copy,
// as the compaction's blocks have twice the threads of their rows): survivor
// bits and ranks come
// from pass 1's ballots, so the chunk counts, the bits and the old list are
// loaded side by side and the mask is not read again. new_n[p] bounds every
// slot written; rows are copied only for precisions whose new bucket pointer
// is set.
template <bool WIDE>
__global__ __launch_bounds__(kEvictThreads) void kv_evict_lists(
    EvictLists L, const int32_t* __restrict__ chunk_count,
    const unsigned long long* __restrict__ chunk_bits, int64_t S, int64_t H, Buckets dst,
    Buckets src, RowGeom geo, NewLists nl, int32_t* __restrict__ new_slot) {
  constexpr int kWaves = kEvictThreads / 64;
  __shared__ int64_t srcs[kEvictRows];
  __shared__ int64_t part[kWaves];
  const int64_t blk = blockIdx.x;
  int64_t s0;
  int rows;
  const int p = evict_chunk(L, blk, &s0, &rows);
  const int64_t first = p > 0 ? L.blk_end[p - 1] : 0;
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  unsigned long long bits[kEvictWords];
#pragma unroll
  for (int x = 0; x < kEvictWords; ++x) bits[x] = chunk_bits[blk * kEvictWords + x];
  const int64_t f = (int)threadIdx.x < rows ? L.flat[p][s0 + threadIdx.x] : -1;
  // survivors in the earlier chunks of this precision: each thread issues its
  // loads in batches of 8, so a late chunk of a long list waits for one round
  // trip per 8 * kEvictRows chunks instead of one per kEvictRows
  constexpr int kBatch = 8;
  int64_t acc = 0;
  for (int64_t j0 = first + threadIdx.x; j0 < blk; j0 += kBatch * kEvictThreads) {
    int32_t c[kBatch];
#pragma unroll
    for (int b = 0; b < kBatch; ++b) {
      const int64_t j = j0 + (int64_t)b * kEvictThreads;
      c[b] = j < blk ? chunk_count[j] : 0;
    }
#pragma unroll
    for (int b = 0; b < kBatch; ++b) acc += c[b];
  }
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) acc += __shfl_xor(acc, o);
  if (lane == 0) part[w] = acc;
  unsigned k = 0, tot = 0;
#pragma unroll
  for (int x = 0; x < kEvictWords; ++x) {
    const unsigned c = (unsigned)__popcll(bits[x]);
    k += x < w ? c : 0u;
    tot += c;
  }
  unsigned long long wb = w == 0 ? bits[0] : 0ull;  // this wave's word (none past the rows)
#pragma unroll
  for (int x = 1; x < kEvictWords; ++x) wb = w == x ? bits[x] : wb;
  const bool keep = ((wb >> lane) & 1ull) != 0 && (int)threadIdx.x < rows;
  k += (unsigned)__popcll(wb & ((1ull << lane) - 1ull));
  __syncthreads();
  int64_t prefix = 0;
#pragma unroll
  for (int x = 0; x < kWaves; ++x) prefix += part[x];
  const int64_t limit = nl.n[p];
  if (keep) {
    const int64_t ns = prefix + (int64_t)k;
    if (ns < limit) {
      srcs[k] = s0 + threadIdx.x;
      const uint32_t fu = (uint32_t)f, su = (uint32_t)S;  // S * H < 2^31
      new_slot[(int64_t)(fu % su) * H + (fu / su)] = (int32_t)ns;
      if (nl.flat[p] != nullptr) nl.flat[p][ns] = f;
    }
  }
  __syncthreads();
  const int n_rows = (int)max<int64_t>(0, min<int64_t>((int64_t)tot, limit - prefix));
  if (n_rows == 0) return;
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    copy_rows<WIDE>(dst.p[4 * p + j], src.p[4 * p + j], geo.data_bytes[p], prefix, n_rows, srcs,
                    nullptr);
    if (geo.scale_bytes[p] > 0)
      copy_rows<WIDE>(dst.p[4 * p + 2 + j], src.p[4 * p + 2 + j], geo.scale_bytes[p], prefix,
                      n_rows, srcs, nullptr);
  }
}

// ---------------------------------------------------------------------------
// Token-order reuse (si_kv_reuse, for callers without the plan's flat lists).
// A block owns kTileEntries consecutive entries e = t*H + h: its threads read
// their entries' codes, mask and slots with coalesced loads, gather the rows
// to copy into one LDS list ordered by precision, then copy each precision's
// rows with every thread of the block (within a tile the rows of one
// precision have increasing slots on both sides, and no wave mixes
// precisions inside a copy loop). 19.7 us for a 1 x 32 x 8192 x 128 layer
// with half its entries reused, against 47.7 us for lanes that each walked
// one entry; the bucket-order copy (si_kv_reuse_flat) takes 16.6 us.
// ---------------------------------------------------------------------------
constexpr int kTileThreads = 256;
constexpr int kTileEntries = kTileThreads;  // one entry per thread
constexpr int kTileUnroll = 2;              // 16-byte units in flight per lane

// Exclusive block scan of four 16-bit counters packed in a u64 (a tile holds
// at most 256 entries, so no field overflows); *total gets the block sums.
__device__ __forceinline__ unsigned long long tile_scan4(unsigned long long v,
                                                         unsigned long long* lds,
                                                         unsigned long long* total) {
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  unsigned long long x = v;
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) {
    const unsigned long long y = __shfl_up(x, off, 64);
    if (lane >= off) x += y;
  }
  if (lane == 63) lds[w] = x;
  __syncthreads();
  unsigned long long before = 0, tot = 0;
#pragma unroll
  for (int i = 0; i < kTileThreads / 64; ++i) {
    before += i < w ? lds[i] : 0ull;
    tot += lds[i];
  }
  __syncthreads();
  *total = tot;
  return before + x - v;
}

// apply_reuse_mask (packed_kv_cache.py:791-852) in token order: entry e of
// the current cache takes its previous row when mask[e] is set, t < S_prev and
// the previous code equals its own; a previous code of another precision is
// counted as skipped.
__global__ __launch_bounds__(kTileThreads) void kv_reuse_tiles(
    const int8_t* __restrict__ cur_code, const int32_t* __restrict__ cur_slot, Buckets dst,
    int64_t S, const int8_t* __restrict__ prev_code, const int32_t* __restrict__ prev_slot,
    Buckets src, int64_t S_prev, const uint8_t* __restrict__ mask, int64_t H, RowGeom geo,
    unsigned long long* __restrict__ stats) {
  __shared__ int64_t srcs[kTileEntries];
  __shared__ int32_t dsts[kTileEntries];
  __shared__ unsigned long long scan_lds[kTileThreads / 64];
  const int64_t n = S * H, n_prev = S_prev * H;
  const int64_t e = (int64_t)blockIdx.x * kTileEntries + threadIdx.x;
  int c = 4, pc = 4, mk = 0;
  int32_t cs = -1, ps = -1;
  if (e < n) {
    c = cur_code[e];
    mk = mask[e];
    cs = cur_slot[e];
  }
  if (e < n_prev) {  // t < S_prev: the previous cache's entry e
    pc = prev_code[e];
    ps = prev_slot[e];
  }
  c = (c < 0 || c > 3) ? 4 : c;
  pc = (pc < 0 || pc > 3) ? 4 : pc;
  const bool sel = c < 4 && mk != 0;
  const bool take = sel && pc == c;
  const bool skip = sel && pc < 4 && pc != c;
  unsigned long long tot;
  const unsigned long long before = tile_scan4(take ? (1ull << (16 * c)) : 0ull, scan_lds, &tot);
  int base[4], nn[4];
#pragma unroll
  for (int p = 0, acc = 0; p < 4; ++p) {
    nn[p] = (int)((tot >> (16 * p)) & 0xffffull);
    base[p] = acc;
    acc += nn[p];
  }
  if (take) {
    int k = 0;
#pragma unroll
    for (int p = 0; p < 4; ++p)
      if (c == p) k = base[p] + (int)((before >> (16 * p)) & 0xffffull);
    srcs[k] = ps;
    dsts[k] = cs;
  }
  if (stats != nullptr) {
    const unsigned long long a = __ballot(take), b = __ballot(skip);
    if ((threadIdx.x & 63) == 0 && (a | b)) {
      atomicAdd(stats, (unsigned long long)__popcll(a));
      atomicAdd(stats + 1, (unsigned long long)__popcll(b));
    }
  }
  __syncthreads();
#pragma unroll
  for (int p = 0; p < 4; ++p) {
    if (nn[p] == 0) continue;
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      copy_rows<false, kTileUnroll>(dst.p[4 * p + j], src.p[4 * p + j], geo.data_bytes[p], 0,
                                    nn[p], srcs + base[p], dsts + base[p]);
      if (geo.scale_bytes[p] > 0)
        copy_rows<false, kTileUnroll>(dst.p[4 * p + 2 + j], src.p[4 * p + 2 + j],
                                      geo.scale_bytes[p], 0, nn[p], srcs + base[p],
                                      dsts + base[p]);
    }
  }
}

// ---------------------------------------------------------------------------
// Paged store (PagedKVStore, shadowinfer/shadowkv/paged_kv_store.py). A page
// holds one precision for tokens [start, start + n) of every (b, h) in
// capacity buffers [B, H, P, ...]: payload rows of D values in the input
// dtype ("fp32" pages keep the input as it is, :189-193), fp16, int8, or
// ceil(D/2) int4 bytes (high nibble first, code + 8), with per-row int8
// scales [B, H, P, 1] and per-group int4 scales [B, H, P, G, 1] in the input
// dtype. Quantization is the pack's row arithmetic, so page rows equal the
// rows PackedKVCache would hold.
// ---------------------------------------------------------------------------

// Writes tokens t0 .. t0+take-1 of k/v [B, H, T, D] into rows off .. of the
// page (append :248-307, rewrite_tokens :407-447). Page pointers sit in the
// bucket slots of `prec`. Grid: blockIdx.y = b*H + h.
template <int DT, int LPR>
__global__ __launch_bounds__(256) void page_write_fast(const void* __restrict__ kin,
                                                       const void* __restrict__ vin, int T, int t0,
                                                       int take, int P, int off, int prec, int lpg,
                                                       Buckets pg) {
  constexpr int EPL = Chunk<DT>::EPL;
  constexpr int D = EPL * LPR;
  constexpr int RPP = 256 / LPR;
  constexpr int ES = DT == SI_DT_F32 ? 4 : 2;
  const int lane = threadIdx.x % LPR;
  const int j = blockIdx.x * RPP + threadIdx.x / LPR;
  if (j >= take) return;
  const int64_t bh = blockIdx.y;
  const int64_t src = (bh * T + t0 + j) * D + lane * EPL;
  // Row off + j of (b, h) in a run of pages of P rows each, B*H*P rows per page.
  const int r = off + j;
  const int dst = (r / P) * ((int)gridDim.y * P) + (int)bh * P + r % P;
  if (prec == SI_PREC_FP32) {  // the input dtype, unchanged
    typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
    const u32x4 a = *reinterpret_cast<const u32x4*>(reinterpret_cast<const char*>(kin) + src * ES);
    const u32x4 b = *reinterpret_cast<const u32x4*>(reinterpret_cast<const char*>(vin) + src * ES);
    const int64_t o = ((int64_t)dst * D + lane * EPL) * ES;
    *reinterpret_cast<u32x4*>(reinterpret_cast<char*>(pg.p[0]) + o) = a;
    *reinterpret_cast<u32x4*>(reinterpret_cast<char*>(pg.p[1]) + o) = b;
    return;
  }
  float xk[EPL], xv[EPL];
  load_chunk<DT>(kin, src, xk);
  load_chunk<DT>(vin, src, xv);
  pack_row<DT, LPR, false>(xk, xv, prec, dst, 0, 1, lane, lpg, pg, nullptr, nullptr);
}

// Any D and group: one thread per (b, h, token) row.
template <int DT>
__global__ __launch_bounds__(256) void page_write_generic(const void* __restrict__ kin,
                                                          const void* __restrict__ vin, int64_t BH,
                                                          int64_t T, int64_t D, int64_t t0,
                                                          int64_t take, int64_t P, int64_t off,
                                                          int prec, int64_t g, Buckets pg) {
  constexpr int ES = DT == SI_DT_F32 ? 4 : 2;
  for (int64_t r = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; r < BH * take;
       r += (int64_t)gridDim.x * blockDim.x) {
    const int64_t bh = r / take;
    const int64_t j = r - bh * take;
    const int64_t src = (bh * T + t0 + j) * D;
    const int64_t rr = off + j;  // row of (b, h) in a run of pages of P rows each
    const int64_t dst = (rr / P) * (BH * P) + bh * P + rr % P;
    if (prec == SI_PREC_FP32) {
      for (int64_t d = 0; d < D * ES; ++d) {
        reinterpret_cast<char*>(pg.p[0])[dst * D * ES + d] = reinterpret_cast<const char*>(kin)[src * ES + d];
        reinterpret_cast<char*>(pg.p[1])[dst * D * ES + d] = reinterpret_cast<const char*>(vin)[src * ES + d];
      }
      continue;
    }
    const char* kr = reinterpret_cast<const char*>(kin) + src * ES;
    const char* vr = reinterpret_cast<const char*>(vin) + src * ES;
    pack_entry_generic<DT>(kr, 1, 1, 1, D, g, 0, 0, prec, dst, pg.p[4 * prec + 0],
                           pg.p[4 * prec + 2], nullptr);
    pack_entry_generic<DT>(vr, 1, 1, 1, D, g, 0, 0, prec, dst, pg.p[4 * prec + 1],
                           pg.p[4 * prec + 3], nullptr);
  }
}

// One page-table row: precision, k, v, scale_k, scale_v, start token, tokens,
// capacity (int64 each).
// One row of the device page table: precision, the page's input dtype (the
// dtype of its scales and of "fp32" payloads), payload and scale pointers,
// first token, tokens held, capacity in rows.
struct PageRow {
  int64_t prec, dt, k, v, sk, sv, start, ntok, cap;
};
constexpr int kPageRowWords = 9;

template <int SDT>
__device__ __forceinline__ float page_value(const PageRow& pr, int j, int64_t row, int64_t d,
                                            int64_t D, int64_t g) {
  const int64_t e = row * D + d;
  switch (pr.prec) {
    case SI_PREC_FP32: return load_any(reinterpret_cast<const void*>(j ? pr.v : pr.k), SDT, e);
    case SI_PREC_FP16:
      return f16_bits_to_f32(reinterpret_cast<const uint16_t*>(j ? pr.v : pr.k)[e]);
    case SI_PREC_INT8:
      return (float)reinterpret_cast<const int8_t*>(j ? pr.v : pr.k)[e] *
             load_any(reinterpret_cast<const void*>(j ? pr.sv : pr.sk), SDT, row);
    default: {
      const int64_t rb = (D + 1) / 2;
      const uint32_t byte = reinterpret_cast<const uint8_t*>(j ? pr.v : pr.k)[row * rb + d / 2];
      const int nib = (d & 1) ? (int)(byte & 0xfu) : (int)(byte >> 4);
      return (float)(nib - 8) *
             load_any(reinterpret_cast<const void*>(j ? pr.sv : pr.sk), SDT, row * (D / g) + d / g);
    }
  }
}

// Four consecutive values (one group) of a page row, decoded to fp32.
template <int SDT, int PREC>
__device__ __forceinline__ void page_values4(const void* pay, const void* sc, int64_t row,
                                             int d, int D, int g, float* o) {
  if constexpr (PREC == SI_PREC_FP32) {  // the input dtype
    if constexpr (SDT == SI_DT_F32) {
      const float4 x = *reinterpret_cast<const float4*>(reinterpret_cast<const float*>(pay) + row * D + d);
      o[0] = x.x; o[1] = x.y; o[2] = x.z; o[3] = x.w;
    } else {
      const uint2 x = *reinterpret_cast<const uint2*>(reinterpret_cast<const uint16_t*>(pay) + row * D + d);
      const uint32_t w[2] = {x.x, x.y};
#pragma unroll
      for (int i = 0; i < 2; ++i) {
        o[2 * i] = SDT == SI_DT_BF16 ? bf16_bits_to_f32(w[i] & 0xffffu) : f16_bits_to_f32(w[i] & 0xffffu);
        o[2 * i + 1] = SDT == SI_DT_BF16 ? bf16_bits_to_f32(w[i] >> 16) : f16_bits_to_f32(w[i] >> 16);
      }
    }
  } else if constexpr (PREC == SI_PREC_FP16) {
    const uint2 x = *reinterpret_cast<const uint2*>(reinterpret_cast<const uint16_t*>(pay) + row * D + d);
    o[0] = f16_bits_to_f32(x.x & 0xffffu);
    o[1] = f16_bits_to_f32(x.x >> 16);
    o[2] = f16_bits_to_f32(x.y & 0xffffu);
    o[3] = f16_bits_to_f32(x.y >> 16);
  } else if constexpr (PREC == SI_PREC_INT8) {
    const uint32_t x = *reinterpret_cast<const uint32_t*>(reinterpret_cast<const int8_t*>(pay) + row * D + d);
    const float s = load_any(sc, SDT, row);
#pragma unroll
    for (int i = 0; i < 4; ++i) o[i] = (float)(int8_t)(x >> (8 * i)) * s;
  } else {
    const uint32_t x = *reinterpret_cast<const uint16_t*>(reinterpret_cast<const uint8_t*>(pay) + row * (D / 2) + d / 2);
    const float s = load_any(sc, SDT, row * (D / g) + d / g);
    o[0] = (float)((int)((x >> 4) & 0xfu) - 8) * s;
    o[1] = (float)((int)(x & 0xfu) - 8) * s;
    o[2] = (float)((int)((x >> 12) & 0xfu) - 8) * s;
    o[3] = (float)((int)((x >> 8) & 0xfu) - 8) * s;
  }
}

template <int SDT, int PREC>
__device__ __forceinline__ void gather_page_vec(const PageRow& pr, int64_t bh, int64_t S, int D,
                                                int g, float* __restrict__ ok,
                                                float* __restrict__ ov) {
  typedef float f32x4 __attribute__((ext_vector_type(4)));
  const int n4 = (int)pr.ntok * (D / 4);
  const int q4 = D / 4;
  for (int i = threadIdx.x; i < n4; i += blockDim.x) {
    const int jt = i / q4;
    const int d = (i - jt * q4) * 4;
    const int64_t row = bh * pr.cap + jt;
    const int64_t o = (bh * S + pr.start + jt) * D + d;
    float a[4], b[4];
    page_values4<SDT, PREC>(reinterpret_cast<const void*>(pr.k), reinterpret_cast<const void*>(pr.sk), row, d, D, g, a);
    page_values4<SDT, PREC>(reinterpret_cast<const void*>(pr.v), reinterpret_cast<const void*>(pr.sv), row, d, D, g, b);
    __builtin_nontemporal_store(f32x4{a[0], a[1], a[2], a[3]}, reinterpret_cast<f32x4*>(ok + o));
    __builtin_nontemporal_store(f32x4{b[0], b[1], b[2], b[3]}, reinterpret_cast<f32x4*>(ov + o));
  }
}

// gather (:326-405): every page's rows decoded to fp32 [B, H, S, D] in one
// launch. Grid: blockIdx.x = page, blockIdx.y = b*H + h; each block reads its
// page's input dtype from the table (pages of one store may differ). VEC: four
// values of one group per thread, loads and 16-byte stores specialised for the
// page's precision (D % 4 == 0, group % 4 == 0, 16-byte aligned rows).
template <int SDT, bool VEC>
__device__ __forceinline__ void gather_page(const PageRow& pr, int64_t bh, int64_t S, int64_t D,
                                            int64_t g, float* __restrict__ ok,
                                            float* __restrict__ ov) {
  if constexpr (VEC) {
    switch ((int)pr.prec) {
      case SI_PREC_FP32: gather_page_vec<SDT, SI_PREC_FP32>(pr, bh, S, (int)D, (int)g, ok, ov); break;
      case SI_PREC_FP16: gather_page_vec<SDT, SI_PREC_FP16>(pr, bh, S, (int)D, (int)g, ok, ov); break;
      case SI_PREC_INT8: gather_page_vec<SDT, SI_PREC_INT8>(pr, bh, S, (int)D, (int)g, ok, ov); break;
      default: gather_page_vec<SDT, SI_PREC_INT4>(pr, bh, S, (int)D, (int)g, ok, ov); break;
    }
  } else {
    const int64_t n = pr.ntok * D;
    for (int64_t i = threadIdx.x; i < n; i += blockDim.x) {
      const int64_t jt = i / D;
      const int64_t d = i - jt * D;
      const int64_t row = bh * pr.cap + jt;
      const int64_t o = (bh * S + pr.start + jt) * D + d;
      ok[o] = page_value<SDT>(pr, 0, row, d, D, g);
      ov[o] = page_value<SDT>(pr, 1, row, d, D, g);
    }
  }
}

template <bool VEC>
__global__ __launch_bounds__(256) void page_gather_kernel(const int64_t* __restrict__ table,
                                                          int64_t S, int64_t D, int64_t g,
                                                          float* __restrict__ ok,
                                                          float* __restrict__ ov) {
  const int64_t* t = table + (int64_t)blockIdx.x * kPageRowWords;
  const PageRow pr{t[0], t[1], t[2], t[3], t[4], t[5], t[6], t[7], t[8]};
  const int64_t bh = blockIdx.y;
  switch ((int)pr.dt) {
    case SI_DT_F32: gather_page<SI_DT_F32, VEC>(pr, bh, S, D, g, ok, ov); break;
    case SI_DT_F16: gather_page<SI_DT_F16, VEC>(pr, bh, S, D, g, ok, ov); break;
    default: gather_page<SI_DT_BF16, VEC>(pr, bh, S, D, g, ok, ov); break;
  }
}

// ---------------------------------------------------------------------------
// Host side
// ---------------------------------------------------------------------------

unsigned grid_for(int64_t work_items, int per_block, int64_t cap = 262144) {
  int64_t blocks = ceil_div(work_items, per_block);
  if (blocks < 1) blocks = 1;
  if (blocks > cap) blocks = cap;
  return (unsigned)blocks;
}

bool pow2(int64_t x) { return x > 0 && (x & (x - 1)) == 0; }

template <int DT>
int launch_pack(const void* k, const void* v, int64_t B, int64_t H, int64_t S, int64_t D,
                int64_t g, const int8_t* code, const int32_t* slot, const Buckets& bk,
                const WorkCopy& wc, hipStream_t st) {
  constexpr int EPL = Chunk<DT>::EPL;
#ifndef SI_PACK_FAST_U
#define SI_PACK_FAST_U 1
#endif
  constexpr int U = SI_PACK_FAST_U;
  const int64_t lpr = D / EPL;
  const int64_t lpg = g / EPL;
  const bool aligned = ((reinterpret_cast<uintptr_t>(k) | reinterpret_cast<uintptr_t>(v) |
                         reinterpret_cast<uintptr_t>(wc.k) | reinterpret_cast<uintptr_t>(wc.v) |
                         reinterpret_cast<uintptr_t>(wc.kp) | reinterpret_cast<uintptr_t>(wc.vp)) &
                        15) == 0;
  const bool copy = wc.k != nullptr;
  const bool small = B * H < 65536 && S * H < ((int64_t)1 << 31) && B * H * S * D < ((int64_t)1 << 40);
  const bool fast = aligned && small && D % EPL == 0 && pow2(lpr) && lpr >= 4 && lpr <= 64 &&
                    g % EPL == 0 && pow2(lpg) && lpg <= lpr;
  if (fast) {
    const int rpb = (int)(256 / lpr) * U;
    const dim3 grid((unsigned)ceil_div(S, rpb), (unsigned)(B * H));
#define SI_PACK_CASE(L)                                                                     \
  case L:                                                                                   \
    if (copy)                                                                               \
      kv_pack_fast<DT, L, U, true><<<grid, 256, 0, st>>>(k, v, (int)B, (int)H, (int)S,      \
                                                         (int)lpg, code, slot, bk, wc);     \
    else                                                                                    \
      kv_pack_fast<DT, L, U, false><<<grid, 256, 0, st>>>(k, v, (int)B, (int)H, (int)S,     \
                                                          (int)lpg, code, slot, bk, wc);    \
    break;
    switch (lpr) {
      SI_PACK_CASE(4)
      SI_PACK_CASE(8)
      SI_PACK_CASE(16)
      SI_PACK_CASE(32)
      SI_PACK_CASE(64)
    }
#undef SI_PACK_CASE
    return check_launch("si_kv_pack/fast");
  }
  kv_pack_generic<DT><<<grid_for(S * H, 256), 256, 0, st>>>(k, v, B, H, S, D, g, code, slot, bk,
                                                              wc);
  return check_launch("si_kv_pack/generic");
}

template <int D>
void launch_unpack_sorted(int sdt, const int8_t* code, const int32_t* slot, const Buckets& bk,
                          int64_t B, int64_t H, int64_t S, int64_t g, float* ok, float* ov,
                          hipStream_t st) {
  constexpr int U = 2;
  const dim3 grid((unsigned)ceil_div(S, 64), (unsigned)(B * H));
  switch (sdt) {
    case SI_DT_F32:
      kv_unpack_sorted<D, SI_DT_F32, U><<<grid, 256, 0, st>>>(code, slot, bk, (int)B, (int)H, (int)S, (int)g, ok, ov);
      break;
    case SI_DT_F16:
      kv_unpack_sorted<D, SI_DT_F16, U><<<grid, 256, 0, st>>>(code, slot, bk, (int)B, (int)H, (int)S, (int)g, ok, ov);
      break;
    default:
      kv_unpack_sorted<D, SI_DT_BF16, U><<<grid, 256, 0, st>>>(code, slot, bk, (int)B, (int)H, (int)S, (int)g, ok, ov);
  }
}

}  // namespace
}  // namespace si

using namespace si;

extern "C" int si_kv_pack(const void* k, const void* v, int dtype, int64_t B, int64_t H,
                          int64_t S, int64_t D, int64_t group, const int8_t* code,
                          const int32_t* slot, void* const* buckets, si_stream_t stream) {
  clear_error();
  SI_CHECK_ARG(dtype_ok(dtype), "si_kv_pack: unsupported dtype %d", dtype);
  SI_CHECK_ARG(B >= 0 && H >= 0 && S >= 0 && D > 0, "si_kv_pack: bad shape");
  SI_CHECK_ARG(group > 0 && D % group == 0, "si_kv_pack: group %lld must divide D %lld",
               (long long)group, (long long)D);
  SI_CHECK_ARG(buckets != nullptr, "si_kv_pack: buckets table is NULL");
  if (B * H * S == 0) return SI_OK;
  SI_CHECK_ARG(k && v && code && slot, "si_kv_pack: NULL input");
  const Buckets bk = to_buckets(buckets);
  hipStream_t st = as_stream(stream);
  const WorkCopy none{nullptr, nullptr, nullptr, nullptr, nullptr};
  switch (dtype) {
    case SI_DT_F32: return launch_pack<SI_DT_F32>(k, v, B, H, S, D, group, code, slot, bk, none, st);
    case SI_DT_F16: return launch_pack<SI_DT_F16>(k, v, B, H, S, D, group, code, slot, bk, none, st);
    default: return launch_pack<SI_DT_BF16>(k, v, B, H, S, D, group, code, slot, bk, none, st);
  }
}

extern "C" int si_kv_pack_copy(const void* k, const void* v, int dtype, int64_t B, int64_t H,
                               int64_t S, int64_t D, int64_t group, const int8_t* code,
                               const int32_t* slot, void* const* buckets, const void* k_prev,
                               const void* v_prev, const uint8_t* reuse_mask, void* out_k,
                               void* out_v, si_stream_t stream) {
  clear_error();
  SI_CHECK_ARG(dtype_ok(dtype), "si_kv_pack_copy: unsupported dtype %d", dtype);
  SI_CHECK_ARG(B >= 0 && H >= 0 && S >= 0 && D > 0, "si_kv_pack_copy: bad shape");
  SI_CHECK_ARG(group > 0 && D % group == 0, "si_kv_pack_copy: group %lld must divide D %lld",
               (long long)group, (long long)D);
  SI_CHECK_ARG(buckets != nullptr, "si_kv_pack_copy: buckets table is NULL");
  if (B * H * S == 0) return SI_OK;
  SI_CHECK_ARG(k && v && code && slot && out_k && out_v, "si_kv_pack_copy: NULL input or output");
  SI_CHECK_ARG(reuse_mask == nullptr || (k_prev != nullptr && v_prev != nullptr),
               "si_kv_pack_copy: reuse_mask needs k_prev and v_prev");
  const Buckets bk = to_buckets(buckets);
  hipStream_t st = as_stream(stream);
  const WorkCopy wc{out_k, out_v, reuse_mask ? k_prev : nullptr, reuse_mask ? v_prev : nullptr,
                    reuse_mask};
  switch (dtype) {
    case SI_DT_F32: return launch_pack<SI_DT_F32>(k, v, B, H, S, D, group, code, slot, bk, wc, st);
    case SI_DT_F16: return launch_pack<SI_DT_F16>(k, v, B, H, S, D, group, code, slot, bk, wc, st);
    default: return launch_pack<SI_DT_BF16>(k, v, B, H, S, D, group, code, slot, bk, wc, st);
  }
}

extern "C" int si_kv_unpack(const int8_t* code, const int32_t* slot, const void* const* buckets,
                            int scale_dtype, int64_t B, int64_t H, int64_t S, int64_t D,
                            int64_t group, float* out_k, float* out_v, si_stream_t stream) {
  clear_error();
  SI_CHECK_ARG(dtype_ok(scale_dtype), "si_kv_unpack: unsupported scale dtype %d", scale_dtype);
  SI_CHECK_ARG(B >= 0 && H >= 0 && S >= 0 && D > 0, "si_kv_unpack: bad shape");
  SI_CHECK_ARG(group > 0 && D % group == 0, "si_kv_unpack: group must divide D");
  const int64_t total = B * H * S * D;
  if (total == 0) return SI_OK;
  SI_CHECK_ARG(code && slot && out_k && out_v && buckets, "si_kv_unpack: NULL argument");
  const Buckets bk = to_buckets(buckets);
  hipStream_t st = as_stream(stream);
  const bool vec = D % 4 == 0 && group % 4 == 0 &&
                   ((reinterpret_cast<uintptr_t>(out_k) | reinterpret_cast<uintptr_t>(out_v)) & 15) == 0;
  const bool small = B * H < 65536 && S * H < ((int64_t)1 << 31) && group < ((int64_t)1 << 31);
  if (vec && small && (D == 128 || D == 64)) {
    if (D == 128)
      launch_unpack_sorted<128>(scale_dtype, code, slot, bk, B, H, S, group, out_k, out_v, st);
    else
      launch_unpack_sorted<64>(scale_dtype, code, slot, bk, B, H, S, group, out_k, out_v, st);
    return check_launch("si_kv_unpack/fast");
  }
  if (vec) {
    const unsigned grid = grid_for(total / 4, 256);
    switch (scale_dtype) {
      case SI_DT_F32:
        kv_unpack_vec4<SI_DT_F32><<<grid, 256, 0, st>>>(code, slot, bk, B, H, S, D, group, out_k, out_v);
        break;
      case SI_DT_F16:
        kv_unpack_vec4<SI_DT_F16><<<grid, 256, 0, st>>>(code, slot, bk, B, H, S, D, group, out_k, out_v);
        break;
      default:
        kv_unpack_vec4<SI_DT_BF16><<<grid, 256, 0, st>>>(code, slot, bk, B, H, S, D, group, out_k, out_v);
    }
    return check_launch("si_kv_unpack/vec4");
  }
  kv_unpack_generic<<<grid_for(total, 256), 256, 0, st>>>(code, slot, bk, scale_dtype, B, H, S, D,
                                                         group, out_k, out_v);
  return check_launch("si_kv_unpack/generic");
}

extern "C" int si_kv_reuse(const int8_t* cur_code, const int32_t* cur_slot, void* const* cur_buckets,
                           int64_t S, const int8_t* prev_code, const int32_t* prev_slot,
                           const void* const* prev_buckets, int64_t S_prev, const uint8_t* mask,
                           int64_t H, int64_t B, int64_t D, int64_t group, int scale_dtype,
                           int64_t* stats, si_stream_t stream) {
  clear_error();
  SI_CHECK_ARG(dtype_ok(scale_dtype), "si_kv_reuse: unsupported scale dtype %d", scale_dtype);
  SI_CHECK_ARG(S >= 0 && S_prev >= 0 && H >= 0 && B >= 0 && D > 0, "si_kv_reuse: bad shape");
  SI_CHECK_ARG(group > 0 && D % group == 0, "si_kv_reuse: group must divide D");
  const int64_t n = S * H;
  if (n == 0) return SI_OK;
  SI_CHECK_ARG(cur_code && cur_slot && mask && cur_buckets && prev_buckets,
               "si_kv_reuse: NULL argument");
  SI_CHECK_ARG(S_prev == 0 || (prev_code && prev_slot), "si_kv_reuse: NULL previous plan");
  SI_CHECK_ARG(n < ((int64_t)1 << 31), "si_kv_reuse: S * H must be < 2^31");
  const RowGeom geo = make_geom(B, D, group, scale_dtype);
  kv_reuse_tiles<<<(unsigned)ceil_div(n, kTileEntries), kTileThreads, 0, as_stream(stream)>>>(
      cur_code, cur_slot, to_buckets(cur_buckets), S, prev_code, prev_slot,
      to_buckets(prev_buckets), S_prev, mask, H, geo,
      reinterpret_cast<unsigned long long*>(stats));
  return check_launch("si_kv_reuse");
}

extern "C" int si_kv_compact(const int8_t* old_code, const int32_t* old_slot,
                             const void* const* old_buckets, const int8_t* new_code,
                             const int32_t* new_slot, void* const* new_buckets, int64_t n,
                             int64_t B, int64_t D, int64_t group, int scale_dtype,
                             si_stream_t stream) {
  clear_error();
  SI_CHECK_ARG(dtype_ok(scale_dtype), "si_kv_compact: unsupported scale dtype %d", scale_dtype);
  SI_CHECK_ARG(n >= 0 && B >= 0 && D > 0, "si_kv_compact: bad shape");
  SI_CHECK_ARG(group > 0 && D % group == 0, "si_kv_compact: group must divide D");
  if (n == 0) return SI_OK;
  SI_CHECK_ARG(old_code && old_slot && new_code && new_slot && old_buckets && new_buckets,
               "si_kv_compact: NULL argument");
  const RowGeom geo = make_geom(B, D, group, scale_dtype);
  kv_compact_kernel<<<grid_for(n * kCopyLanes, 256), 256, 0, as_stream(stream)>>>(
      old_code, old_slot, to_buckets(old_buckets), new_code, new_slot, to_buckets(new_buckets), n,
      geo);
  return check_launch("si_kv_compact");
}

extern "C" int si_kv_reuse_flat(const int64_t* const* cur_flat, const int64_t* cur_counts,
                                void* const* cur_buckets, int64_t S, const int8_t* prev_code,
                                const int32_t* prev_slot, const void* const* prev_buckets,
                                int64_t S_prev, const uint8_t* mask, int64_t H, int64_t B,
                                int64_t D, int64_t group, int scale_dtype, int64_t* stats,
                                si_stream_t stream) {
  clear_error();
  SI_CHECK_ARG(dtype_ok(scale_dtype), "si_kv_reuse_flat: unsupported scale dtype %d", scale_dtype);
  SI_CHECK_ARG(S >= 0 && S_prev >= 0 && H >= 0 && B >= 0 && D > 0, "si_kv_reuse_flat: bad shape");
  SI_CHECK_ARG(group > 0 && D % group == 0, "si_kv_reuse_flat: group must divide D");
  if (S * H == 0 || S_prev == 0) return SI_OK;
  SI_CHECK_ARG(cur_flat && cur_counts && cur_buckets && prev_code && prev_slot && prev_buckets && mask,
               "si_kv_reuse_flat: NULL argument");
  const Buckets dst = to_buckets(cur_buckets);
  CopyLists L;
  const int64_t blocks = copy_lists_setup(L, cur_flat, cur_counts, dst);
  for (int p = 0; p < 4; ++p)
    SI_CHECK_ARG(L.n[p] == 0 || L.flat[p] != nullptr, "si_kv_reuse_flat: NULL list %d", p);
  if (blocks == 0) return SI_OK;
  SI_CHECK_ARG(blocks < ((int64_t)1 << 31), "si_kv_reuse_flat: too many blocks");
  const RowGeom geo = make_geom(B, D, group, scale_dtype);
  if (list_rows_wide(B, D))
    kv_copy_lists<true, true><<<(unsigned)blocks, 256, 0, as_stream(stream)>>>(
        L, dst, to_buckets(prev_buckets), prev_code, prev_slot, mask, S, H, S_prev, geo,
        reinterpret_cast<unsigned long long*>(stats));
  else
    kv_copy_lists<true, false><<<(unsigned)blocks, 256, 0, as_stream(stream)>>>(
        L, dst, to_buckets(prev_buckets), prev_code, prev_slot, mask, S, H, S_prev, geo,
        reinterpret_cast<unsigned long long*>(stats));
  return check_launch("si_kv_reuse_flat");
}

extern "C" int si_kv_compact_flat(const int32_t* old_slot, const void* const* old_buckets,
                                  const int64_t* const* new_flat, const int64_t* new_counts,
                                  void* const* new_buckets, int64_t S, int64_t H, int64_t B,
                                  int64_t D, int64_t group, int scale_dtype, si_stream_t stream) {
  clear_error();
  SI_CHECK_ARG(dtype_ok(scale_dtype), "si_kv_compact_flat: unsupported scale dtype %d",
               scale_dtype);
  SI_CHECK_ARG(S >= 0 && H >= 0 && B >= 0 && D > 0, "si_kv_compact_flat: bad shape");
  SI_CHECK_ARG(group > 0 && D % group == 0, "si_kv_compact_flat: group must divide D");
  if (S * H == 0) return SI_OK;
  SI_CHECK_ARG(old_slot && old_buckets && new_flat && new_counts && new_buckets,
               "si_kv_compact_flat: NULL argument");
  const Buckets dst = to_buckets(new_buckets);
  CopyLists L;
  const int64_t blocks = copy_lists_setup(L, new_flat, new_counts, dst);
  for (int p = 0; p < 4; ++p)
    SI_CHECK_ARG(L.n[p] == 0 || L.flat[p] != nullptr, "si_kv_compact_flat: NULL list %d", p);
  if (blocks == 0) return SI_OK;
  SI_CHECK_ARG(blocks < ((int64_t)1 << 31), "si_kv_compact_flat: too many blocks");
  const RowGeom geo = make_geom(B, D, group, scale_dtype);
  if (list_rows_wide(B, D))
    kv_copy_lists<false, true><<<(unsigned)blocks, 256, 0, as_stream(stream)>>>(
        L, dst, to_buckets(old_buckets), nullptr, old_slot, nullptr, S, H, S, geo, nullptr);
  else
    kv_copy_lists<false, false><<<(unsigned)blocks, 256, 0, as_stream(stream)>>>(
        L, dst, to_buckets(old_buckets), nullptr, old_slot, nullptr, S, H, S, geo, nullptr);
  return check_launch("si_kv_compact_flat");
}

extern "C" int64_t si_kv_evict_chunk_words(void) { return kEvictWords; }

extern "C" int64_t si_kv_evict_chunks(const int64_t* old_counts) {
  if (old_counts == nullptr) return -1;
  int64_t acc = 0;
  for (int p = 0; p < 4; ++p) {
    if (old_counts[p] < 0) return -1;
    acc += ceil_div(old_counts[p], (int64_t)kEvictRows);
  }
  return acc;
}

namespace {
int evict_check_lists(const int64_t* const* old_flat, const int64_t* old_counts, int64_t n,
                      const char* who) {
  int64_t listed = 0;
  for (int p = 0; p < 4; ++p) {
    SI_CHECK_ARG(old_counts[p] >= 0, "%s: negative bucket size %lld", who, (long long)old_counts[p]);
    SI_CHECK_ARG(old_counts[p] == 0 || old_flat[p] != nullptr, "%s: NULL list %d", who, p);
    listed += old_counts[p];
  }
  SI_CHECK_ARG(listed <= n, "%s: the lists hold %lld entries, the code matrix %lld", who,
               (long long)listed, (long long)n);
  return SI_OK;
}
}  // namespace

extern "C" int si_kv_evict_count(const int8_t* old_code, const int64_t* const* old_flat,
                                 const int64_t* old_counts, const uint8_t* evict_mask, int64_t S,
                                 int64_t H, int8_t* new_code, int32_t* new_slot,
                                 int32_t* chunk_counts, uint64_t* chunk_bits, si_stream_t stream) {
  clear_error();
  SI_CHECK_ARG(S >= 0 && H >= 0, "si_kv_evict_count: negative shape");
  const int64_t n = S * H;
  if (n == 0) return SI_OK;
  SI_CHECK_ARG(old_code && old_flat && old_counts && evict_mask && new_code && new_slot,
               "si_kv_evict_count: NULL argument");
  SI_CHECK_ARG(n < ((int64_t)1 << 31), "si_kv_evict_count: %lld entries (slots are int32)",
               (long long)n);
  if (int rc = evict_check_lists(old_flat, old_counts, n, "si_kv_evict_count")) return rc;
  EvictLists L;
  const int64_t chunks = evict_lists_setup(L, old_flat, old_counts);
  SI_CHECK_ARG(chunks == 0 || (chunk_counts != nullptr && chunk_bits != nullptr),
               "si_kv_evict_count: NULL chunk counts or bits");
  const int64_t fix = ceil_div(n, (int64_t)kEvictRows * kEvictFixEntries);
  kv_evict_count<<<(unsigned)(chunks + fix), kEvictRows, 0, as_stream(stream)>>>(
      L, chunks, old_code, evict_mask, S, H, new_code, new_slot, chunk_counts,
      reinterpret_cast<unsigned long long*>(chunk_bits));
  return check_launch("si_kv_evict_count");
}

extern "C" int si_kv_evict_flat(const int64_t* const* old_flat, const int64_t* old_counts,
                                const int32_t* chunk_counts, const uint64_t* chunk_bits, int64_t S,
                                int64_t H, const void* const* old_buckets,
                                int64_t* const* new_flat, const int64_t* new_counts,
                                void* const* new_buckets, int32_t* new_slot, int64_t B, int64_t D,
                                int64_t group, int scale_dtype, si_stream_t stream) {
  clear_error();
  SI_CHECK_ARG(dtype_ok(scale_dtype), "si_kv_evict_flat: unsupported scale dtype %d", scale_dtype);
  SI_CHECK_ARG(S >= 0 && H >= 0 && B >= 0 && D > 0, "si_kv_evict_flat: bad shape");
  SI_CHECK_ARG(group > 0 && D % group == 0, "si_kv_evict_flat: group must divide D");
  const int64_t n = S * H;
  if (n == 0) return SI_OK;
  SI_CHECK_ARG(old_flat && old_counts && old_buckets && new_flat && new_counts && new_buckets &&
                   new_slot,
               "si_kv_evict_flat: NULL argument");
  SI_CHECK_ARG(n < ((int64_t)1 << 31), "si_kv_evict_flat: %lld entries (slots are int32)",
               (long long)n);
  if (int rc = evict_check_lists(old_flat, old_counts, n, "si_kv_evict_flat")) return rc;
  EvictLists L;
  const int64_t chunks = evict_lists_setup(L, old_flat, old_counts);
  if (chunks == 0) return SI_OK;
  SI_CHECK_ARG(chunk_counts != nullptr && chunk_bits != nullptr,
               "si_kv_evict_flat: NULL chunk counts or bits");
  NewLists nl;
  for (int p = 0; p < 4; ++p) {
    SI_CHECK_ARG(new_counts[p] >= 0 && new_counts[p] <= old_counts[p],
                 "si_kv_evict_flat: new bucket %d holds %lld rows, the old one %lld", p,
                 (long long)new_counts[p], (long long)old_counts[p]);
    nl.flat[p] = new_flat[p];
    nl.n[p] = new_counts[p];
    const bool copy = new_buckets[4 * p] != nullptr;
    for (int j = 0; j < 4; ++j) {
      if (j >= 2 && p < 2) continue;  // fp32 / fp16 have no scales
      SI_CHECK_ARG(!copy || (new_buckets[4 * p + j] != nullptr && old_buckets[4 * p + j] != nullptr),
                   "si_kv_evict_flat: precision %d: NULL bucket tensor %d", p, j);
    }
  }
  const RowGeom geo = make_geom(B, D, group, scale_dtype);
  const Buckets dst = to_buckets(new_buckets), src = to_buckets(old_buckets);
  if (B * D * 4 * kEvictRows >= ((int64_t)1 << 32))  // 32-bit unit indices up to here
    kv_evict_lists<true><<<(unsigned)chunks, kEvictThreads, 0, as_stream(stream)>>>(
        L, chunk_counts, reinterpret_cast<const unsigned long long*>(chunk_bits), S, H, dst, src,
        geo, nl, new_slot);
  else
    kv_evict_lists<false><<<(unsigned)chunks, kEvictThreads, 0, as_stream(stream)>>>(
        L, chunk_counts, reinterpret_cast<const unsigned long long*>(chunk_bits), S, H, dst, src,
        geo, nl, new_slot);
  return check_launch("si_kv_evict_flat");
}

namespace {
int page_write_run(const void* k, const void* v, int dtype, int64_t B, int64_t H, int64_t T,
                   int64_t D, int64_t t0, int64_t take, int precision, int64_t group,
                   void* const* page, int64_t capacity, int64_t offset, int64_t n_pages,
                   si_stream_t stream) {
  SI_CHECK_ARG(dtype_ok(dtype), "si_page_write: unsupported dtype %d", dtype);
  SI_CHECK_ARG(precision >= SI_PREC_FP32 && precision <= SI_PREC_INT4,
               "si_page_write: precision %d is not 0..3", precision);
  SI_CHECK_ARG(B >= 0 && H >= 0 && T >= 0 && D > 0 && take >= 0 && t0 >= 0 && t0 + take <= T,
               "si_page_write: tokens [%lld, %lld) outside [0, %lld)", (long long)t0,
               (long long)(t0 + take), (long long)T);
  SI_CHECK_ARG(n_pages >= 1 && capacity > 0 && offset >= 0 && offset + take <= capacity * n_pages,
               "si_page_write: rows [%lld, %lld) outside %lld page(s) of %lld rows",
               (long long)offset, (long long)(offset + take), (long long)n_pages,
               (long long)capacity);
  SI_CHECK_ARG(group > 0 && D % group == 0, "si_page_write: group must divide D");
  if (B * H * take == 0) return SI_OK;
  SI_CHECK_ARG(k && v && page && page[0] && page[1], "si_page_write: NULL argument");
  SI_CHECK_ARG(precision < SI_PREC_INT8 || (page[2] && page[3]), "si_page_write: NULL scales");
  SI_CHECK_ARG(B * H < 65536 && B * H * capacity * n_pages < ((int64_t)1 << 31),
               "si_page_write: store too large for one launch");
  Buckets pg = to_buckets(nullptr);
  const int base = precision == SI_PREC_FP32 ? 0 : 4 * precision;
  for (int j = 0; j < 4; ++j) pg.p[base + j] = page[j];
  hipStream_t st = as_stream(stream);
  const int es = dtype_size(dtype);
  const int epl = 16 / es;
  const int64_t lpr = D / epl;
  const int64_t lpg = group / epl;
  uintptr_t bits = reinterpret_cast<uintptr_t>(k) | reinterpret_cast<uintptr_t>(v);
  for (int j = 0; j < 4; ++j) bits |= reinterpret_cast<uintptr_t>(page[j]);
  const bool fast = (bits & 15) == 0 && D % epl == 0 && pow2(lpr) && lpr >= 4 && lpr <= 64 &&
                    group % epl == 0 && pow2(lpg) && lpg <= lpr && T < ((int64_t)1 << 31);
  if (fast) {
    const int rpb = (int)(256 / lpr);
    const dim3 grid((unsigned)ceil_div(take, rpb), (unsigned)(B * H));
#define SI_PW(DT_, L)                                                                         \
  page_write_fast<DT_, L><<<grid, 256, 0, st>>>(k, v, (int)T, (int)t0, (int)take, (int)capacity, \
                                               (int)offset, precision, (int)lpg, pg)
#define SI_PW_DT(DT_)              \
  switch (lpr) {                   \
    case 4: SI_PW(DT_, 4); break;  \
    case 8: SI_PW(DT_, 8); break;  \
    case 16: SI_PW(DT_, 16); break; \
    case 32: SI_PW(DT_, 32); break; \
    default: SI_PW(DT_, 64); break; \
  }
    if (dtype == SI_DT_F32) { SI_PW_DT(SI_DT_F32) }
    else if (dtype == SI_DT_F16) { SI_PW_DT(SI_DT_F16) }
    else { SI_PW_DT(SI_DT_BF16) }
#undef SI_PW_DT
#undef SI_PW
    return check_launch("si_page_write/fast");
  }
  const unsigned grid = grid_for(B * H * take, 256);
  if (dtype == SI_DT_F32)
    page_write_generic<SI_DT_F32><<<grid, 256, 0, st>>>(k, v, B * H, T, D, t0, take, capacity, offset, precision, group, pg);
  else if (dtype == SI_DT_F16)
    page_write_generic<SI_DT_F16><<<grid, 256, 0, st>>>(k, v, B * H, T, D, t0, take, capacity, offset, precision, group, pg);
  else
    page_write_generic<SI_DT_BF16><<<grid, 256, 0, st>>>(k, v, B * H, T, D, t0, take, capacity, offset, precision, group, pg);
  return check_launch("si_page_write/generic");
}
}  // namespace

extern "C" int si_page_write(const void* k, const void* v, int dtype, int64_t B, int64_t H,
                             int64_t T, int64_t D, int64_t t0, int64_t take, int precision,
                             int64_t group, void* const* page, int64_t capacity, int64_t offset,
                             si_stream_t stream) {
  clear_error();
  return page_write_run(k, v, dtype, B, H, T, D, t0, take, precision, group, page, capacity,
                        offset, 1, stream);
}

extern "C" int si_page_write_pages(const void* k, const void* v, int dtype, int64_t B, int64_t H,
                                   int64_t T, int64_t D, int64_t t0, int64_t n_pages,
                                   int precision, int64_t group, void* const* pages,
                                   int64_t capacity, si_stream_t stream) {
  clear_error();
  return page_write_run(k, v, dtype, B, H, T, D, t0, n_pages * capacity, precision, group, pages,
                        capacity, 0, n_pages, stream);
}

extern "C" int si_page_gather(const int64_t* table, int64_t n_pages, int64_t B, int64_t H,
                              int64_t S, int64_t D, int64_t group, float* out_k, float* out_v,
                              si_stream_t stream) {
  clear_error();
  SI_CHECK_ARG(n_pages >= 0 && B >= 0 && H >= 0 && S >= 0 && D > 0, "si_page_gather: bad shape");
  SI_CHECK_ARG(group > 0 && D % group == 0, "si_page_gather: group must divide D");
  if (n_pages == 0 || B * H == 0) return SI_OK;
  SI_CHECK_ARG(table && out_k && out_v, "si_page_gather: NULL argument");
  SI_CHECK_ARG(B * H < 65536 && n_pages < ((int64_t)1 << 31), "si_page_gather: too many pages");
  const dim3 grid((unsigned)n_pages, (unsigned)(B * H));
  // The vector path also needs aligned page rows: every page buffer is a
  // fresh allocation and rows are D values long, so D % 4 == 0 keeps the 4-,
  // 8- and 16-byte loads aligned.
  const bool vec = D % 4 == 0 && group % 4 == 0 && D < (1 << 20) &&
                   ((reinterpret_cast<uintptr_t>(out_k) | reinterpret_cast<uintptr_t>(out_v)) & 15) == 0;
  hipStream_t st = as_stream(stream);
  if (vec) page_gather_kernel<true><<<grid, 256, 0, st>>>(table, S, D, group, out_k, out_v);
  else page_gather_kernel<false><<<grid, 256, 0, st>>>(table, S, D, group, out_k, out_v);
  return check_launch("si_page_gather");
}

extern "C" int si_kv_unpack_flat(const int8_t* code, const int32_t* slot,
                                 const int64_t* const* flat, const int64_t* counts,
                                 const void* const* buckets, int scale_dtype, int64_t B,
                                 int64_t H, int64_t S, int64_t D, int64_t group, float* out_k,
                                 float* out_v, si_stream_t stream) {
  clear_error();
  SI_CHECK_ARG(dtype_ok(scale_dtype), "si_kv_unpack_flat: unsupported scale dtype %d", scale_dtype);
  SI_CHECK_ARG(B >= 0 && H >= 0 && S >= 0 && D > 0, "si_kv_unpack_flat: bad shape");
  SI_CHECK_ARG(group > 0 && D % group == 0, "si_kv_unpack_flat: group must divide D");
  const int64_t total = B * H * S * D;
  if (total == 0) return SI_OK;
  SI_CHECK_ARG(code && slot && flat && counts && out_k && out_v && buckets,
               "si_kv_unpack_flat: NULL argument");
  int64_t nsum = 0;
  for (int p = 0; p < 5; ++p) {
    SI_CHECK_ARG(counts[p] >= 0, "si_kv_unpack_flat: negative count");
    nsum += counts[p];
  }
  SI_CHECK_ARG(nsum == H * S, "si_kv_unpack_flat: counts sum to %lld, not S*H = %lld",
               (long long)nsum, (long long)(H * S));
  for (int p = 0; p < 4; ++p)
    SI_CHECK_ARG(counts[p] == 0 || flat[p] != nullptr, "si_kv_unpack_flat: NULL flat list %d", p);
  const bool vec = group % 4 == 0 &&
                   ((reinterpret_cast<uintptr_t>(out_k) | reinterpret_cast<uintptr_t>(out_v)) & 15) == 0;
  const bool small = B * H * S < ((int64_t)1 << 31) && B < ((int64_t)1 << 31);
  if (!(vec && small && (D == 128 || D == 64)))  // other shapes: the token-order kernels
    return si_kv_unpack(code, slot, buckets, scale_dtype, B, H, S, D, group, out_k, out_v, stream);
  const Buckets bk = to_buckets(buckets);
  // Rows per thread (U) and threads per block (NT) of the bucket-order pack and
  // unpack are compile-time constants (-D overrides for tuning builds). On a
  // 7B-shaped layer one row per thread is fastest: unpack 55.8 us (U = 2:
  // 55.9, 4: 58.8, 8: 62.3), pack 43.2 us (U = 2: 46.1, 4: 49.4, 8: 56.5);
  // 64- to 512-thread blocks are within 2% of each other.
#ifndef SI_UNPACK_LISTS_U
#define SI_UNPACK_LISTS_U 1
#endif
  constexpr int U = SI_UNPACK_LISTS_U;
#ifndef SI_UNPACK_LISTS_NT
#define SI_UNPACK_LISTS_NT 256
#endif
  constexpr int NT = SI_UNPACK_LISTS_NT;
  const int64_t rpb = (NT / (D / 4)) * U;
  UnpackLists L;
  int64_t acc = 0;
  for (int p = 0; p < 4; ++p) {
    L.flat[p] = flat[p];
    L.n[p] = counts[p];
    acc += ceil_div(counts[p] * B, rpb);
    L.blk_end[p] = acc;
  }
  L.blk_end[4] = acc + (counts[4] > 0 ? ceil_div(H * S, rpb) : 0);
  SI_CHECK_ARG(L.blk_end[4] < ((int64_t)1 << 31), "si_kv_unpack_flat: too many blocks");
  if (L.blk_end[4] == 0) return SI_OK;
  const dim3 grid((unsigned)L.blk_end[4]);
  hipStream_t st = as_stream(stream);
#define SI_UL(D_, SDT_) \
  kv_unpack_lists<D_, SDT_, U, NT><<<grid, NT, 0, st>>>(L, code, bk, (int)B, (int)H, (int)S, (int)group, out_k, out_v)
  if (D == 128) {
    if (scale_dtype == SI_DT_F32) SI_UL(128, SI_DT_F32);
    else if (scale_dtype == SI_DT_F16) SI_UL(128, SI_DT_F16);
    else SI_UL(128, SI_DT_BF16);
  } else {
    if (scale_dtype == SI_DT_F32) SI_UL(64, SI_DT_F32);
    else if (scale_dtype == SI_DT_F16) SI_UL(64, SI_DT_F16);
    else SI_UL(64, SI_DT_BF16);
  }
#undef SI_UL
  return check_launch("si_kv_unpack_flat");
}

extern "C" int si_kv_pack_flat(const void* k, const void* v, int dtype, int64_t B, int64_t H,
                               int64_t S, int64_t D, int64_t group, const int8_t* code,
                               const int32_t* slot, const int64_t* const* flat,
                               const int64_t* counts, void* const* buckets, si_stream_t stream) {
  clear_error();
  SI_CHECK_ARG(dtype_ok(dtype), "si_kv_pack_flat: unsupported dtype %d", dtype);
  SI_CHECK_ARG(B >= 0 && H >= 0 && S >= 0 && D > 0, "si_kv_pack_flat: bad shape");
  SI_CHECK_ARG(group > 0 && D % group == 0, "si_kv_pack_flat: group must divide D");
  SI_CHECK_ARG(buckets != nullptr && flat != nullptr && counts != nullptr,
               "si_kv_pack_flat: NULL table");
  if (B * H * S == 0) return SI_OK;
  int64_t nsum = 0;
  for (int p = 0; p < 5; ++p) {
    SI_CHECK_ARG(counts[p] >= 0, "si_kv_pack_flat: negative count");
    nsum += counts[p];
  }
  SI_CHECK_ARG(nsum == H * S, "si_kv_pack_flat: counts sum to %lld, not S*H = %lld",
               (long long)nsum, (long long)(H * S));
  for (int p = 0; p < 4; ++p)
    SI_CHECK_ARG(counts[p] == 0 || flat[p] != nullptr, "si_kv_pack_flat: NULL flat list %d", p);
  const Buckets bk = to_buckets(buckets);
  hipStream_t st = as_stream(stream);
  const int es = dtype_size(dtype);
  const int epl = 16 / es;
  const int64_t lpr = D / epl;
  const int64_t lpg = group / epl;
  const bool aligned = ((reinterpret_cast<uintptr_t>(k) | reinterpret_cast<uintptr_t>(v)) & 15) == 0;
  const bool fast = aligned && D % epl == 0 && pow2(lpr) && lpr >= 4 && lpr <= 64 &&
                    group % epl == 0 && pow2(lpg) && lpg <= lpr && B * H * S < ((int64_t)1 << 31);
  if (!fast) return si_kv_pack(k, v, dtype, B, H, S, D, group, code, slot, buckets, stream);
#ifndef SI_PACK_LISTS_U
#define SI_PACK_LISTS_U 1
#endif
  constexpr int U = SI_PACK_LISTS_U;
#ifndef SI_PACK_LISTS_NT
#define SI_PACK_LISTS_NT 256
#endif
  constexpr int NT = SI_PACK_LISTS_NT;
  const int64_t rpb = (NT / lpr) * U;
  UnpackLists L;
  int64_t acc = 0;
  for (int p = 0; p < 4; ++p) {
    L.flat[p] = flat[p];
    L.n[p] = counts[p];
    acc += ceil_div(counts[p] * B, rpb);
    L.blk_end[p] = acc;
  }
  L.blk_end[4] = acc;
  if (acc == 0) return SI_OK;
  SI_CHECK_ARG(acc < ((int64_t)1 << 31), "si_kv_pack_flat: too many blocks");
  const dim3 grid((unsigned)acc);
#define SI_PL(DT_, L_) \
  kv_pack_lists<DT_, L_, U, NT><<<grid, NT, 0, st>>>(k, v, L, (int)B, (int)H, (int)S, (int)lpg, bk)
#define SI_PL_DT(DT_)               \
  switch (lpr) {                    \
    case 4: SI_PL(DT_, 4); break;   \
    case 8: SI_PL(DT_, 8); break;   \
    case 16: SI_PL(DT_, 16); break; \
    case 32: SI_PL(DT_, 32); break; \
    default: SI_PL(DT_, 64); break; \
  }
  if (dtype == SI_DT_F32) { SI_PL_DT(SI_DT_F32) }
  else if (dtype == SI_DT_F16) { SI_PL_DT(SI_DT_F16) }
  else { SI_PL_DT(SI_DT_BF16) }
#undef SI_PL_DT
#undef SI_PL
  return check_launch("si_kv_pack_flat");
}

extern "C" int si_kv_pack_rope_flat(const void* qkv, const void* cos, const void* sin, int dtype,
                                    int64_t B, int64_t H, int64_t S, int64_t D, int64_t group,
                                    const int8_t* code, const int32_t* slot,
                                    const int64_t* const* flat, const int64_t* counts,
                                    void* const* buckets, si_stream_t stream) {
  clear_error();
  SI_CHECK_ARG(dtype == SI_DT_BF16 || dtype == SI_DT_F16,
               "si_kv_pack_rope_flat: dtype must be bf16 or fp16 (got %d)", dtype);
  SI_CHECK_ARG(B >= 0 && H >= 0 && S >= 0 && (D == 64 || D == 128),
               "si_kv_pack_rope_flat: bad shape (D must be 64 or 128)");
  SI_CHECK_ARG(group > 0 && D % group == 0 && group % 8 == 0 && pow2(group / 8),
               "si_kv_pack_rope_flat: group must divide D and be 8 times a power of two");
  SI_CHECK_ARG(buckets != nullptr && flat != nullptr && counts != nullptr,
               "si_kv_pack_rope_flat: NULL table");
  SI_CHECK_ARG(B * H * S < ((int64_t)1 << 31) && S < ((int64_t)1 << 31),
               "si_kv_pack_rope_flat: too many rows");
  if (B * H * S == 0) return SI_OK;
  SI_CHECK_ARG(qkv != nullptr && cos != nullptr && sin != nullptr,
               "si_kv_pack_rope_flat: NULL argument");
  SI_CHECK_ARG(((reinterpret_cast<uintptr_t>(qkv) | reinterpret_cast<uintptr_t>(cos) |
                 reinterpret_cast<uintptr_t>(sin)) & 15) == 0,
               "si_kv_pack_rope_flat: qkv, cos and sin must be 16-byte aligned");
  int64_t nsum = 0;
  for (int p = 0; p < 5; ++p) {
    SI_CHECK_ARG(counts[p] >= 0, "si_kv_pack_rope_flat: negative count");
    nsum += counts[p];
  }
  SI_CHECK_ARG(nsum == H * S, "si_kv_pack_rope_flat: counts sum to %lld, not S*H = %lld",
               (long long)nsum, (long long)(H * S));
  for (int p = 0; p < 4; ++p)
    SI_CHECK_ARG(counts[p] == 0 || flat[p] != nullptr, "si_kv_pack_rope_flat: NULL flat list %d",
                 p);
  const Buckets bk = to_buckets(buckets);
  hipStream_t st = as_stream(stream);
  constexpr int U = SI_PACK_LISTS_U;
  constexpr int NT = SI_PACK_LISTS_NT;
  const int64_t lpr = D / 8;
  const int64_t lpg = group / 8;
  const int64_t rpb = (NT / lpr) * U;
  UnpackLists L;
  int64_t acc = 0;
  for (int p = 0; p < 4; ++p) {
    L.flat[p] = flat[p];
    L.n[p] = counts[p];
    acc += ceil_div(counts[p] * B, rpb);
    L.blk_end[p] = acc;
  }
  L.blk_end[4] = acc;
  if (acc == 0) return SI_OK;
  const dim3 grid((unsigned)acc);
  const RopeSrc rs{qkv, cos, sin, (int)S, (int)H};
#define SI_PR(DT_, L_)                                                                   \
  kv_pack_lists<DT_, L_, U, NT, true><<<grid, NT, 0, st>>>(nullptr, nullptr, L, (int)B, (int)H, \
                                                          (int)S, (int)lpg, bk, rs)
  if (dtype == SI_DT_F16) {
    if (lpr == 8) SI_PR(SI_DT_F16, 8); else SI_PR(SI_DT_F16, 16);
  } else {
    if (lpr == 8) SI_PR(SI_DT_BF16, 8); else SI_PR(SI_DT_BF16, 16);
  }
#undef SI_PR
  return check_launch("si_kv_pack_rope_flat");
}
