/*
 * Oracle: plain-C restatement of the reference's quantized data-plane arithmetic.
 *
 * TEST INFRASTRUCTURE ONLY. Nothing in the product (shadow-infer_amd/) links,
 * loads or calls this file; only tests/, __graft_entry__.smoke() and bench.py's
 * cpu_baseline leg use it, as the checker.
 *
 * Every routine restates the torch op chain that the reference runs on the CPU,
 * with the same rounding at every step. dtype codes: 0 = fp32, 1 = fp16, 2 = bf16.
 * fp16 and bf16 values travel as uint16_t bit patterns.
 *
 * Built with -O2 -ffp-contract=off so that no multiply-add is fused: each
 * operation rounds exactly as the corresponding torch CPU kernel does.
 */
#include <math.h>
#include <stdint.h>
#include <string.h>

/* ------------------------------------------------------------------------ */
/* Scalar conversions (IEEE round-to-nearest-even).                         */
/* ------------------------------------------------------------------------ */

static inline float bits_to_f32(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }
static inline uint32_t f32_to_bits(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }

/* bf16 -> fp32 is exact: the bf16 pattern is the top half of an fp32. */
float or_bf16_to_f32(uint16_t h) { return bits_to_f32((uint32_t)h << 16); }

/* fp32 -> bf16, round to nearest even; NaN -> canonical quiet NaN 0x7FC0
 * (c10::BFloat16 round_to_nearest_even behaviour). */
uint16_t or_f32_to_bf16(float f) {
  uint32_t u = f32_to_bits(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return 0x7fc0;
  u += 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}

/* fp16 -> fp32 (exact). */
float or_f16_to_f32(uint16_t h) {
  uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
  uint32_t exp = (h >> 10) & 0x1fu;
  uint32_t man = h & 0x3ffu;
  if (exp == 0x1fu) return bits_to_f32(sign | 0x7f800000u | (man << 13));
  if (exp == 0) {
    /* zero or subnormal: man * 2^-24, exact in fp32 */
    float v = (float)man * 5.9604644775390625e-08f;
    return sign ? -v : v;
  }
  return bits_to_f32(sign | ((exp + 112u) << 23) | (man << 13));
}

/* fp32 -> fp16, round to nearest even, overflow to inf. */
uint16_t or_f32_to_f16(float f) {
  uint32_t x = f32_to_bits(f);
  uint16_t sign = (uint16_t)((x >> 16) & 0x8000u);
  x &= 0x7fffffffu;
  if (x > 0x7f800000u) return sign | 0x7e00u;          /* NaN */
  if (x >= 0x477ff000u) return sign | 0x7c00u;         /* >= 65520 rounds to inf */
  if (x < 0x38800000u) {                               /* below 2^-14: fp16 subnormal */
    float a = bits_to_f32(x) * 16777216.0f;            /* exact scaling by 2^24 */
    return sign | (uint16_t)nearbyintf(a);             /* RNE; 1024 is the min normal */
  }
  x += 0xfffu + ((x >> 13) & 1u);
  x -= 0x38000000u;                                    /* rebias 127 -> 15 */
  return sign | (uint16_t)(x >> 13);
}

static inline float load_elem(const void* p, int dtype, int64_t i) {
  if (dtype == 0) return ((const float*)p)[i];
  if (dtype == 1) return or_f16_to_f32(((const uint16_t*)p)[i]);
  return or_bf16_to_f32(((const uint16_t*)p)[i]);
}

/* Round an fp32 value to the storage dtype and widen it back (torch's
 * reduced-precision result rounding). Identity for fp32. */
static inline float round_to(float v, int dtype) {
  if (dtype == 0) return v;
  if (dtype == 1) return or_f16_to_f32(or_f32_to_f16(v));
  return or_bf16_to_f32(or_f32_to_bf16(v));
}

static inline void store_elem(void* p, int dtype, int64_t i, float v) {
  if (dtype == 0) ((float*)p)[i] = v;
  else if (dtype == 1) ((uint16_t*)p)[i] = or_f32_to_f16(v);
  else ((uint16_t*)p)[i] = or_f32_to_bf16(v);
}

/* torch's max reduction propagates NaN. */
static inline float amax_update(float m, float v) {
  float a = fabsf(v);
  if (isnan(a) || isnan(m)) return NAN;
  return a > m ? a : m;
}

/* ------------------------------------------------------------------------ */
/* Quantizer.quantize_int8 (shadowinfer/utils/quantization.py:120-142)       */
/*   scale = x.abs().max(-1, keepdim) / 127.0      (input dtype T)           */
/*   scale = where(scale == 0, 1, scale)                                     */
/*   q = round(x / scale).clamp(-128, 127).to(int8)                          */
/* rows x D values; q[rows*D] int8; scale[rows] in dtype T.                  */
/* ------------------------------------------------------------------------ */
void or_quant_rows_i8(const void* x, int dtype, int64_t rows, int64_t D,
                      int8_t* q, void* scale) {
  for (int64_t r = 0; r < rows; ++r) {
    float m = 0.0f;
    for (int64_t d = 0; d < D; ++d) m = amax_update(m, load_elem(x, dtype, r * D + d));
    float s = round_to(m / 127.0f, dtype);
    if (s == 0.0f) s = 1.0f;
    store_elem(scale, dtype, r, s);
    for (int64_t d = 0; d < D; ++d) {
      float t = round_to(load_elem(x, dtype, r * D + d) / s, dtype);
      t = nearbyintf(t);
      if (t < -128.0f) t = -128.0f;
      if (t > 127.0f) t = 127.0f;
      q[r * D + d] = (int8_t)t;
    }
  }
}

/* ------------------------------------------------------------------------ */
/* Quantizer.quantize_int4 (shadowinfer/utils/quantization.py:144-178)       */
/*   groups of g along the last dim; scale = amax/7.0 (T), 0 -> 1;           */
/*   q = round(x/scale).clamp(-8, 7) as int8.                                */
/* q[rows*D]; scale[rows*(D/g)] in T.                                        */
/* ------------------------------------------------------------------------ */
void or_quant_rows_i4(const void* x, int dtype, int64_t rows, int64_t D, int64_t g,
                      int8_t* q, void* scale) {
  int64_t G = D / g;
  for (int64_t r = 0; r < rows; ++r) {
    for (int64_t gi = 0; gi < G; ++gi) {
      int64_t base = r * D + gi * g;
      float m = 0.0f;
      for (int64_t d = 0; d < g; ++d) m = amax_update(m, load_elem(x, dtype, base + d));
      float s = round_to(m / 7.0f, dtype);
      if (s == 0.0f) s = 1.0f;
      store_elem(scale, dtype, r * G + gi, s);
      for (int64_t d = 0; d < g; ++d) {
        float t = round_to(load_elem(x, dtype, base + d) / s, dtype);
        t = nearbyintf(t);
        if (t < -8.0f) t = -8.0f;
        if (t > 7.0f) t = 7.0f;
        q[base + d] = (int8_t)t;
      }
    }
  }
}

/* ------------------------------------------------------------------------ */
/* PackedKVCache._pack_int4_rows (shadowinfer/shadowkv/packed_kv_cache.py:   */
/* 367-388): per row of L codes, nibble u = (q + 8) as uint8; a zero nibble  */
/* pads odd L; byte j = u[2j] << 4 | (u[2j+1] & 0xF). Row bytes ceil(L/2).   */
/* ------------------------------------------------------------------------ */
void or_pack_int4_rows(const int8_t* q, int64_t rows, int64_t L, uint8_t* out) {
  int64_t rb = (L + 1) / 2;
  for (int64_t r = 0; r < rows; ++r) {
    for (int64_t j = 0; j < rb; ++j) {
      uint8_t hi = (uint8_t)(q[r * L + 2 * j] + 8);
      uint8_t lo = (2 * j + 1 < L) ? (uint8_t)(q[r * L + 2 * j + 1] + 8) : 0;
      out[r * rb + j] = (uint8_t)((uint8_t)(hi << 4) | (lo & 0x0f));
    }
  }
}

/* Inverse (packed_kv_cache.py:646-650; kernels/__init__.py:405-420):
 * high nibble first, code = nibble - 8. rows of rb bytes -> rows of L codes. */
void or_unpack_int4_rows(const uint8_t* in, int64_t rows, int64_t rb, int64_t L,
                         int8_t* out) {
  for (int64_t r = 0; r < rows; ++r) {
    for (int64_t i = 0; i < L; ++i) {
      uint8_t b = in[r * rb + i / 2];
      uint8_t nib = (i & 1) ? (b & 0x0f) : ((b >> 4) & 0x0f);
      out[r * L + i] = (int8_t)((int)nib - 8);
    }
  }
}

/* Dequantize: Quantizer.dequantize_int8 / dequantize_int4
 * (quantization.py:180-219): float(q) * float(scale), one multiply.
 * rows x D codes, one scale per group of g (g = D for per-row int8). */
void or_dequant_rows(const int8_t* q, const void* scale, int scale_dtype, int64_t rows,
                     int64_t D, int64_t g, float* out) {
  int64_t G = D / g;
  for (int64_t r = 0; r < rows; ++r)
    for (int64_t d = 0; d < D; ++d)
      out[r * D + d] = (float)q[r * D + d] * load_elem(scale, scale_dtype, r * G + d / g);
}

/* Elementwise dtype conversion through fp32 (Tensor.to(dtype)). */
void or_convert(const void* x, int src_dtype, int64_t n, void* out, int dst_dtype) {
  for (int64_t i = 0; i < n; ++i) store_elem(out, dst_dtype, i, load_elem(x, src_dtype, i));
}

/* ------------------------------------------------------------------------ */
/* INT8Linear.from_linear (shadowinfer/ffn_optimizer/int8_linear.py:65-82)   */
/*   w fp32 [N,K]; s = (amax_k|w| / 127).clamp_min(1e-8) (fp32)              */
/*   q = round(w / s).clamp(-127, 127) int8, stored transposed [K,N].        */
/* ------------------------------------------------------------------------ */
void or_weight_quant_i8(const float* w, int64_t N, int64_t K, int8_t* qT, float* s_out) {
  const float eps = 1e-8f;
  for (int64_t n = 0; n < N; ++n) {
    float m = 0.0f;
    for (int64_t k = 0; k < K; ++k) m = amax_update(m, w[n * K + k]);
    float s = m / 127.0f;
    if (s < eps) s = eps;
    s_out[n] = s;
    for (int64_t k = 0; k < K; ++k) {
      float t = nearbyintf(w[n * K + k] / s);
      if (t < -127.0f) t = -127.0f;
      if (t > 127.0f) t = 127.0f;
      qT[k * N + n] = (int8_t)t;
    }
  }
}

/* INT8Linear.forward activation quantization (int8_linear.py:96-98):
 *   xf = x.float(); s = (amax/127).clamp_min(1e-8); q = round(xf/s).clamp(+-127). */
void or_act_quant_i8(const void* x, int dtype, int64_t M, int64_t K, int8_t* q, float* s_out) {
  const float eps = 1e-8f;
  for (int64_t m = 0; m < M; ++m) {
    float a = 0.0f;
    for (int64_t k = 0; k < K; ++k) a = amax_update(a, load_elem(x, dtype, m * K + k));
    float s = a / 127.0f;
    if (s < eps) s = eps;
    s_out[m] = s;
    for (int64_t k = 0; k < K; ++k) {
      float t = nearbyintf(load_elem(x, dtype, m * K + k) / s);
      if (t < -127.0f) t = -127.0f;
      if (t > 127.0f) t = 127.0f;
      q[m * K + k] = (int8_t)t;
    }
  }
}

/* torch._int_mm (int8_linear.py:102): exact integer product, int32 result.
 * a [M,K] int8, b [K,N] int8 -> c [M,N] int32. |a|,|b| <= 127 keeps the sum
 * below 2^31 for K <= 133143, so int32 accumulation is exact. */
void or_gemm_i8(const int8_t* a, const int8_t* b, int64_t M, int64_t N, int64_t K,
                int32_t* c) {
  for (int64_t m = 0; m < M; ++m) {
    for (int64_t n = 0; n < N; ++n) c[m * N + n] = 0;
    for (int64_t k = 0; k < K; ++k) {
      int32_t av = a[m * K + k];
      if (av == 0) continue;
      const int8_t* brow = b + k * N;
      int32_t* crow = c + m * N;
      for (int64_t n = 0; n < N; ++n) crow[n] += av * (int32_t)brow[n];
    }
  }
}

/* Epilogue (int8_linear.py:112-115):
 *   out = acc.float() * (s_x[:,None] * s_w[None,:]);  out = out + bias;  .to(T) */
void or_int8_epilogue(const int32_t* acc, const float* sx, const float* sw, const float* bias,
                      int64_t M, int64_t N, void* out, int out_dtype) {
  for (int64_t m = 0; m < M; ++m)
    for (int64_t n = 0; n < N; ++n) {
      float sc = sx[m] * sw[n];
      float o = (float)acc[m * N + n] * sc;
      if (bias) o = o + bias[n];
      store_elem(out, out_dtype, m * N + n, o);
    }
}

/* Dense bidirectional attention in double precision over fp32 K/V
 * (the unpack -> softmax(q k^T / sqrt(D)) v path of
 * shadowinfer/models/simple_diffusion_llm.py:165-169, no mask).
 * q [BH, Sq, D] (fp32 values), k/v [BH, Skv, D] fp32, out [BH, Sq, D] fp32. */
void or_attention(const float* q, const float* k, const float* v, int64_t BH, int64_t Sq,
                  int64_t Skv, int64_t D, double sm_scale, float* out, double* work) {
  for (int64_t bh = 0; bh < BH; ++bh) {
    const float* qb = q + bh * Sq * D;
    const float* kb = k + bh * Skv * D;
    const float* vb = v + bh * Skv * D;
    for (int64_t i = 0; i < Sq; ++i) {
      double mx = -INFINITY;
      for (int64_t j = 0; j < Skv; ++j) {
        double s = 0.0;
        for (int64_t d = 0; d < D; ++d) s += (double)qb[i * D + d] * (double)kb[j * D + d];
        s *= sm_scale;
        work[j] = s;
        if (s > mx) mx = s;
      }
      double den = 0.0;
      for (int64_t j = 0; j < Skv; ++j) { work[j] = exp(work[j] - mx); den += work[j]; }
      for (int64_t d = 0; d < D; ++d) {
        double acc = 0.0;
        for (int64_t j = 0; j < Skv; ++j) acc += work[j] * (double)vb[j * D + d];
        out[(bh * Sq + i) * D + d] = (float)(acc / den);
      }
    }
  }
}

/* ------------------------------------------------------------------------ */
/* kv_sensitivity (shadowinfer/shadowkv/rd_allocator.py:47-61)               */
/*   k_abs = k.abs().amax(dim=(0, -1)); v_abs likewise      [H, S], dtype T   */
/*   s = (k_abs.square() + v_abs.square()) / 2.0            every op in T     */
/*   out = s.transpose(0, 1)                                [S, H]            */
/* k, v [B, H, S, D] in dtype T; out [S, H] in T.                            */
void or_kv_sensitivity(const void* k, const void* v, int dtype, int64_t B, int64_t H,
                       int64_t S, int64_t D, void* out) {
  for (int64_t t = 0; t < S; ++t) {
    for (int64_t h = 0; h < H; ++h) {
      float ka = 0.0f, va = 0.0f;
      for (int64_t b = 0; b < B; ++b) {
        const int64_t row = ((b * H + h) * S + t) * D;
        for (int64_t d = 0; d < D; ++d) {
          ka = amax_update(ka, load_elem(k, dtype, row + d));
          va = amax_update(va, load_elem(v, dtype, row + d));
        }
      }
      const float sk = round_to(ka * ka, dtype);
      const float sv = round_to(va * va, dtype);
      const float sum = round_to(sk + sv, dtype);
      store_elem(out, dtype, t * H + h, sum / 2.0f);
    }
  }
}
