/*
 * Exhaustive check of the two division-free quotients of the denoising-step
 * row kernels (shadow-infer_amd/csrc/si_step.hip) against correctly rounded
 * division:
 *
 *  1. RMSNorm, bf16 rows: bf16(x * RN(1/rs)) must equal bf16(RN(x / rs)) for
 *     every bf16 rs in [2^-40, 2^40] and every finite bf16 x (the kernel then
 *     multiplies by the weight and rounds again, identically on both paths).
 *  2. INT8Linear activation quantization: with s = max(RN(amax / 127), 1e-8),
 *     r = RN(1/s), q0 = x * r, e = fma(-q0, s, x), q1 = fma(e, r, q0):
 *     a) rint(q1) must equal rint(RN(x / s)) for every finite bf16 amax and
 *        every bf16 x with |x| <= amax (every value a bf16 row can hold);
 *     b) q1 must equal RN(x / s) bit for bit whenever |x / s| >= 2^-10;
 *     c) the same two checks for every finite fp16 amax and every fp16 x with
 *        |x| <= amax (fp16 rows);
 *     d) and on 10^8 random fp32 pairs (fp32 rows), x drawn with |x| <= amax,
 *        amax spanning 2^-40 .. 2^40.
 * Prints the mismatch counts; exit status 0 iff all are 0.
 */
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <string.h>

static float f_of(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }
static uint32_t u_of(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static float bf16_round(float f) {
  uint32_t u = u_of(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return f_of(0x7fc00000u);
  u += 0x7fffu + ((u >> 16) & 1u);
  return f_of(u & 0xffff0000u);
}
/* fp16 bits -> float (exact) */
static float f16_to_f(uint32_t h) {
  const uint32_t sgn = (h & 0x8000u) << 16, ex = (h >> 10) & 0x1fu, man = h & 0x3ffu;
  float v;
  if (ex == 0) v = ldexpf((float)man, -24);
  else v = ldexpf((float)(man | 0x400u), (int)ex - 25);
  return sgn ? -v : v;
}
static uint64_t rng_state = 0x9E3779B97F4A7C15ull;
static uint64_t rnd(uint64_t* s) {  /* splitmix64 */
  uint64_t z = (*s += 0x9E3779B97F4A7C15ull);
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  return z ^ (z >> 31);
}

static int check_quant(float x, float amax, long long* bad_rint, long long* bad_bits) {
  float s = amax / 127.0f;
  s = s < 1e-8f ? 1e-8f : s;
  const float r = 1.0f / s;
  const float q0 = x * r;
  const float e = fmaf(-q0, s, x);
  const float q1 = fmaf(e, r, q0);
  const float qt = x / s;
  if (rintf(q1) != rintf(qt)) ++*bad_rint;
  if (fabsf(qt) >= 0.0009765625f && u_of(q1) != u_of(qt)) ++*bad_bits;
  return 1;
}

int main(void) {
  long long bad_rms = 0, rms_pairs = 0;
  const uint32_t lo = u_of(0x1p-40f) >> 16, hi = u_of(0x1p40f) >> 16;
#pragma omp parallel for schedule(dynamic, 16) reduction(+ : bad_rms, rms_pairs)
  for (uint32_t hr = lo; hr <= hi; ++hr) {
    const float rs = f_of(hr << 16);
    const float rinv = 1.0f / rs;
    for (uint32_t hx = 0; hx < 0x10000u; ++hx) {
      if ((hx & 0x7fffu) >= 0x7f80u) continue; /* inf / NaN */
      const float x = f_of(hx << 16);
      ++rms_pairs;
      if (u_of(bf16_round(x * rinv)) != u_of(bf16_round(x / rs))) ++bad_rms;
    }
  }
  long long bad_rint = 0, bad_bits = 0, q_pairs = 0;
#pragma omp parallel for schedule(dynamic, 64) reduction(+ : bad_rint, bad_bits, q_pairs)
  for (uint32_t ha = 0; ha < 0x7f80u; ++ha) {
    const float amax = f_of(ha << 16);
    for (uint32_t hx = 0; hx < 0x10000u; ++hx) {
      if ((hx & 0x7fffu) >= 0x7f80u) continue;
      const float x = f_of(hx << 16);
      if (fabsf(x) > amax) continue;
      q_pairs += check_quant(x, amax, &bad_rint, &bad_bits);
    }
  }
  long long bad_rint16 = 0, bad_bits16 = 0, h_pairs = 0;
#pragma omp parallel for schedule(dynamic, 64) reduction(+ : bad_rint16, bad_bits16, h_pairs)
  for (uint32_t ha = 0; ha < 0x7c00u; ++ha) {
    const float amax = f16_to_f(ha);
    for (uint32_t hx = 0; hx < 0x10000u; ++hx) {
      if ((hx & 0x7fffu) >= 0x7c00u) continue;
      const float x = f16_to_f(hx);
      if (fabsf(x) > amax) continue;
      h_pairs += check_quant(x, amax, &bad_rint16, &bad_bits16);
    }
  }
  long long bad_rint32 = 0, bad_bits32 = 0;
  for (long long i = 0; i < 100000000LL; ++i) {
    const uint64_t z = rnd(&rng_state);
    const float m = 1.0f + (float)(z & 0xffffffu) * 0x1p-24f;       /* [1, 2) */
    const int ex = (int)((z >> 24) % 81) - 40;                      /* 2^-40 .. 2^40 */
    const float amax = ldexpf(m, ex);
    const float frac = (float)((z >> 32) & 0xffffffu) * 0x1p-24f;   /* [0, 1) */
    const float x = ((z >> 63) ? -1.0f : 1.0f) * amax * frac;
    check_quant(x, amax, &bad_rint32, &bad_bits32);
  }
  printf("rmsnorm_mismatches %lld quant_rint_mismatches %lld quant_bit_mismatches %lld "
         "fp32_rint_mismatches %lld fp32_bit_mismatches %lld rms_pairs %lld quant_pairs %lld "
         "fp16_rint_mismatches %lld fp16_bit_mismatches %lld fp16_pairs %lld\n",
         bad_rms, bad_rint, bad_bits, bad_rint32, bad_bits32, rms_pairs, q_pairs, bad_rint16,
         bad_bits16, h_pairs);
  return (bad_rms || bad_rint || bad_bits || bad_rint32 || bad_bits32 || bad_rint16 ||
          bad_bits16) ? 1 : 0;
}
