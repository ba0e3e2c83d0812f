/*
 * Exhaustive check of the fast bf16 quantization arithmetic used by the pack
 * kernel (shadow-infer_amd/csrc/si_kv.hip) against correctly rounded division:
 *
 *  1. scale: s = bf16(amax / d) for d in {127, 7}, computed as
 *       q0 = amax * R; e = fma(-q0, d, amax); q = fma(e, R, q0),  R = RN(1/d)
 *     must equal bf16(RN(amax / d)) for every finite non-negative bf16 amax.
 *  2. element quotient: for every bf16 s >= 2^-100 (finite) and every bf16 x
 *     with |x| <= 128 s (the domain of a row: |x| <= amax, s ~ amax/127 or
 *     amax/7), with r = RN(1/s):
 *       q0 = x * r; e = fma(-q0, s, x); q1 = fma(e, r, q0)
 *     a) rint(bf16(q1)) must equal rint(bf16(RN(x / s))) (what the kernel
 *        stores), for every pair;
 *     b) q1 must equal RN(x / s) bit for bit whenever |x / s| >= 2^-10 (the
 *        remainder is inexact only for quotients far below 0.5, which round
 *        to 0 either way).
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

int main(void) {
  long long bad_scale = 0, bad_quot = 0, bad_final = 0, checked = 0;
  const float divs[2] = {127.0f, 7.0f};
  for (int k = 0; k < 2; ++k) {
    const float d = divs[k];
    const float R = 1.0f / d;
    for (uint32_t h = 0; h < 0x7f80u; ++h) {
      const float a = f_of(h << 16);
      const float q0 = a * R;
      const float e = fmaf(-q0, d, a);
      const float q = fmaf(e, R, q0);
      if (u_of(bf16_round(q)) != u_of(bf16_round(a / d))) ++bad_scale;
    }
  }
  const float tiny = 7.8886090522101181e-31f; /* 2^-100 */
#pragma omp parallel for schedule(dynamic, 64) reduction(+ : bad_quot, bad_final, checked)
  for (uint32_t hs = 0x0080u; hs < 0x7f80u; ++hs) {
    const float s = f_of(hs << 16);
    if (!(s >= tiny)) continue;
    const float r = 1.0f / s;
    const float lim = 128.0f * s;
    for (uint32_t hx = 0; hx < 0x10000u; ++hx) {
      if ((hx & 0x7fffu) >= 0x7f80u) continue; /* inf / NaN */
      const float x = f_of(hx << 16);
      if (fabsf(x) > lim) continue;
      const float q0 = x * r;
      const float e = fmaf(-q0, s, x);
      const float q1 = fmaf(e, r, q0);
      const float qt = x / s;
      ++checked;
      if (rintf(bf16_round(q1)) != rintf(bf16_round(qt))) ++bad_final;
      if (fabsf(qt) >= 0.0009765625f && u_of(q1) != u_of(qt)) ++bad_quot;
    }
  }
  printf("scale_mismatches %lld final_mismatches %lld quotient_mismatches %lld pairs %lld\n",
         bad_scale, bad_final, bad_quot, checked);
  return (bad_scale || bad_final || bad_quot) ? 1 : 0;
}
