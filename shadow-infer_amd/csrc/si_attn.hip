// Fused dequantize + bidirectional attention over a packed KV cache (gfx950).
//
// Semantics: out = softmax(q k^T * sm_scale) v with no mask, where k/v are the
// values PackedKVCache.unpack() would produce (packed_kv_cache.py:535-577):
// evicted or absent token-heads are zero vectors and still take part in the
// softmax, exactly as in unpack() -> dense attention
// (models/simple_diffusion_llm.py:165-169). The dense K/V never exist: each
// 64-token tile is dequantized straight into LDS as fp16.
//
// Work split: one block of 8 wavefronts (two per SIMD) owns 256 queries of one
// (b, h); each wave owns 32 queries. Per 64-key tile a wave computes S^T = K Q^T
// with v_mfma_f32_32x32x16_f16, so lane l holds scores of query (l % 32) for 16
// of the tile's keys and lane l ^ 32 the other 16: the online-softmax max takes
// one exchange of the wave halves per tile, and each half keeps its own row sum
// until the last tile. O^T = V^T P^T then reuses the score registers
// as the B operand; the k order of an MFMA only has to match between its A and
// B operands, so V^T is read from LDS (V row-major, read with the transposing
// ds_read_b64_tr_b16) in the key order the score accumulator already has
// (keys 8*(i/4) + 4*(l/32) + i%4 of each 16-key chunk).
//
// Precision: fp16 operands (10-bit mantissa) with fp32 accumulation and an
// fp32 online softmax; fp16 entries of the cache are exact in fp16, int8/int4
// values q*s are rounded once to fp16, and P is rounded to fp16 for the P.V
// MFMAs (its row sum adds the same fp16 values).
#include <atomic>
#include <type_traits>

#include "si_kv_common.h"

namespace si {
namespace {

typedef _Float16 v8h __attribute__((ext_vector_type(8)));
typedef _Float16 v4h __attribute__((ext_vector_type(4)));
typedef float v16f __attribute__((ext_vector_type(16)));
typedef int v4i __attribute__((ext_vector_type(4)));

constexpr int BN = 64;   // keys per tile
constexpr int KPAD = 8;  // fp16 padding per K row in LDS

// Capacity of one head's slot list: every precision region starts at a multiple of BN.
inline int64_t list_cap(int64_t Skv) { return (Skv + BN - 1) / BN * BN + 4 * BN; }

// ---------------------------------------------------------------------------
// Per-head slot lists. Softmax attention without a mask does not depend on the
// order of the keys, so the attention kernel visits each head's keys bucket
// by bucket: tiles then hold one precision (branch-free decode, contiguous
// rows). For head h: lists[h * cap + off_p + i] = slot of the i-th entry of
// precision p (token order), off_p = sum over q < p of n_q rounded up to BN;
// counts[h * 8 + p] = n_p, counts[h * 8 + 4] = keys that are evicted or absent
// (they attend as zero vectors: score 0, value 0).
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void attn_lists(const int8_t* __restrict__ code,
                                                  const int32_t* __restrict__ slot, int64_t H,
                                                  int64_t Skv, int64_t cap,
                                                  int32_t* __restrict__ counts,
                                                  int32_t* __restrict__ lists) {
  __shared__ int wtot[5][4];
  const int64_t h = blockIdx.x;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int64_t per = (Skv + 255) / 256;
  const int64_t t0 = min<int64_t>(Skv, tid * per), t1 = min<int64_t>(Skv, t0 + per);
  int n[5] = {0, 0, 0, 0, 0};
  for (int64_t t = t0; t < t1; ++t) {
    const int c = code[t * H + h];
    ++n[(c >= 0 && c <= 3) ? c : 4];
  }
  // Exclusive prefix of each counter over the threads (token order).
  int pre[5];
#pragma unroll
  for (int p = 0; p < 5; ++p) {
    int v = n[p];
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
      const int u = __shfl_up(v, o, 64);
      if (lane >= o) v += u;
    }
    pre[p] = v - n[p];
    if (lane == 63) wtot[p][wave] = v;
  }
  __syncthreads();
  int tot[5];
#pragma unroll
  for (int p = 0; p < 5; ++p) {
    int before = 0, all = 0;
#pragma unroll
    for (int w = 0; w < 4; ++w) {
      before += w < wave ? wtot[p][w] : 0;
      all += wtot[p][w];
    }
    pre[p] += before;
    tot[p] = all;
  }
  int off[4];
  off[0] = 0;
#pragma unroll
  for (int p = 1; p < 4; ++p) off[p] = off[p - 1] + (tot[p - 1] + BN - 1) / BN * BN;
  int32_t* lh = lists + h * cap;
  for (int64_t t = t0; t < t1; ++t) {
    const int64_t e = t * H + h;
    const int c = code[e];
    if (c >= 0 && c <= 3) lh[off[c] + pre[c]++] = slot[e];
  }
  if (tid == 0) {
#pragma unroll
    for (int p = 0; p < 5; ++p) counts[h * 8 + p] = tot[p];
  }
}

template <int QDT>
__device__ __forceinline__ float q_to_f(uint32_t bits) {
  return QDT == SI_DT_BF16 ? bf16_bits_to_f32(bits) : f16_bits_to_f32(bits);
}

__device__ __forceinline__ uint32_t pack_h2(_Float16 lo, _Float16 hi) {
  return (uint32_t)__builtin_bit_cast(uint16_t, lo) | ((uint32_t)__builtin_bit_cast(uint16_t, hi) << 16);
}

// NB bytes at p (aligned to NB) into 32-bit words.
template <int NB>
__device__ __forceinline__ void load_raw(const void* p, uint32_t* r) {
  if constexpr (NB == 16) {
    const uint4 v = *reinterpret_cast<const uint4*>(p);
    r[0] = v.x; r[1] = v.y; r[2] = v.z; r[3] = v.w;
  } else if constexpr (NB == 8) {
    const uint2 v = *reinterpret_cast<const uint2*>(p);
    r[0] = v.x; r[1] = v.y;
  } else if constexpr (NB == 4) {
    r[0] = *reinterpret_cast<const uint32_t*>(p);
  } else if constexpr (NB == 2) {
    r[0] = *reinterpret_cast<const uint16_t*>(p);
  } else {
    r[0] = *reinterpret_cast<const uint8_t*>(p);
  }
}

template <int D>
struct AttnCfg {
  static constexpr int NW = 8;              // waves per block (two per SIMD)
  static constexpr int BMQ = 32 * NW;       // queries per block
  static constexpr int DPT = D / (4 * NW);  // head-dim values per thread in the decode stage
  static constexpr int DGN = 4 * NW;        // dim groups (threads per key group)
  static constexpr int RW = DPT / 2;        // 32-bit words of one key's fp16 values
  // V row pitch (fp16): V is kept row-major like K and read transposed with
  // ds_read_b64_tr_b16 (tile_pv). A pitch of an odd multiple of 16 dwords puts
  // the 8-byte reads of the four rows and two 16-dim halves one transposed
  // read of 32 lanes covers on 64 distinct banks.
  static constexpr int VROW = D == 128 ? 160 : 96;
  // Output staging (finish_rows): a wave's 32 rows pass through LDS in chunks
  // of SRB bytes per row (pitch SRB + 16), so every global store instruction
  // writes whole contiguous row pieces. Waves 0-3 stage in the K tile
  // buffers, waves 4-7 in the V tile buffers (both free after the last tile).
  static constexpr int SRB = D == 128 ? 256 : 128;
  static constexpr int SPITCH = SRB + 16;
  static constexpr int STAGE = 32 * SPITCH;  // bytes per wave
};

typedef short v4s __attribute__((ext_vector_type(4)));
typedef unsigned int v2u __attribute__((ext_vector_type(2)));
typedef __attribute__((address_space(3))) v4s lds_v4s;

typedef _Float16 h2 __attribute__((ext_vector_type(2)));

// Workgroup barrier for LDS traffic only: waits for this wave's LDS accesses
// (lgkmcnt(0)) but, unlike __syncthreads(), not for its global loads, so
// prefetches stay in flight across it. The signal fences keep the compiler
// from moving memory accesses across the barrier.
__device__ __forceinline__ void lds_barrier() {
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
  __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0); vmcnt / expcnt untouched
  __builtin_amdgcn_s_barrier();
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
}

template <int SDT>
__device__ __forceinline__ uint32_t load_scale_bits(const void* p, int64_t i) {
  if (SDT == SI_DT_F32) return reinterpret_cast<const uint32_t*>(p)[i];
  return reinterpret_cast<const uint16_t*>(p)[i];
}
template <int SDT>
__device__ __forceinline__ float scale_from_bits(uint32_t b) {
  if (SDT == SI_DT_F32) return __builtin_bit_cast(float, b);
  return SDT == SI_DT_F16 ? f16_bits_to_f32(b) : bf16_bits_to_f32(b);
}

__device__ __forceinline__ h2 as_h2(uint32_t w) { return __builtin_bit_cast(h2, w); }
__device__ __forceinline__ uint32_t as_u32(h2 v) { return __builtin_bit_cast(uint32_t, v); }

// Bytes b0..b3 of w (two's-complement int8) as fp16 integer pairs
// {b0, b1}, {b2, b3}: 0x64xx is the fp16 1024 + xx, so (w ^ 0x80) bytes give
// 1024 + q + 128 exactly, minus 1152.
__device__ __forceinline__ void i8x4_to_h(uint32_t w, uint32_t& lo, uint32_t& hi) {
  const uint32_t u = w ^ 0x80808080u;
  const h2 bias = {(_Float16)1152.0f, (_Float16)1152.0f};
  lo = as_u32(as_h2(__builtin_amdgcn_perm(0x64646464u, u, 0x04010400u)) - bias);
  hi = as_u32(as_h2(__builtin_amdgcn_perm(0x64646464u, u, 0x04030402u)) - bias);
}

// The low two bytes of w (int4 pairs, high nibble first, offset-binary q + 8)
// as fp16 integer pairs {e0, e1}, {e2, e3}.
__device__ __forceinline__ void i4x4_to_h(uint32_t w, uint32_t& lo, uint32_t& hi) {
  const uint32_t hn = (w >> 4) & 0x0f0fu;  // bytes: e0, e2
  const uint32_t ln = w & 0x0f0fu;         // bytes: e1, e3
  const uint32_t n = __builtin_amdgcn_perm(hn, ln, 0x01050004u);  // e0, e1, e2, e3
  const h2 bias = {(_Float16)1032.0f, (_Float16)1032.0f};
  lo = as_u32(as_h2(__builtin_amdgcn_perm(0x64646464u, n, 0x04010400u)) - bias);
  hi = as_u32(as_h2(__builtin_amdgcn_perm(0x64646464u, n, 0x04030402u)) - bias);
}

// True when fp16(q) * fp16(s) rounds exactly like fp16(float(q) * float(s))
// for every integer |q| <= qmax (128 for int8, 8 for int4): s exact in fp16,
// normal, and |q * s| <= 65504 (q * s is then exact in fp32, and the fp16
// multiply rounds it once). bf16 and fp16 scales always fit fp16's
// significand, so their test is a range test on the raw bits: 2^-14 <= s and
// s <= 65504 / qmax (bf16 0x3880 .. 0x43FF / 0x45FF, fp16 0x0400 .. 0x5FFF /
// 0x6FFF), which also rejects negative scales.
template <int SDT, bool I8>
__device__ __forceinline__ bool h_exact(uint32_t bits, float s) {
  if constexpr (SDT == SI_DT_BF16) return bits - 0x3880u <= (I8 ? 0x43FFu : 0x45FFu) - 0x3880u;
  if constexpr (SDT == SI_DT_F16) return bits - 0x0400u <= (I8 ? 0x5FFFu : 0x6FFFu) - 0x0400u;
  const float qmax = I8 ? 128.0f : 8.0f;
  return s >= 6.103515625e-05f && s * qmax <= 65504.0f && (float)(_Float16)s == s;
}

// The fp16 pair {s, s} of a scale that passed h_exact. A bf16 scale in that
// range is a normal fp16 value with the same 7-bit significand, so its fp16
// bits are its bf16 bits with the exponent rebiased from 127 to 15:
// (bits << 3) - (112 << 10), formed in 32 bits (one shift-add) and splatted
// from the low half. fp16 scales are their bits; fp32 scales are converted
// (exactly).
template <int SDT>
__device__ __forceinline__ h2 scale_h2(uint32_t bits, float s) {
  if constexpr (SDT == SI_DT_F32) {
    const _Float16 h = (_Float16)s;
    return h2{h, h};
  } else {
    const uint32_t w = SDT == SI_DT_BF16 ? (bits << 3) - 0x1C000u : bits;
    const h2 p = __builtin_bit_cast(h2, w);
    return __builtin_shufflevector(p, p, 0, 0);
  }
}

// The two halves of a wave exchanged with v_permlane32_swap_b32 (a VALU op,
// no LDS round trip): lane l receives the value of lane l ^ 32 in one of the
// two results and keeps its own in the other, so max / sum of the pair is the
// pair's max / sum in every lane. The elements are read into scalars before
// the bit cast: clang lowers __builtin_bit_cast of a vector element lvalue
// as a load of element 0.
__device__ __forceinline__ void halves_swap(float v, float& x, float& y) {
  const uint32_t u = __builtin_bit_cast(uint32_t, v);
  const v2u r = __builtin_amdgcn_permlane32_swap(u, u, false, false);
  const uint32_t r0 = r.x, r1 = r.y;
  x = __builtin_bit_cast(float, r0);
  y = __builtin_bit_cast(float, r1);
}
__device__ __forceinline__ float halves_max(float v) {
  float x, y;
  halves_swap(v, x, y);
  return fmaxf(x, y);
}
__device__ __forceinline__ float halves_sum(float v) {
  float x, y;
  halves_swap(v, x, y);
  return x + y;
}

// ---------------------------------------------------------------------------
// The three parts of one 64-key tile for the 32 queries of a wave.
//
// tile_qk: S^T = K Q^T - m on v_mfma_f32_32x32x16_f16. The accumulators start
// at -m_run (0 before the first tile), so the MFMAs return the scores already
// shifted by the running max; lane l holds scores of query l % 32 for 16 keys
// (lane l ^ 32 the other 16). K fragments of k-step ks+1 are read while the
// MFMAs of k-step ks run. Raises the wave priority (the caller lowers it after
// the tile's last P.V MFMA): when both waves of a SIMD have instructions
// ready, the one feeding the matrix core issues first.
template <int D>
__device__ __forceinline__ void tile_qk(const _Float16 (*Ks)[D + KPAD], const v8h* qf, int col,
                                        int grp, const v16f& cinit, v16f (&sacc)[2]) {
  constexpr int KS = D / 16;
  v8h ka[2][2];
  auto load_k = [&](int ks, v8h* a) __attribute__((always_inline)) {
    a[0] = *reinterpret_cast<const v8h*>(&Ks[col][ks * 16 + 8 * grp]);
    a[1] = *reinterpret_cast<const v8h*>(&Ks[32 + col][ks * 16 + 8 * grp]);
  };
  load_k(0, ka[0]);
  __builtin_amdgcn_s_setprio(1);
#pragma unroll
  for (int ks = 0; ks < KS; ++ks) {
    if (ks + 1 < KS) load_k(ks + 1, ka[(ks + 1) & 1]);
    sacc[0] = __builtin_amdgcn_mfma_f32_32x32x16_f16(ka[ks & 1][0], qf[ks], ks == 0 ? cinit : sacc[0], 0, 0, 0);
    sacc[1] = __builtin_amdgcn_mfma_f32_32x32x16_f16(ka[ks & 1][1], qf[ks], ks == 0 ? cinit : sacc[1], 0, 0, 0);
    if (ks + 1 < KS) {
      __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);  // the two reads of ks+1
      __builtin_amdgcn_sched_group_barrier(0x008, 2, 0);  // then the two MFMAs of ks
    }
  }
}

// tile_qk_lo: S^T += Klo Q^T for caches of fp32 inputs, whose K values are
// held as an fp16 pair hi + lo (hi = fp16(x), lo = fp16(x - hi)): the scores
// then carry K to about 22 bits instead of fp16's 11. With fp32 K/V holding
// outlier channels, K's fp16 rounding is most of the output's error (a model
// of the kernel's roundings: relL2 8.8e-4 with it, 4.4e-4 without).
template <int D>
__device__ __forceinline__ void tile_qk_lo(const _Float16 (*Kl)[D + KPAD], const v8h* qf, int col,
                                           int grp, v16f (&sacc)[2]) {
  constexpr int KS = D / 16;
#pragma unroll
  for (int ks = 0; ks < KS; ++ks) {
    const v8h a0 = *reinterpret_cast<const v8h*>(&Kl[col][ks * 16 + 8 * grp]);
    const v8h a1 = *reinterpret_cast<const v8h*>(&Kl[32 + col][ks * 16 + 8 * grp]);
    sacc[0] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a0, qf[ks], sacc[0], 0, 0, 0);
    sacc[1] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a1, qf[ks], sacc[1], 0, 0, 0);
  }
}

// tile_softmax: online softmax of one tile's shifted scores in the log2 domain
// (Q carries sm_scale * log2(e)). Keys at or past nv are masked. The running
// max is raised only when a score exceeds it by more than 8 (a factor 2^8),
// and always at the first tile, so the output rescale is rare. P = 2^(s - m)
// as fp16 pairs (the B operand of the P.V MFMAs); the row sum adds the same
// fp16 values in fp32 (v_dot2_f32_f16 with {1, 1}).
template <int D>
__device__ __forceinline__ void tile_softmax(v16f (&sacc)[2], int nv, int grp, float& m_run,
                                             v16f& cinit, float& l_run, v16f* o,
                                             uint32_t (&pw)[16]) {
  constexpr int DB = D / 32;
  const float c0 = m_run == -INFINITY ? 0.0f : -m_run;
  if (nv < BN) {
#pragma unroll
    for (int kb = 0; kb < 2; ++kb)
#pragma unroll
      for (int r = 0; r < 16; ++r)
        if (kb * 32 + 8 * (r >> 2) + 4 * grp + (r & 3) >= nv) sacc[kb][r] = -INFINITY;
  }
  float tm[4] = {-INFINITY, -INFINITY, -INFINITY, -INFINITY};
#pragma unroll
  for (int kb = 0; kb < 2; ++kb)
#pragma unroll
    for (int r = 0; r < 16; ++r) tm[r & 3] = fmaxf(tm[r & 3], sacc[kb][r]);
  float tmax = fmaxf(fmaxf(tm[0], tm[1]), fmaxf(tm[2], tm[3]));
  tmax = halves_max(tmax);
  const bool raise = m_run == -INFINITY || tmax > 8.0f;
  if (__builtin_amdgcn_ballot_w64(raise) != 0) {
    const float m_new = raise ? tmax - c0 : m_run;
    const float alpha = exp2f(m_run - m_new);
    const float delta = m_new + c0;  // tmax when raised, else 0
    l_run *= alpha;
#pragma unroll
    for (int i = 0; i < DB; ++i)
#pragma unroll
      for (int r = 0; r < 16; ++r) o[i][r] *= alpha;
#pragma unroll
    for (int kb = 0; kb < 2; ++kb)
#pragma unroll
      for (int r = 0; r < 16; ++r) sacc[kb][r] -= delta;
    m_run = m_new;
#pragma unroll
    for (int r = 0; r < 16; ++r) cinit[r] = m_new == -INFINITY ? 0.0f : -m_new;
  }
#pragma unroll
  for (int kb = 0; kb < 2; ++kb)
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      // v_exp_f32: arguments are <= 8 here; results below 2^-126 flush to 0
      const h2 pp = {(_Float16)__builtin_amdgcn_exp2f(sacc[kb][2 * j]),
                     (_Float16)__builtin_amdgcn_exp2f(sacc[kb][2 * j + 1])};
      pw[8 * kb + j] = as_u32(pp);
    }
  float ps[4] = {0.0f, 0.0f, 0.0f, 0.0f};
  const h2 ones = {(_Float16)1.0f, (_Float16)1.0f};
#pragma unroll
  for (int w = 0; w < 16; ++w) ps[w & 3] = __builtin_amdgcn_fdot2(as_h2(pw[w]), ones, ps[w & 3], false);
  l_run += (ps[0] + ps[1]) + (ps[2] + ps[3]);  // this half's keys; halves added at the end
}

// tile_pv: O^T += V^T P^T over four 16-key chunks. The score registers are
// the B operand: the k order of an MFMA only has to agree between A and B, so
// V^T is read in the score accumulator's key order 8*(i/4) + 4*(l/32) + i%4.
// V is row-major in LDS; ds_read_b64_tr_b16 transposes 4 keys x 16 dims per
// 16-lane group: lane r of the group receives M[4j + r/4][r%4] (j = 0..3),
// where lane i of the group addressed the 4 dims M[i][0..3]. Lane i therefore
// addresses key k0 + i/4 at dims base + 4*(i%4), and lane r receives dim
// base + r of keys k0 .. k0+3. V^T fragments stream two (chunk, row block)
// steps ahead of their MFMA.
template <int D>
__device__ __forceinline__ void tile_pv(const _Float16 (*Vs)[AttnCfg<D>::VROW],
                                        const uint32_t (&pw)[16], int col, int grp, v16f* o) {
  constexpr int DB = D / 32;
  const int li = col & 15;       // lane within its 16-lane group
  const int half = col >> 4;     // dims 0..15 or 16..31 of a 32-dim block
  auto load_v = [&](int i) __attribute__((always_inline)) {
    const int c = i / DB, db = i % DB;
    const _Float16* vp = &Vs[c * 16 + 4 * grp + (li >> 2)][db * 32 + 16 * half + 4 * (li & 3)];
    const v4h lo = __builtin_bit_cast(v4h, __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4s*)vp));
    const v4h hi = __builtin_bit_cast(
        v4h, __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4s*)(vp + 8 * AttnCfg<D>::VROW)));
    return v8h{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
  };
  constexpr int NV = 4 * DB;
  v8h va[3];
  va[0] = load_v(0);
  va[1] = load_v(1);
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    if (i + 2 < NV) va[(i + 2) % 3] = load_v(i + 2);
    const int c = i / DB, db = i % DB;
    const int base = 4 * c;  // keys 16c .. 16c+15 of the lane's score order
    const v4i pi = {(int)pw[base], (int)pw[base + 1], (int)pw[base + 2], (int)pw[base + 3]};
    o[db] = __builtin_amdgcn_mfma_f32_32x32x16_f16(va[i % 3], __builtin_bit_cast(v8h, pi), o[db], 0, 0, 0);
  }
}

// Q^T fragments (B operand of S^T = K Q^T) of query m: dims ks*16 + 8*grp + 0..7,
// times sm_scale * log2(e), in fp16 (zeros past the last query).
template <int D, int QDT>
__device__ __forceinline__ void load_q(const uint16_t* __restrict__ Q, int64_t b, int64_t H,
                                       int64_t h, int64_t Sq, int64_t m, int grp,
                                       float scale_log2, v8h* qf) {
  const bool m_ok = m < Sq;
  const uint16_t* qrow = Q + (((b * H + h) * Sq) + (m_ok ? m : 0)) * D;
#pragma unroll
  for (int ks = 0; ks < D / 16; ++ks) {
    uint4 raw = make_uint4(0, 0, 0, 0);
    if (m_ok) raw = *reinterpret_cast<const uint4*>(qrow + ks * 16 + 8 * grp);
    const uint32_t w[4] = {raw.x, raw.y, raw.z, raw.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      qf[ks][2 * i] = (_Float16)(q_to_f<QDT>(w[i] & 0xffffu) * scale_log2);
      qf[ks][2 * i + 1] = (_Float16)(q_to_f<QDT>(w[i] >> 16) * scale_log2);
    }
  }
}

// Evicted / absent keys (score 0, value 0) join the softmax denominator
// (n_ev * 2^(0 - m)); then the wave's rows of O^T, divided by their row sums
// and rounded to out_dtype, go to out. Lane l holds dims db*32 + 8i + 4*grp
// .. +3 of query l % 32, so direct stores would scatter 8- or 16-byte pieces
// over 32 rows; instead the rows are staged in LDS (chunks of SRB bytes per
// row) and read back row-contiguous: each store instruction writes 64 x 16
// contiguous bytes of SRB / 16 lanes per row. Row r of the wave is query
// m0 + r at out + obase0 + r * row_stride (elements); rows at or past Sq are
// not stored.
template <int D>
__device__ __forceinline__ void finish_rows(v16f* o, float m_run, float l_run, int n_ev, int col,
                                            int grp, uint8_t* stage, int64_t m0, int64_t Sq,
                                            int64_t obase0, int64_t row_stride, void* O,
                                            int odt) {
  using C = AttnCfg<D>;
  constexpr int DB = D / 32;
  constexpr int CPR = C::SRB / 16;  // 16-byte chunks per staged row
  const int lane = (grp << 5) | col;
  l_run = halves_sum(l_run);  // each half summed its own keys
  if (n_ev > 0) {
    const float m_fin = fmaxf(m_run, 0.0f);
    const float alpha = exp2f(m_run - m_fin);
    l_run = l_run * alpha + (float)n_ev * exp2f(-m_fin);
#pragma unroll
    for (int i = 0; i < DB; ++i)
#pragma unroll
      for (int r = 0; r < 16; ++r) o[i][r] *= alpha;
  }
  const float inv = 1.0f / l_run;  // rows past Sq may divide by 0: never stored
  // Device-scope (sc1) buffer stores from the wave's first row: the rows are
  // written through as they leave, so less dirty output waits in L2 for the
  // end-of-kernel writeback (S=2048 83.5 -> 82.0 us with 50-launch medians
  // over 12 interleaved rounds; non-temporal stores gain the same but would
  // push the output out of the caches before the next projection reads it).
  // Byte offsets within the wave's 32 rows stay below 2^30: row_stride is D or
  // H * D with H < 65536.
  auto store_chunks = [&](int es, int pd0) __attribute__((always_inline)) {
    __builtin_amdgcn_wave_barrier();
    typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
    const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(
        wave_uniform(reinterpret_cast<uint8_t*>(O) + obase0 * es), (short)0, -1, 0x00020000);
#pragma unroll
    for (int j = 0; j < CPR / 2; ++j) {
      const int idx = j * 64 + lane;
      const int r = idx / CPR, c = idx % CPR;
      const uint4 v = *reinterpret_cast<const uint4*>(stage + r * C::SPITCH + c * 16);
      if (m0 + r < Sq)
        __builtin_amdgcn_raw_buffer_store_b128(u32x4{v.x, v.y, v.z, v.w}, rs,
                                               (int)(((int64_t)r * row_stride + pd0) * es + c * 16), 0, 16);
    }
    __builtin_amdgcn_wave_barrier();
  };
  if (odt == SI_DT_F32) {
    constexpr int DPP = C::SRB / 4;  // dims per pass
#pragma unroll
    for (int pd0 = 0; pd0 < D; pd0 += DPP) {
#pragma unroll
      for (int db = 0; db < DB; ++db) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int d = db * 32 + 8 * i + 4 * grp;
          if (db * 32 >= pd0 && db * 32 < pd0 + DPP)
            *reinterpret_cast<float4*>(stage + col * C::SPITCH + (d - pd0) * 4) =
                make_float4(o[db][4 * i] * inv, o[db][4 * i + 1] * inv, o[db][4 * i + 2] * inv,
                            o[db][4 * i + 3] * inv);
        }
      }
      store_chunks(4, pd0);
    }
  } else {
    static_assert(C::SRB == 2 * D, "one pass of 16-bit rows");
    const bool bf = odt == SI_DT_BF16;
#pragma unroll
    for (int db = 0; db < DB; ++db) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int d = db * 32 + 8 * i + 4 * grp;
        const float r0 = o[db][4 * i + 0] * inv, r1 = o[db][4 * i + 1] * inv;
        const float r2 = o[db][4 * i + 2] * inv, r3 = o[db][4 * i + 3] * inv;
        const uint32_t w0 = (bf ? f32_to_bf16_bits(r0) : f32_to_f16_bits(r0)) |
                            ((bf ? f32_to_bf16_bits(r1) : f32_to_f16_bits(r1)) << 16);
        const uint32_t w1 = (bf ? f32_to_bf16_bits(r2) : f32_to_f16_bits(r2)) |
                            ((bf ? f32_to_bf16_bits(r3) : f32_to_f16_bits(r3)) << 16);
        *reinterpret_cast<uint2*>(stage + col * C::SPITCH + d * 2) = make_uint2(w0, w1);
      }
    }
    store_chunks(2, 0);
  }
}

// ---------------------------------------------------------------------------
// Fused dequantize + bidirectional attention over a packed KV cache.
//
// out = softmax(q k^T * sm_scale) v with no mask, k/v being the values
// PackedKVCache.unpack() produces (packed_kv_cache.py:535-577); evicted or
// absent token-heads are zero vectors that still take part in the softmax,
// as in unpack() -> dense attention (models/simple_diffusion_llm.py:165-169).
// The dense K/V never exist: each 64-key tile is decoded into LDS as fp16.
//
// One block of 8 waves (two per SIMD) owns 256 queries of one (b, h); each
// wave owns 32. Tiles follow the head's slot list (one precision per tile).
// Per tile:
//  * decode (512 threads, 4 keys x D/32 dims each) from registers loaded one
//    tile ahead (slot lists two tiles ahead), K and V row-major;
//  * S^T = K Q^T on v_mfma_f32_32x32x16_f16: lane l holds scores of query
//    l % 32 for 16 keys (lane l ^ 32 the other 16);
//  * int8 and int4 K/V values q * s are rounded once to fp16 in the decode;
//  * online softmax in the log2 domain: the score accumulators start at -m
//    (the running max), so no subtraction follows the MFMAs; the running max
//    is only raised when a score exceeds it by more than 2^8 (probabilities
//    stay <= 256), so the output rescale is rare; the row sum adds the fp16
//    probabilities with v_dot2_f32_f16;
//  * O^T += V^T P^T reuses the score registers as the B operand (the k order
//    of an MFMA only has to agree between A and B: V^T is read, with
//    transposing LDS loads, in the score accumulator's key order
//    8*(i/4) + 4*(l/32) + i%4).
// Evicted/absent keys have score 0; they are added to the softmax
// denominator at the end (n_ev * 2^(0 - m)).
// ---------------------------------------------------------------------------
// Output element strides of b, h and the query index (the head dim is unit stride).
struct OutStrides {
  int64_t b, h, s;
};

// O32: every bucket and scale buffer is below 2^31 bytes and B * D < 2^21, so
// row addresses are 32-bit byte offsets from the (uniform) buffer base, and
// the full-rate 24-bit multiply forms them: slots are below 2^23 (n_max * B *
// D * 4 < 2^31 with B * D >= 64) and every row stride below 2^24.
template <int D, int SDT, int QDT, bool O32>
__global__ __launch_bounds__(512) void attn_packed_fwd(
    const uint16_t* __restrict__ Q, int64_t B, int64_t H, int64_t Sq, int64_t cap,
    const int32_t* __restrict__ counts, const int32_t* __restrict__ lists, Buckets bk, int64_t g,
    float scale_log2, void* __restrict__ O, int odt, OutStrides os) {
  using C = AttnCfg<D>;
  constexpr int KS = D / 16;  // MFMA k-steps over the head dim
  constexpr int DB = D / 32;  // 32-row blocks of O^T
  constexpr int DPT = C::DPT, RW = C::RW > 0 ? C::RW : 1;
  constexpr int VR = C::VROW;
  // Two tile buffers: tile t+1 is decoded into one while tile t is multiplied from the other.
  __shared__ __attribute__((aligned(16))) _Float16 Ks[2][BN][D + KPAD];
  __shared__ __attribute__((aligned(16))) _Float16 Vs[2][BN][VR];
  // fp32 inputs (fp32 scales): the low fp16 parts of K (tile_qk_lo)
  constexpr bool KLO = SDT == SI_DT_F32;
  __shared__ __attribute__((aligned(16))) _Float16 Kls[KLO ? 2 : 1][KLO ? BN : 1][D + KPAD];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int col = lane & 31;  // query column within the wave
  const int grp = lane >> 5;  // 0/1: k-half of MFMA operands, row quad of results
  // The query blocks of one (b, h) on one XCD, one after another in dispatch
  // order, so the head's packed K/V is fetched into that XCD's L2 once.
  const int nq = (int)gridDim.x;
  const int w_id = xcd_order((int)(blockIdx.x + nq * (blockIdx.y + gridDim.y * blockIdx.z)),
                             nq * (int)(gridDim.y * gridDim.z));
  const int64_t h = (w_id / nq) % (int)gridDim.y;
  const int64_t b = w_id / (nq * (int)gridDim.y);
  const int64_t m = (int64_t)(w_id % nq) * C::BMQ + wave * 32 + col;

  // Q^T fragments (B operand of S^T = K Q^T): query m, dims ks*16 + 8*grp + 0..7.
  v8h qf[KS];
  load_q<D, QDT>(Q, b, H, h, Sq, m, grp, scale_log2, qf);

  // Slots of tile 0, loaded beside the head's counts: the first non-empty
  // precision phase always starts at tile 0, so its first slot load does not
  // wait for the counts (the list holds at least 4 tiles, so the read is in
  // bounds even when every key of the head is evicted).
  const int32_t* lh = lists + h * cap;
  const int kg = tid / C::DGN;
  const int4 sl0 = *reinterpret_cast<const int4*>(lh + 4 * kg);

  // Tile schedule: the head's list regions in order fp32, fp16, int8, int4.
  const int32_t* cnt = counts + h * 8;
  int np[4], tstart[5];
  tstart[0] = 0;
#pragma unroll
  for (int p = 0; p < 4; ++p) {
    np[p] = cnt[p];
    tstart[p + 1] = tstart[p] + (np[p] + BN - 1) / BN;
  }
  const int n_ev = cnt[4];
  auto tile_valid = [&](int tt, int p) __attribute__((always_inline)) { return min(BN, np[p] - (tt - tstart[p]) * BN); };

  // Decode-stage coordinates: keys 4*kg .. 4*kg+3 of the tile, dims d0 .. d0+DPT-1.
  const int dg = tid % C::DGN;
  const int d0 = dg * DPT;
  const int ngrp = (int)(D / g);       // int4 groups per row
  const int my_grp = d0 / (int)g;      // this thread's group (DPT values never straddle one)

  int4 sl = sl0;                    // slots of the next tile to fetch
  int4 sl_data = sl;                 // slots of the tile held in rk / rv
  uint32_t rk[4][RW], rv[4][RW];
  uint32_t skb[4], svb[4];  // raw scale bits, converted at decode time

  // Tiles are processed in precision phases (the list regions): every load
  // and decode below is specialised for the phase's precision P, so no branch
  // inside a phase's tile loop merges registers that still have loads in
  // flight (the compiler would then wait for them in every iteration). Within
  // the loop prefetches are unconditional: indices past the phase's last tile
  // are clamped to it (a harmless re-read). Only the peeled last tile of a
  // phase branches, to load the next phase's first tile.
  int t_last = 0;  // last tile of the current phase
  auto fetch_slots = [&](int tt) __attribute__((always_inline)) {
    tt = min(tt, t_last);
    sl = *reinterpret_cast<const int4*>(lh + (int64_t)tt * BN + 4 * kg);
  };
  // Byte offset of a slot's row = slot * stride + this thread's constant part.
  constexpr uint32_t SS = SDT == SI_DT_F32 ? 4 : 2;  // scale bytes
  const uint32_t st16 = (uint32_t)(2 * B * D), c16 = (uint32_t)(2 * (b * D + d0));
  const uint32_t st8 = (uint32_t)(B * D), c8 = (uint32_t)(b * D + d0);
  const uint32_t st8s = (uint32_t)(B * SS), c8s = (uint32_t)(b * SS);
  const uint32_t st4 = (uint32_t)(B * D / 2), c4 = (uint32_t)((b * D + d0) / 2);
  const uint32_t st4s = (uint32_t)(B * ngrp * SS), c4s = (uint32_t)((b * ngrp + my_grp) * SS);
  auto at = [&](int j, uint32_t off) __attribute__((always_inline)) {
    return reinterpret_cast<const char*>(bk.p[j]) + off;
  };
  // Raw loads of the tile's rows into registers (fp32 tiles are read at decode time).
  auto fetch_data = [&](auto PC, int tt) __attribute__((always_inline)) {
    constexpr int P = decltype(PC)::value;
    tt = min(tt, t_last);
    const int nv = __builtin_amdgcn_readfirstlane(tile_valid(tt, P));
    sl_data = sl;
    int sl4[4] = {sl.x, sl.y, sl.z, sl.w};
    if constexpr (P == SI_PREC_FP32) return;  // read at decode time
    // Keys past the tile's valid count (only in a phase's last tile: nv is
    // wave-uniform) read row 0 of the same (non-empty) bucket: their list
    // entries are not written, and their scores are masked to -inf.
    if (nv < BN) {
#pragma unroll
      for (int i = 0; i < 4; ++i) sl4[i] = 4 * kg + i < nv ? sl4[i] : 0;
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int sli = sl4[i];
      if constexpr (O32) {
        const uint32_t us = (uint32_t)sli;
        __builtin_assume(us < (1u << 23));
        if constexpr (P == SI_PREC_FP16) {
          load_raw<2 * DPT>(at(4, __umul24(us, st16) + c16), rk[i]);
          load_raw<2 * DPT>(at(5, __umul24(us, st16) + c16), rv[i]);
        } else if constexpr (P == SI_PREC_INT8) {
          load_raw<DPT>(at(8, __umul24(us, st8) + c8), rk[i]);
          load_raw<DPT>(at(9, __umul24(us, st8) + c8), rv[i]);
          load_raw<SS>(at(10, __umul24(us, st8s) + c8s), &skb[i]);
          load_raw<SS>(at(11, __umul24(us, st8s) + c8s), &svb[i]);
        } else if constexpr (P == SI_PREC_INT4) {
          load_raw<DPT / 2>(at(12, __umul24(us, st4) + c4), rk[i]);
          load_raw<DPT / 2>(at(13, __umul24(us, st4) + c4), rv[i]);
          load_raw<SS>(at(14, __umul24(us, st4s) + c4s), &skb[i]);
          load_raw<SS>(at(15, __umul24(us, st4s) + c4s), &svb[i]);
        }
        continue;
      }
      const int64_t row = (int64_t)sli * B + b;
      if constexpr (P == SI_PREC_FP16) {
        load_raw<2 * DPT>(reinterpret_cast<const uint16_t*>(bk.p[4]) + row * D + d0, rk[i]);
        load_raw<2 * DPT>(reinterpret_cast<const uint16_t*>(bk.p[5]) + row * D + d0, rv[i]);
      } else if constexpr (P == SI_PREC_INT8) {
        load_raw<DPT>(reinterpret_cast<const int8_t*>(bk.p[8]) + row * D + d0, rk[i]);
        load_raw<DPT>(reinterpret_cast<const int8_t*>(bk.p[9]) + row * D + d0, rv[i]);
        skb[i] = load_scale_bits<SDT>(bk.p[10], row);
        svb[i] = load_scale_bits<SDT>(bk.p[11], row);
      } else if constexpr (P == SI_PREC_INT4) {
        const int64_t rb = B * D / 2;  // bytes of one int4 entry row
        const int64_t off = sli * rb + (b * D + d0) / 2;
        load_raw<DPT / 2>(reinterpret_cast<const uint8_t*>(bk.p[12]) + off, rk[i]);
        load_raw<DPT / 2>(reinterpret_cast<const uint8_t*>(bk.p[13]) + off, rv[i]);
        const int64_t si = row * ngrp + my_grp;
        skb[i] = load_scale_bits<SDT>(bk.p[14], si);
        svb[i] = load_scale_bits<SDT>(bk.p[15], si);
      }
    }
  };

  v16f o[DB];
#pragma unroll
  for (int i = 0; i < DB; ++i)
#pragma unroll
    for (int r = 0; r < 16; ++r) o[i][r] = 0.0f;
  float m_run = -INFINITY;
  v16f cinit = {};  // the QK accumulators' start value: -m_run (0 before the first raise)
  float l_run = 0.0f;

  // Decode tile tt (its rows are in rk / rv) into LDS buffer buf.
  auto decode_tile = [&](auto PC, int tt, int buf) __attribute__((always_inline)) {
    constexpr int P = decltype(PC)::value;
    const int nv = __builtin_amdgcn_readfirstlane(tile_valid(tt, P));
    {
      // The prefetched registers are first read here: nothing computed from
      // them may move earlier (that would wait for the loads in flight).
#pragma unroll
      for (int i = 0; i < 4; ++i) {
#pragma unroll
        for (int x = 0; x < RW; ++x) asm volatile("" : "+v"(rk[i][x]), "+v"(rv[i][x]));
        asm volatile("" : "+v"(skb[i]), "+v"(svb[i]));
      }
      float sk[4], sv[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        sk[i] = scale_from_bits<SDT>(skb[i]);
        sv[i] = scale_from_bits<SDT>(svb[i]);
      }
      // Per key i: fp16 pair words of K (kw) and V (vw), dims (2x, 2x+1);
      // with KLO also the low parts of K (kl).
      uint32_t kw[4][RW], vw[4][RW], kl[4][RW];
      if constexpr (P == SI_PREC_FP16) {
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
          for (int x = 0; x < RW; ++x) {
            kw[i][x] = rk[i][x];
            vw[i][x] = rv[i][x];
          }
      } else if constexpr (P == SI_PREC_INT8 || P == SI_PREC_INT4) {
        // Integer codes as exact fp16 pairs.
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          if constexpr (P == SI_PREC_INT8) {
            uint32_t unused;
            if constexpr (DPT >= 4) {
#pragma unroll
              for (int x = 0; x < DPT / 4; ++x) {
                i8x4_to_h(rk[i][x], kw[i][2 * x], kw[i][2 * x + 1]);
                i8x4_to_h(rv[i][x], vw[i][2 * x], vw[i][2 * x + 1]);
              }
            } else {
              i8x4_to_h(rk[i][0], kw[i][0], unused);
              i8x4_to_h(rv[i][0], vw[i][0], unused);
            }
          } else if constexpr (DPT >= 4) {
#pragma unroll
            for (int x = 0; x < DPT / 4; ++x) {
              i4x4_to_h(rk[i][0] >> (16 * x), kw[i][2 * x], kw[i][2 * x + 1]);
              i4x4_to_h(rv[i][0] >> (16 * x), vw[i][2 * x], vw[i][2 * x + 1]);
            }
          } else {
            const uint32_t kb = rk[i][0] & 0xffu, vb = rv[i][0] & 0xffu;
            kw[i][0] = pack_h2((_Float16)(float)((int)(kb >> 4) - 8), (_Float16)(float)((int)(kb & 0xfu) - 8));
            vw[i][0] = pack_h2((_Float16)(float)((int)(vb >> 4) - 8), (_Float16)(float)((int)(vb & 0xfu) - 8));
          }
        }
        // K and V values float(q) * float(s) rounded once to fp16: a packed fp16
        // multiply when that rounds the same way for the whole wave (always, for
        // scales of ordinary magnitude), else through fp32.
        int fast = 1;  // int, not bool: '&' keeps the eight tests branch-free
#pragma unroll
        for (int i = 0; i < 4; ++i)
          fast &= (int)h_exact<SDT, P == SI_PREC_INT8>(skb[i], sk[i]) &
                  (int)h_exact<SDT, P == SI_PREC_INT8>(svb[i], sv[i]);
        if constexpr (KLO) {
          // K as the fp32 product float(q) * s (the unpack's value) split into
          // fp16 hi + lo; V rounded once to fp16 as below.
#pragma unroll
          for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int x = 0; x < RW; ++x) {
              const h2 a = as_h2(kw[i][x]);
              const float p0 = (float)a[0] * sk[i], p1 = (float)a[1] * sk[i];
              const _Float16 h0 = (_Float16)p0, h1 = (_Float16)p1;
              kw[i][x] = pack_h2(h0, h1);
              kl[i][x] = pack_h2((_Float16)(p0 - (float)h0), (_Float16)(p1 - (float)h1));
            }
        }
        if (__builtin_amdgcn_ballot_w64(fast == 0) == 0) {
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const h2 k2 = scale_h2<SDT>(skb[i], sk[i]), v2 = scale_h2<SDT>(svb[i], sv[i]);
#pragma unroll
            for (int x = 0; x < RW; ++x) {
              if constexpr (!KLO) kw[i][x] = as_u32(as_h2(kw[i][x]) * k2);
              vw[i][x] = as_u32(as_h2(vw[i][x]) * v2);
            }
          }
        } else {
#pragma unroll
          for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int x = 0; x < RW; ++x) {
              const h2 a = as_h2(kw[i][x]), c = as_h2(vw[i][x]);
              if constexpr (!KLO)
                kw[i][x] = pack_h2((_Float16)((float)a[0] * sk[i]), (_Float16)((float)a[1] * sk[i]));
              vw[i][x] = pack_h2((_Float16)((float)c[0] * sv[i]), (_Float16)((float)c[1] * sv[i]));
            }
        }
      } else {  // fp32 bucket rows, read here
        const int sl4[4] = {sl_data.x, sl_data.y, sl_data.z, sl_data.w};
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          float kx[DPT], vx[DPT];
#pragma unroll
          for (int e = 0; e < DPT; ++e) kx[e] = vx[e] = 0.0f;
          if (4 * kg + i < nv) {
            const int64_t row = (int64_t)sl4[i] * B + b;
            const float* kp = reinterpret_cast<const float*>(bk.p[0]) + row * D + d0;
            const float* vp = reinterpret_cast<const float*>(bk.p[1]) + row * D + d0;
#pragma unroll
            for (int e = 0; e < DPT; ++e) {
              kx[e] = kp[e];
              vx[e] = vp[e];
            }
          }
#pragma unroll
          for (int x = 0; x < RW; ++x) {
            const _Float16 h0 = (_Float16)kx[2 * x], h1 = (_Float16)kx[2 * x + 1];
            kw[i][x] = pack_h2(h0, h1);
            if constexpr (KLO)
              kl[i][x] = pack_h2((_Float16)(kx[2 * x] - (float)h0), (_Float16)(kx[2 * x + 1] - (float)h1));
            vw[i][x] = pack_h2((_Float16)vx[2 * x], (_Float16)vx[2 * x + 1]);
          }
        }
      }
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        if constexpr (DPT == 8) {
          *reinterpret_cast<uint4*>(&Ks[buf][4 * kg + i][d0]) =
              make_uint4(kw[i][0], kw[i][1], kw[i][2], kw[i][3]);
        } else if constexpr (DPT == 4) {
          *reinterpret_cast<uint2*>(&Ks[buf][4 * kg + i][d0]) = make_uint2(kw[i][0], kw[i][1]);
        } else {
          *reinterpret_cast<uint32_t*>(&Ks[buf][4 * kg + i][d0]) = kw[i][0];
        }
      }
      if constexpr (KLO && P != SI_PREC_FP16) {  // fp16 rows are exact in fp16: no low part
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          if constexpr (DPT == 8) {
            *reinterpret_cast<uint4*>(&Kls[buf][4 * kg + i][d0]) =
                make_uint4(kl[i][0], kl[i][1], kl[i][2], kl[i][3]);
          } else if constexpr (DPT == 4) {
            *reinterpret_cast<uint2*>(&Kls[buf][4 * kg + i][d0]) = make_uint2(kl[i][0], kl[i][1]);
          } else {
            *reinterpret_cast<uint32_t*>(&Kls[buf][4 * kg + i][d0]) = kl[i][0];
          }
        }
      }
      // V rows like K rows (tile_pv reads them transposed)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        if constexpr (DPT == 8) {
          *reinterpret_cast<uint4*>(&Vs[buf][4 * kg + i][d0]) =
              make_uint4(vw[i][0], vw[i][1], vw[i][2], vw[i][3]);
        } else if constexpr (DPT == 4) {
          *reinterpret_cast<uint2*>(&Vs[buf][4 * kg + i][d0]) = make_uint2(vw[i][0], vw[i][1]);
        } else {
          *reinterpret_cast<uint32_t*>(&Vs[buf][4 * kg + i][d0]) = vw[i][0];
        }
      }
    }
  };

  // S^T = K Q^T, online softmax and O^T += V^T P^T for the tile in buffer buf.
  auto compute_tile = [&](auto PC, int nv, int buf) __attribute__((always_inline)) {
    constexpr int P = decltype(PC)::value;
    v16f sacc[2];
    uint32_t pw[16];
    tile_qk<D>(Ks[buf], qf, col, grp, cinit, sacc);
    if constexpr (KLO && P != SI_PREC_FP16) tile_qk_lo<D>(Kls[buf], qf, col, grp, sacc);
    tile_softmax<D>(sacc, nv, grp, m_run, cinit, l_run, o, pw);
    tile_pv<D>(Vs[buf], pw, col, grp, o);
    __builtin_amdgcn_s_setprio(0);
  };

  int buf = 0;
  // Slots of the first tile of the next non-empty phase: loaded when a phase
  // starts (clamped to the head's last tile, so always in bounds), they have
  // landed by the time the phase's tiles are done, and the next phase's first
  // data load waits for nothing else (tile 0: loaded at the kernel start).
  int4 sl_nx = sl0;
  // Slots of the second tile of the next phase, clamped to that phase's last
  // tile. For the first non-empty phase (it starts at tile 0 and ends before
  // the first tstart[q] > 0): tile min(1, its last tile), loaded here.
  int4 sl_n2;
  {
    const int fl = tstart[1] > 0 ? tstart[1] - 1
                 : tstart[2] > 0 ? tstart[2] - 1
                 : tstart[3] > 0 ? tstart[3] - 1
                                 : max(tstart[4] - 1, 0);
    sl_n2 = *reinterpret_cast<const int4*>(lh + (int64_t)min(1, fl) * BN + 4 * kg);
  }
  // During a phase's last tile, the first tile of the next non-empty phase
  // (precision Q > P, the phase starting at tile tstart[P + 1]) is loaded into
  // rk / rv with Q's loads, so the next phase starts with its decode. The
  // choice of Q is a wave-uniform branch; its loads are first read by that
  // decode, which needs them anyway.
  bool pref = false;  // rk / rv hold the first tile of the phase about to run
  auto fetch_first = [&](auto QC) __attribute__((always_inline)) {
    constexpr int Q = decltype(QC)::value;
    t_last = tstart[Q + 1] - 1;
    sl = sl_nx;
    fetch_data(QC, tstart[Q]);
    pref = true;
  };
  auto prefetch_next = [&](auto PC) __attribute__((always_inline)) {
    constexpr int P = decltype(PC)::value;
    if constexpr (P + 1 <= SI_PREC_INT4) {
      if (tstart[P + 1] < tstart[P + 2]) {
        fetch_first(std::integral_constant<int, P + 1>{});
      } else if constexpr (P + 2 <= SI_PREC_INT4) {
        if (tstart[P + 2] < tstart[P + 3]) {
          fetch_first(std::integral_constant<int, P + 2>{});
        } else if constexpr (P + 3 <= SI_PREC_INT4) {
          if (tstart[P + 3] < tstart[P + 4]) fetch_first(std::integral_constant<int, P + 3>{});
        }
      }
    }
  };
  auto run_phase = [&](auto PC) __attribute__((always_inline)) {
    constexpr int P = decltype(PC)::value;
    const int t0 = tstart[P], t1 = tstart[P + 1];
    if (t0 >= t1) return;
    t_last = t1 - 1;
    sl = sl_nx;
    if (!pref) fetch_data(PC, t0);  // else loaded during the last phase's last tile
    pref = false;
    sl_nx = *reinterpret_cast<const int4*>(lh + (int64_t)min(t1, tstart[4] - 1) * BN + 4 * kg);
    sl = sl_n2;  // slots of tile min(t0 + 1, t_last), loaded before this phase
    decode_tile(PC, t0, buf);
    fetch_data(PC, t0 + 1);
    fetch_slots(t0 + 2);
    lds_barrier();
    // All tiles but the last; the loop body has no branch over loads in flight.
    for (int tt = t0; tt < t1 - 1; ++tt) {
      compute_tile(PC, __builtin_amdgcn_readfirstlane(tile_valid(tt, P)), buf);
      // Decode the next tile into the other buffer, then prefetch.
      decode_tile(PC, min(tt + 1, t_last), buf ^ 1);
      fetch_data(PC, tt + 2);
      fetch_slots(tt + 3);
      // Buffer buf ^ 1 is complete and every wave is done with buffer buf.
      lds_barrier();
      buf ^= 1;
    }
    // The last tile; meanwhile the next phase's first tile is loaded, and the
    // slots of its second tile (clamped to that phase's last tile, nl).
    {
      // the next non-empty phase ends at the first tstart[q] > t1, q > P + 1
      int nl = t1;
      if constexpr (P + 2 <= 4) {
        if (tstart[P + 2] > t1) {
          nl = tstart[P + 2] - 1;
        } else if constexpr (P + 3 <= 4) {
          if (tstart[P + 3] > t1) {
            nl = tstart[P + 3] - 1;
          } else if constexpr (P + 4 <= 4) {
            if (tstart[P + 4] > t1) nl = tstart[P + 4] - 1;
          }
        }
      }
      const int i2 = min(min(t1 + 1, nl), max(tstart[4] - 1, 0));
      sl_n2 = *reinterpret_cast<const int4*>(lh + (int64_t)i2 * BN + 4 * kg);
    }
    compute_tile(PC, __builtin_amdgcn_readfirstlane(tile_valid(t_last, P)), buf);
    prefetch_next(PC);
    lds_barrier();  // also frees the tile buffers for the output staging
    buf ^= 1;
  };
  run_phase(std::integral_constant<int, SI_PREC_FP32>{});
  run_phase(std::integral_constant<int, SI_PREC_FP16>{});
  run_phase(std::integral_constant<int, SI_PREC_INT8>{});
  run_phase(std::integral_constant<int, SI_PREC_INT4>{});

  // Every wave is past the last tile's barrier: the tile buffers are free.
  static_assert(4 * C::STAGE <= (int)sizeof(Ks) && 4 * C::STAGE <= (int)sizeof(Vs),
                "output staging fits the tile buffers");
  uint8_t* stage = wave < 4 ? reinterpret_cast<uint8_t*>(&Ks[0][0][0]) + wave * C::STAGE
                            : reinterpret_cast<uint8_t*>(&Vs[0][0][0]) + (wave - 4) * C::STAGE;
  const int64_t m0 = m - col;
  finish_rows<D>(o, m_run, l_run, n_ev, col, grp, stage, m0, Sq, b * os.b + h * os.h + m0 * os.s,
                 os.s, O, odt);
}

template <int D, int QDT, bool O32>
void launch_attn_o(int sdt, dim3 grid, hipStream_t st, const uint16_t* q, int64_t B, int64_t H,
                   int64_t Sq, int64_t cap, const int32_t* counts, const int32_t* lists,
                   const Buckets& bk, int64_t g, float scale_log2, void* out, int odt,
                   const OutStrides& os) {
  constexpr int NT = 64 * AttnCfg<D>::NW;
  switch (sdt) {
    case SI_DT_F32:
      attn_packed_fwd<D, SI_DT_F32, QDT, O32><<<grid, NT, 0, st>>>(q, B, H, Sq, cap, counts, lists,
                                                                   bk, g, scale_log2, out, odt, os);
      break;
    case SI_DT_F16:
      attn_packed_fwd<D, SI_DT_F16, QDT, O32><<<grid, NT, 0, st>>>(q, B, H, Sq, cap, counts, lists,
                                                                   bk, g, scale_log2, out, odt, os);
      break;
    default:
      attn_packed_fwd<D, SI_DT_BF16, QDT, O32><<<grid, NT, 0, st>>>(q, B, H, Sq, cap, counts, lists,
                                                                    bk, g, scale_log2, out, odt, os);
  }
}

// Set by si_tune_attn_offset64 (tests): 64-bit addressing at every size.
std::atomic<int> g_force_offset64{0};

// A bucket holds at most n_max = S_kv * H entries; fp32 rows (B * D * 4 bytes)
// bound the byte offsets of every bucket and scale buffer.
template <int D, int QDT>
void launch_attn(int sdt, dim3 grid, hipStream_t st, const uint16_t* q, int64_t B, int64_t H,
                 int64_t Sq, int64_t cap, const int32_t* counts, const int32_t* lists,
                 const Buckets& bk, int64_t g, float scale_log2, void* out, int odt,
                 const OutStrides& os, int64_t n_max) {
  // si_tune_attn_offset64 selects the 64-bit addressing at every size, so tests can
  // compare the two paths on small caches.
  if (n_max * B * D * 4 < ((int64_t)1 << 31) && B * D < ((int64_t)1 << 21) &&
      !g_force_offset64.load(std::memory_order_relaxed))
    launch_attn_o<D, QDT, true>(sdt, grid, st, q, B, H, Sq, cap, counts, lists, bk, g, scale_log2,
                                out, odt, os);
  else
    launch_attn_o<D, QDT, false>(sdt, grid, st, q, B, H, Sq, cap, counts, lists, bk, g, scale_log2,
                                 out, odt, os);
}

}  // namespace
}  // namespace si

using namespace si;

extern "C" void si_tune_attn_offset64(int on) {
  g_force_offset64.store(on != 0 ? 1 : 0, std::memory_order_relaxed);
}

extern "C" size_t si_attn_workspace_bytes(int64_t H, int64_t S_kv) {
  if (H <= 0 || S_kv <= 0) return 0;
  return (size_t)H * 8 * sizeof(int32_t) + (size_t)H * (size_t)list_cap(S_kv) * sizeof(int32_t);
}

namespace {
int run_attn(const void* q, int q_dtype, int64_t B, int64_t H, int64_t S_q, int64_t D,
             const int8_t* code, const int32_t* slot, const void* const* buckets, int scale_dtype,
             int64_t S_kv, int64_t group, float sm_scale, void* out, int out_dtype,
             const OutStrides& os, void* workspace, size_t workspace_bytes, bool build_lists,
             hipStream_t st) {
  SI_CHECK_ARG(q_dtype == SI_DT_BF16 || q_dtype == SI_DT_F16,
               "si_attn_packed_fwd: q dtype must be bf16 or fp16 (got %d)", q_dtype);
  SI_CHECK_ARG(dtype_ok(scale_dtype), "si_attn_packed_fwd: unsupported scale dtype %d",
               scale_dtype);
  SI_CHECK_ARG(dtype_ok(out_dtype), "si_attn_packed_fwd: unsupported out dtype %d", out_dtype);
  SI_CHECK_ARG(D == 64 || D == 128, "si_attn_packed_fwd: head_dim must be 64 or 128 (got %lld)",
               (long long)D);
  SI_CHECK_ARG(B >= 0 && H >= 0 && S_q >= 0 && S_kv > 0, "si_attn_packed_fwd: bad shape");
  SI_CHECK_ARG(group > 0 && D % group == 0 && group % (D / 32) == 0,
               "si_attn_packed_fwd: int4 group must divide head_dim and be a multiple of %lld",
               (long long)(D / 32));
  SI_CHECK_ARG(H < 65536 && B < 65536 && S_kv < ((int64_t)1 << 30),
               "si_attn_packed_fwd: H and B must be < 65536, S_kv < 2^30");
  if (B * H * S_q == 0) return SI_OK;
  SI_CHECK_ARG(q && buckets && out && (!build_lists || (code && slot)),
               "si_attn_packed_fwd: NULL argument");
  const size_t need = si_attn_workspace_bytes(H, S_kv);
  SI_CHECK_ARG(workspace != nullptr && workspace_bytes >= need &&
                   (reinterpret_cast<uintptr_t>(workspace) & 15) == 0,
               "si_attn_packed_fwd: workspace too small or misaligned (%zu < %zu bytes)",
               workspace_bytes, need);
  SI_CHECK_ARG((reinterpret_cast<uintptr_t>(q) & 15) == 0 &&
                   (reinterpret_cast<uintptr_t>(out) & 15) == 0,
               "si_attn_packed_fwd: q and out must be 16-byte aligned");
  const Buckets bk = to_buckets(buckets);
  const int64_t cap = list_cap(S_kv);
  int32_t* counts = reinterpret_cast<int32_t*>(workspace);
  int32_t* lists = counts + H * 8;
  if (build_lists) {
    attn_lists<<<(unsigned)H, 256, 0, st>>>(code, slot, H, S_kv, cap, counts, lists);
    if (int rc = check_launch("si_attn_packed_fwd")) return rc;
  }
  const int64_t bmq = D == 128 ? AttnCfg<128>::BMQ : AttnCfg<64>::BMQ;
  SI_CHECK_ARG(ceil_div(S_q, bmq) * H * B < ((int64_t)1 << 31),
               "si_attn_packed_fwd: %lld query blocks (at most 2^31 - 1)",
               (long long)(ceil_div(S_q, bmq) * H * B));
  const dim3 grid((unsigned)ceil_div(S_q, bmq), (unsigned)H, (unsigned)B);
  const float scale_log2 = sm_scale * 1.4426950408889634f;
  const uint16_t* qp = reinterpret_cast<const uint16_t*>(q);
  if (D == 128) {
    if (q_dtype == SI_DT_BF16)
      launch_attn<128, SI_DT_BF16>(scale_dtype, grid, st, qp, B, H, S_q, cap, counts, lists, bk,
                                   group, scale_log2, out, out_dtype, os, S_kv * H);
    else
      launch_attn<128, SI_DT_F16>(scale_dtype, grid, st, qp, B, H, S_q, cap, counts, lists, bk,
                                  group, scale_log2, out, out_dtype, os, S_kv * H);
  } else {
    if (q_dtype == SI_DT_BF16)
      launch_attn<64, SI_DT_BF16>(scale_dtype, grid, st, qp, B, H, S_q, cap, counts, lists, bk,
                                  group, scale_log2, out, out_dtype, os, S_kv * H);
    else
      launch_attn<64, SI_DT_F16>(scale_dtype, grid, st, qp, B, H, S_q, cap, counts, lists, bk,
                                 group, scale_log2, out, out_dtype, os, S_kv * H);
  }
  return check_launch("si_attn_packed_fwd");
}
}  // namespace

extern "C" int si_attn_packed_fwd(const void* q, int q_dtype, int64_t B, int64_t H, int64_t S_q,
                                  int64_t D, const int8_t* code, const int32_t* slot,
                                  const void* const* buckets, int scale_dtype, int64_t S_kv,
                                  int64_t group, float sm_scale, void* out, int out_dtype,
                                  void* workspace, size_t workspace_bytes, si_stream_t stream) {
  clear_error();
  const OutStrides os{H * S_q * D, S_q * D, D};
  return run_attn(q, q_dtype, B, H, S_q, D, code, slot, buckets, scale_dtype, S_kv, group,
                  sm_scale, out, out_dtype, os, workspace, workspace_bytes, true,
                  as_stream(stream));
}

extern "C" int si_attn_packed_fwd_tokens(const void* q, int q_dtype, int64_t B, int64_t H,
                                         int64_t S_q, int64_t D, const int8_t* code,
                                         const int32_t* slot, const void* const* buckets,
                                         int scale_dtype, int64_t S_kv, int64_t group,
                                         float sm_scale, void* out, int out_dtype,
                                         void* workspace, size_t workspace_bytes,
                                         si_stream_t stream) {
  clear_error();
  const OutStrides os{S_q * H * D, D, H * D};
  return run_attn(q, q_dtype, B, H, S_q, D, code, slot, buckets, scale_dtype, S_kv, group,
                  sm_scale, out, out_dtype, os, workspace, workspace_bytes, true,
                  as_stream(stream));
}

extern "C" int si_attn_build_lists(const int8_t* code, const int32_t* slot, int64_t H,
                                   int64_t S_kv, void* workspace, size_t workspace_bytes,
                                   si_stream_t stream) {
  clear_error();
  SI_CHECK_ARG(H >= 0 && H < 65536 && S_kv > 0 && S_kv < ((int64_t)1 << 30),
               "si_attn_build_lists: bad shape");
  if (H == 0) return SI_OK;
  SI_CHECK_ARG(code && slot, "si_attn_build_lists: NULL argument");
  const size_t need = si_attn_workspace_bytes(H, S_kv);
  SI_CHECK_ARG(workspace != nullptr && workspace_bytes >= need &&
                   (reinterpret_cast<uintptr_t>(workspace) & 15) == 0,
               "si_attn_build_lists: workspace too small or misaligned (%zu < %zu bytes)",
               workspace_bytes, need);
  int32_t* counts = reinterpret_cast<int32_t*>(workspace);
  attn_lists<<<(unsigned)H, 256, 0, as_stream(stream)>>>(code, slot, H, S_kv, list_cap(S_kv),
                                                          counts, counts + H * 8);
  return check_launch("si_attn_build_lists");
}

extern "C" int si_attn_packed_fwd_built(const void* q, int q_dtype, int64_t B, int64_t H,
                                        int64_t S_q, int64_t D, const void* lists,
                                        size_t lists_bytes, const void* const* buckets,
                                        int scale_dtype, int64_t S_kv, int64_t group,
                                        float sm_scale, void* out, int out_dtype,
                                        int token_major, si_stream_t stream) {
  clear_error();
  const OutStrides os = token_major ? OutStrides{S_q * H * D, D, H * D}
                                    : OutStrides{H * S_q * D, S_q * D, D};
  return run_attn(q, q_dtype, B, H, S_q, D, nullptr, nullptr, buckets, scale_dtype, S_kv, group,
                  sm_scale, out, out_dtype, os, const_cast<void*>(lists), lists_bytes, false,
                  as_stream(stream));
}
