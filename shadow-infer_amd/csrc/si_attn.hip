// Fused dequantize + bidirectional attention over a packed KV cache (gfx950).
//
// Semantics: out = softmax(q k^T * sm_scale) v with no mask, where k/v are the
// values PackedKVCache.unpack() would produce (packed_kv_cache.py:535-577):
// evicted or absent token-heads are zero vectors and still take part in the
// softmax, exactly as in unpack() -> dense attention
// (models/simple_diffusion_llm.py:165-169). The dense K/V never exist: each
// 64-token tile is dequantized straight into LDS as fp16.
//
// Work split: one block of 4 wavefronts owns 128 queries of one (b, h); each
// wave owns 32 queries. Per 64-key tile a wave computes S^T = K Q^T with
// v_mfma_f32_32x32x16_f16, so lane l holds scores of query (l % 32) for 16 of
// the tile's keys and lane l ^ 32 the other 16: the online-softmax max and sum
// need one cross-lane shuffle. O^T = V^T P^T then reuses the score registers
// as the B operand; the k order of an MFMA only has to match between its A and
// B operands, so V^T is read from LDS in the key order the score accumulator
// already has (keys 8*(i/4) + 4*(l/32) + i%4 of each 16-key chunk).
//
// Precision: fp16 operands (10-bit mantissa) with fp32 accumulation and an
// fp32 online softmax; fp16 entries of the cache are exact in fp16, int8/int4
// values q*s are rounded once to fp16.
#include "si_kv_common.h"

namespace si {
namespace {

typedef _Float16 v8h __attribute__((ext_vector_type(8)));
typedef _Float16 v4h __attribute__((ext_vector_type(4)));
typedef float v16f __attribute__((ext_vector_type(16)));

constexpr int BM = 128;  // queries per block
constexpr int BN = 64;   // keys per tile
constexpr int KPAD = 8;  // fp16 padding per LDS row

template <int QDT>
__device__ __forceinline__ _Float16 q_to_h(uint32_t bits) {
  const float f = QDT == SI_DT_BF16 ? bf16_bits_to_f32(bits) : f16_bits_to_f32(bits);
  return (_Float16)f;
}


template <int D, int SDT, int QDT>
__global__ __launch_bounds__(256) void attn_packed_fwd(const uint16_t* __restrict__ Q,
                                                       int64_t B, int64_t H, int64_t Sq,
                                                       int64_t Skv, const int8_t* __restrict__ code,
                                                       const int32_t* __restrict__ slot,
                                                       Buckets bk, int64_t g, float scale_log2,
                                                       void* __restrict__ O, int odt) {
  constexpr int KS = D / 16;   // MFMA k-steps over the head dim
  constexpr int DB = D / 32;   // 32-row blocks of O^T
  constexpr int DPT = D / 4;   // head-dim values per thread in the dequant stage
  __shared__ __attribute__((aligned(16))) _Float16 Ks[BN][D + KPAD];
  __shared__ __attribute__((aligned(16))) _Float16 Vt[D][BN + KPAD];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int col = lane & 31;  // query column within the wave
  const int grp = lane >> 5;  // 0/1: k-half of MFMA operands, row quad of results
  const int64_t h = blockIdx.y;
  const int64_t b = blockIdx.z;
  const int64_t m = (int64_t)blockIdx.x * BM + wave * 32 + col;
  const bool m_ok = m < Sq;

  // Q^T fragments (B operand of S^T = K Q^T): query m, dims ks*16 + 8*grp + 0..7.
  v8h qf[KS];
  {
    const uint16_t* qrow = Q + (((b * H + h) * Sq) + (m_ok ? m : 0)) * D;
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      uint4 raw = make_uint4(0, 0, 0, 0);
      if (m_ok) raw = *reinterpret_cast<const uint4*>(qrow + ks * 16 + 8 * grp);
      const uint32_t w[4] = {raw.x, raw.y, raw.z, raw.w};
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        qf[ks][2 * i] = q_to_h<QDT>(w[i] & 0xffffu);
        qf[ks][2 * i + 1] = q_to_h<QDT>(w[i] >> 16);
      }
    }
  }

  v16f o[DB];
#pragma unroll
  for (int i = 0; i < DB; ++i)
#pragma unroll
    for (int r = 0; r < 16; ++r) o[i][r] = 0.0f;
  float m_run = -INFINITY;
  float l_run = 0.0f;

  const int dj = tid >> 2;          // key of this thread in the dequant stage
  const int dd = (tid & 3) * DPT;   // first head-dim value of this thread

  for (int64_t kv0 = 0; kv0 < Skv; kv0 += BN) {
    // ---- dequantize the K/V tile into LDS ----
    __syncthreads();
    {
      const int64_t t = kv0 + dj;
      int c = SI_PREC_EVICTED;
      int64_t s = 0;
      if (t < Skv) {
        const int64_t e = t * H + h;
        c = code[e];
        if (c >= 0 && c <= 3) s = slot[e];
      }
      const bool present = c >= 0 && c <= 3;
#pragma unroll
      for (int d4 = 0; d4 < DPT; d4 += 4) {
        float4 kv = make_float4(0.f, 0.f, 0.f, 0.f), vv = kv;
        if (present) {
          kv = dequant4<SDT>(bk, 0, c, s, b, dd + d4, B, D, g);
          vv = dequant4<SDT>(bk, 1, c, s, b, dd + d4, B, D, g);
        }
        v4h kh;
        kh[0] = (_Float16)kv.x;
        kh[1] = (_Float16)kv.y;
        kh[2] = (_Float16)kv.z;
        kh[3] = (_Float16)kv.w;
        *reinterpret_cast<v4h*>(&Ks[dj][dd + d4]) = kh;
        Vt[dd + d4 + 0][dj] = (_Float16)vv.x;
        Vt[dd + d4 + 1][dj] = (_Float16)vv.y;
        Vt[dd + d4 + 2][dj] = (_Float16)vv.z;
        Vt[dd + d4 + 3][dj] = (_Float16)vv.w;
      }
    }
    __syncthreads();

    // ---- S^T = K Q^T for keys kv0 + [0, 64) ----
    v16f sacc[2];
#pragma unroll
    for (int kb = 0; kb < 2; ++kb) {
#pragma unroll
      for (int r = 0; r < 16; ++r) sacc[kb][r] = 0.0f;
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) {
        const v8h a = *reinterpret_cast<const v8h*>(&Ks[kb * 32 + col][ks * 16 + 8 * grp]);
        sacc[kb] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, qf[ks], sacc[kb], 0, 0, 0);
      }
    }

    // ---- online softmax (log2 domain) ----
    float tmax = -INFINITY;
#pragma unroll
    for (int kb = 0; kb < 2; ++kb) {
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int key = kb * 32 + 8 * (r >> 2) + 4 * grp + (r & 3);
        float v = sacc[kb][r] * scale_log2;
        if (kv0 + key >= Skv) v = -INFINITY;
        sacc[kb][r] = v;
        tmax = fmaxf(tmax, v);
      }
    }
    tmax = fmaxf(tmax, __shfl_xor(tmax, 32, 64));
    const float m_new = fmaxf(m_run, tmax);
    const float alpha = exp2f(m_run - m_new);
    float psum = 0.0f;
#pragma unroll
    for (int kb = 0; kb < 2; ++kb) {
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const float p = exp2f(sacc[kb][r] - m_new);
        sacc[kb][r] = p;
        psum += p;
      }
    }
    psum += __shfl_xor(psum, 32, 64);
    l_run = l_run * alpha + psum;
    m_run = m_new;
#pragma unroll
    for (int i = 0; i < DB; ++i)
#pragma unroll
      for (int r = 0; r < 16; ++r) o[i][r] *= alpha;

    // ---- O^T += V^T P^T over four 16-key chunks ----
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      const int kb = c >> 1;
      const int hc = c & 1;
      v8h pb;
#pragma unroll
      for (int i = 0; i < 8; ++i) pb[i] = (_Float16)sacc[kb][8 * hc + i];
#pragma unroll
      for (int db = 0; db < DB; ++db) {
        const _Float16* vrow = &Vt[db * 32 + col][c * 16 + 4 * grp];
        const v4h lo = *reinterpret_cast<const v4h*>(vrow);
        const v4h hi = *reinterpret_cast<const v4h*>(vrow + 8);
        const v8h a = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
        o[db] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, pb, o[db], 0, 0, 0);
      }
    }
  }

  if (!m_ok) return;
  const float inv = 1.0f / l_run;
  const int64_t obase = ((b * H + h) * Sq + m) * D;
#pragma unroll
  for (int db = 0; db < DB; ++db) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int d = db * 32 + 8 * i + 4 * grp;
      const float r0 = o[db][4 * i + 0] * inv, r1 = o[db][4 * i + 1] * inv;
      const float r2 = o[db][4 * i + 2] * inv, r3 = o[db][4 * i + 3] * inv;
      if (odt == SI_DT_F32) {
        *reinterpret_cast<float4*>(reinterpret_cast<float*>(O) + obase + d) =
            make_float4(r0, r1, r2, r3);
      } else {
        const bool bf = odt == SI_DT_BF16;
        const uint32_t w0 = (bf ? f32_to_bf16_bits(r0) : f32_to_f16_bits(r0)) |
                            ((bf ? f32_to_bf16_bits(r1) : f32_to_f16_bits(r1)) << 16);
        const uint32_t w1 = (bf ? f32_to_bf16_bits(r2) : f32_to_f16_bits(r2)) |
                            ((bf ? f32_to_bf16_bits(r3) : f32_to_f16_bits(r3)) << 16);
        *reinterpret_cast<uint2*>(reinterpret_cast<uint16_t*>(O) + obase + d) = make_uint2(w0, w1);
      }
    }
  }
}

template <int D, int QDT>
void launch_attn(int sdt, dim3 grid, hipStream_t st, const uint16_t* q, int64_t B, int64_t H,
                 int64_t Sq, int64_t Skv, const int8_t* code, const int32_t* slot,
                 const Buckets& bk, int64_t g, float scale_log2, void* out, int odt) {
  switch (sdt) {
    case SI_DT_F32:
      attn_packed_fwd<D, SI_DT_F32, QDT><<<grid, 256, 0, st>>>(q, B, H, Sq, Skv, code, slot, bk, g,
                                                               scale_log2, out, odt);
      break;
    case SI_DT_F16:
      attn_packed_fwd<D, SI_DT_F16, QDT><<<grid, 256, 0, st>>>(q, B, H, Sq, Skv, code, slot, bk, g,
                                                               scale_log2, out, odt);
      break;
    default:
      attn_packed_fwd<D, SI_DT_BF16, QDT><<<grid, 256, 0, st>>>(q, B, H, Sq, Skv, code, slot, bk,
                                                                g, scale_log2, out, odt);
  }
}

}  // namespace
}  // namespace si

using namespace si;

extern "C" int si_attn_packed_fwd(const void* q, int q_dtype, int64_t B, int64_t H, int64_t S_q,
                                  int64_t D, const int8_t* code, const int32_t* slot,
                                  const void* const* buckets, int scale_dtype, int64_t S_kv,
                                  int64_t group, float sm_scale, void* out, int out_dtype,
                                  si_stream_t stream) {
  clear_error();
  SI_CHECK_ARG(q_dtype == SI_DT_BF16 || q_dtype == SI_DT_F16,
               "si_attn_packed_fwd: q dtype must be bf16 or fp16 (got %d)", q_dtype);
  SI_CHECK_ARG(dtype_ok(scale_dtype), "si_attn_packed_fwd: unsupported scale dtype %d",
               scale_dtype);
  SI_CHECK_ARG(dtype_ok(out_dtype), "si_attn_packed_fwd: unsupported out dtype %d", out_dtype);
  SI_CHECK_ARG(D == 64 || D == 128, "si_attn_packed_fwd: head_dim must be 64 or 128 (got %lld)",
               (long long)D);
  SI_CHECK_ARG(B >= 0 && H >= 0 && S_q >= 0 && S_kv > 0, "si_attn_packed_fwd: bad shape");
  SI_CHECK_ARG(group > 0 && D % group == 0 && group % 4 == 0,
               "si_attn_packed_fwd: int4 group must divide head_dim and be a multiple of 4");
  SI_CHECK_ARG(H < 65536 && B < 65536, "si_attn_packed_fwd: H and B must be < 65536");
  if (B * H * S_q == 0) return SI_OK;
  SI_CHECK_ARG(q && code && slot && buckets && out, "si_attn_packed_fwd: NULL argument");
  const Buckets bk = to_buckets(buckets);
  const dim3 grid((unsigned)ceil_div(S_q, BM), (unsigned)H, (unsigned)B);
  const float scale_log2 = sm_scale * 1.4426950408889634f;
  const uint16_t* qp = reinterpret_cast<const uint16_t*>(q);
  hipStream_t st = as_stream(stream);
  if (D == 128) {
    if (q_dtype == SI_DT_BF16)
      launch_attn<128, SI_DT_BF16>(scale_dtype, grid, st, qp, B, H, S_q, S_kv, code, slot, bk,
                                   group, scale_log2, out, out_dtype);
    else
      launch_attn<128, SI_DT_F16>(scale_dtype, grid, st, qp, B, H, S_q, S_kv, code, slot, bk,
                                  group, scale_log2, out, out_dtype);
  } else {
    if (q_dtype == SI_DT_BF16)
      launch_attn<64, SI_DT_BF16>(scale_dtype, grid, st, qp, B, H, S_q, S_kv, code, slot, bk,
                                  group, scale_log2, out, out_dtype);
    else
      launch_attn<64, SI_DT_F16>(scale_dtype, grid, st, qp, B, H, S_q, S_kv, code, slot, bk,
                                 group, scale_log2, out, out_dtype);
  }
  return check_launch("si_attn_packed_fwd");
}
