// int8 x int8 -> int32 GEMM on gfx950 MFMA with the INT8Linear dequant
// epilogue (ffn_optimizer/int8_linear.py:102-115).
//
// Operands: A = quantized activations [M, K], B = quantized weight [N, K]
// (nn.Linear's layout). Both are K-contiguous, which is the register layout
// of MFMA fragments, so tiles move as 16-byte chunks with no transposition.
//
// Kernels (choose() picks one per shape):
//  * gemm_dma (M > 32, and M > 16 outside gemm_rows' widths): BM x BN x BK
//    tiles copied global -> LDS by buffer_load_dwordx4 ... lds (no register
//    staging) into separate A and B rings, the weight k-tiles further ahead,
//    XOR-swizzled 16-byte chunks, v_mfma_i32_32x32x32_i8 on a 2x2, 4x2 or
//    2x4 wave grid; K split over the grid where the tiles alone leave CUs idle.
//  * gemm_rows (M <= 32, 16-48 weight rows per CU): one block per CU streams
//    its own weight rows once through 256-byte LDS runs.
//  * gemm_stream (M <= 16 on the other widths): weight and activation
//    fragments straight into registers, K split over the block's waves and
//    the int32 partials added in LDS.
//  * gemm_tile: register-staged copies into double-buffered, padded LDS;
//    where K is not a multiple of 64 or an operand reaches 2^31 bytes.
//  * gemm_skinny: split-K weight streaming with global partials, reachable
//    only through si_tune_gemm_plan; gemm_i8_scalar: K not a multiple of 32.
//
// Fragment layouts: 16x16x64 - lane l holds A row (l%16) / B row (l%16), 16
// consecutive k starting at 16*(l/16); C lane l holds rows 4*(l/16)+r, r<4, of
// column l%16. 32x32x32 - lane l holds A/B row (l%32), 16 consecutive k
// starting at 16*(l/32); C lane l holds rows 8*(r/4) + 4*(l/32) + r%4, r<16,
// of column l%32. The k order inside a fragment only has to agree between A
// and B, which it does by construction, so the int32 sums are exact.
//
// Split-K partial sums are int32 and are added by gemm_finalize (integer adds:
// the result does not depend on the order).
#include <atomic>
#include <mutex>

#include "si_common.h"

namespace si {
namespace {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));

enum Epi { EPI_I32 = 0, EPI_PARTIAL = 1, EPI_DEQUANT = 2, EPI_RESID = 256 };

struct EpiArgs {
  const float* sx;
  const float* sw;
  const float* bias;
  void* out;
  int out_dtype;
  int32_t* partial;  // [splits, M, N] when EPI_PARTIAL
  int vec;           // 16-byte stores allowed: N % 8 == 0 and every output/scale pointer aligned
  const void* resid; // [M, N] in the output dtype, or null: out = T(resid + T(projection))
};

// The residual add that follows a projection in the reference's decoder layer
// (models/diffusion_llama.py:421-423): the INT8Linear output is rounded to the
// output dtype T (int8_linear.py:115), then added to the residual stream in T.
// The caller's store rounds the sum to T. `out` may alias `resid`: every
// element is read by the thread that writes it, before the write.
template <int ODT>
__device__ __forceinline__ float add_resid(const EpiArgs& ep, int64_t idx, float o) {
  if (ep.resid == nullptr) return o;
  return round_to(o, ODT) + load_any(ep.resid, ODT, idx);
}
__device__ __forceinline__ float add_resid_rt(const EpiArgs& ep, int64_t idx, float o) {
  if (ep.resid == nullptr) return o;
  return round_to(o, ep.out_dtype) + load_any(ep.resid, ep.out_dtype, idx);
}

// out = T(float(acc) * (sx * sw) [+ bias]) with the reference's rounding order
// (then the residual add when ep.resid is set).
__device__ __forceinline__ void store_dequant(const EpiArgs& ep, int64_t idx, int32_t acc, float sx,
                                              float sw, float bias) {
  const float sc = sx * sw;
  float o = (float)acc * sc;
  if (ep.bias != nullptr) o = o + bias;
  store_any(ep.out, ep.out_dtype, idx, add_resid_rt(ep, idx, o));
}

template <int EPI>
__device__ __forceinline__ void epi_store(const EpiArgs& ep, int32_t* C, int64_t M, int64_t N,
                                          int64_t m, int64_t n, int32_t v, int split) {
  if (EPI == EPI_I32) {
    C[m * N + n] = v;
  } else if (EPI == EPI_PARTIAL) {
    ep.partial[((int64_t)split * M + m) * N + n] = v;
  } else {
    store_dequant(ep, m * N + n, v, ep.sx[m], ep.sw[n], ep.bias != nullptr ? ep.bias[n] : 0.0f);
  }
}

// ---------------------------------------------------------------------------
// Tile kernel. Requires K % BK == 0 (K per split too).
// Pipeline: two LDS stages and two register staging sets. While the MFMAs of
// k-tile t run from LDS stage t%2, the global loads of k-tile t+2 are in
// flight and k-tile t+1 waits in registers to be stored into the other stage
// after the MFMAs. Within a k-tile the fragments of k-step s+1 are read from
// LDS before the MFMAs of k-step s are issued.
// ---------------------------------------------------------------------------
template <int BM, int BN, int BK>
struct TileCfg {
  static constexpr int P = BK + 16;  // LDS row pitch in bytes
  static constexpr int CPR = BK / 16;
  static constexpr int ACH = BM * CPR / 256;
  static constexpr int BCH = BN * CPR / 256;
  static constexpr int STAGE = (BM + BN) * P;
};

template <int BM, int BN, int BK>
__device__ __forceinline__ void tile_gload(v4i* ra, v4i* rb, const int8_t* __restrict__ A,
                                           const int8_t* __restrict__ B, int M, int N, int K,
                                           int m0, int n0, int k0) {
  using C = TileCfg<BM, BN, BK>;
  const int tid = threadIdx.x;
#pragma unroll
  for (int i = 0; i < C::ACH; ++i) {
    const int c = tid + i * 256;
    const int m = m0 + c / C::CPR;
    ra[i] = m < M ? *reinterpret_cast<const v4i*>(A + (int64_t)m * K + k0 + (c % C::CPR) * 16)
                  : v4i{0, 0, 0, 0};
  }
#pragma unroll
  for (int i = 0; i < C::BCH; ++i) {
    const int c = tid + i * 256;
    const int n = n0 + c / C::CPR;
    rb[i] = n < N ? *reinterpret_cast<const v4i*>(B + (int64_t)n * K + k0 + (c % C::CPR) * 16)
                  : v4i{0, 0, 0, 0};
  }
}

template <int BM, int BN, int BK>
__device__ __forceinline__ void tile_sstore(int8_t* stage, const v4i* ra, const v4i* rb) {
  using C = TileCfg<BM, BN, BK>;
  const int tid = threadIdx.x;
#pragma unroll
  for (int i = 0; i < C::ACH; ++i) {
    const int c = tid + i * 256;
    *reinterpret_cast<v4i*>(stage + (c / C::CPR) * C::P + (c % C::CPR) * 16) = ra[i];
  }
#pragma unroll
  for (int i = 0; i < C::BCH; ++i) {
    const int c = tid + i * 256;
    *reinterpret_cast<v4i*>(stage + (BM + c / C::CPR) * C::P + (c % C::CPR) * 16) = rb[i];
  }
}

template <int BM, int BN, int BK, int WM, int WN>
__device__ __forceinline__ void tile_compute(const int8_t* stage, v16i (*acc)[BN / WN / 32],
                                             int wm, int wn, int lane) {
  using C = TileCfg<BM, BN, BK>;
  constexpr int TM = BM / WM, TN = BN / WN;
  constexpr int FM = TM / 32, FN = TN / 32;
  constexpr int KS = BK / 32;
  const int8_t* As = stage + (wm * TM + (lane & 31)) * C::P + (lane >> 5) * 16;
  const int8_t* Bs = stage + (BM + wn * TN + (lane & 31)) * C::P + (lane >> 5) * 16;
  v4i af[2][FM], bf[2][FN];
#pragma unroll
  for (int i = 0; i < FM; ++i) af[0][i] = *reinterpret_cast<const v4i*>(As + i * 32 * C::P);
#pragma unroll
  for (int j = 0; j < FN; ++j) bf[0][j] = *reinterpret_cast<const v4i*>(Bs + j * 32 * C::P);
#pragma unroll
  for (int ks = 0; ks < KS; ++ks) {
    const int cur = ks & 1;
    if (ks + 1 < KS) {
#pragma unroll
      for (int i = 0; i < FM; ++i)
        af[cur ^ 1][i] = *reinterpret_cast<const v4i*>(As + i * 32 * C::P + (ks + 1) * 32);
#pragma unroll
      for (int j = 0; j < FN; ++j)
        bf[cur ^ 1][j] = *reinterpret_cast<const v4i*>(Bs + j * 32 * C::P + (ks + 1) * 32);
    }
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
      for (int j = 0; j < FN; ++j)
        acc[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(af[cur][i], bf[cur][j], acc[i][j], 0, 0, 0);
  }
}

// Dequant store with the output dtype fixed at compile time.
template <int ODT>
__device__ __forceinline__ void store_out(void* out, int64_t idx, float v) {
  if (ODT == SI_DT_F32) {
    reinterpret_cast<float*>(out)[idx] = v;
  } else {
    const uint32_t h = ODT == SI_DT_F16 ? f32_to_f16_bits(v) : f32_to_bf16_bits(v);
    reinterpret_cast<uint16_t*>(out)[idx] = (uint16_t)h;
  }
}

// EPI: EPI_I32 / EPI_PARTIAL; EPI_DEQUANT + 16 * out dtype for the dequant
// epilogue, + EPI_RESID when a residual is added (ep.resid set).
template <int BM, int BN, int BK, int WM, int WN, int EPI>
__global__ __launch_bounds__(256) void gemm_tile(const int8_t* __restrict__ A,
                                                 const int8_t* __restrict__ B, int M, int N, int K,
                                                 int k_split, int32_t* __restrict__ Cout,
                                                 EpiArgs ep) {
  static_assert(WM * WN == 4, "four waves per block");
  using C = TileCfg<BM, BN, BK>;
  constexpr int TM = BM / WM, TN = BN / WN;
  constexpr int FM = TM / 32, FN = TN / 32;
  static_assert(C::ACH * 256 == BM * C::CPR && C::BCH * 256 == BN * C::CPR, "chunks per thread");
  __shared__ __attribute__((aligned(16))) int8_t lds[2 * C::STAGE];

  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int wm = wave / WN;
  const int wn = wave % WN;
  const int m0 = blockIdx.y * BM;
  const int n0 = blockIdx.x * BN;
  const int kb = blockIdx.z * k_split;
  const int ke = min(kb + k_split, K);
  const int nk = (ke - kb) / BK;

  v16i acc[FM][FN];
#pragma unroll
  for (int i = 0; i < FM; ++i)
#pragma unroll
    for (int j = 0; j < FN; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0;

  v4i ra0[C::ACH], rb0[C::BCH], ra1[C::ACH], rb1[C::BCH];
  int8_t* s0 = lds;
  int8_t* s1 = lds + C::STAGE;
  if (nk > 0) tile_gload<BM, BN, BK>(ra0, rb0, A, B, M, N, K, m0, n0, kb);
  if (nk > 1) tile_gload<BM, BN, BK>(ra1, rb1, A, B, M, N, K, m0, n0, kb + BK);
  if (nk > 0) tile_sstore<BM, BN, BK>(s0, ra0, rb0);
  __syncthreads();
  for (int it = 0; it < nk; it += 2) {
    if (it + 2 < nk) tile_gload<BM, BN, BK>(ra0, rb0, A, B, M, N, K, m0, n0, kb + (it + 2) * BK);
    tile_compute<BM, BN, BK, WM, WN>(s0, acc, wm, wn, lane);
    if (it + 1 < nk) tile_sstore<BM, BN, BK>(s1, ra1, rb1);
    __syncthreads();
    if (it + 1 >= nk) break;
    if (it + 3 < nk) tile_gload<BM, BN, BK>(ra1, rb1, A, B, M, N, K, m0, n0, kb + (it + 3) * BK);
    tile_compute<BM, BN, BK, WM, WN>(s1, acc, wm, wn, lane);
    if (it + 2 < nk) tile_sstore<BM, BN, BK>(s0, ra0, rb0);
    __syncthreads();
  }

  const int col = lane & 31;
  const int rq = (lane >> 5) * 4;
  constexpr int KIND = EPI & 15;
  constexpr int ODT = (EPI >> 4) & 15;
#pragma unroll
  for (int j = 0; j < FN; ++j) {
    const int n = n0 + wn * TN + j * 32 + col;
    if (n >= N) continue;
    float sw = 0.0f, bias = 0.0f;
    if (KIND == EPI_DEQUANT) {
      sw = ep.sw[n];
      if (ep.bias != nullptr) bias = ep.bias[n];
    }
#pragma unroll
    for (int i = 0; i < FM; ++i) {
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int m = m0 + wm * TM + i * 32 + 8 * (r >> 2) + rq + (r & 3);
        if (m >= M) continue;
        const int32_t v = acc[i][j][r];
        const int64_t idx = (int64_t)m * N + n;
        if (KIND == EPI_I32) {
          Cout[idx] = v;
        } else if (KIND == EPI_PARTIAL) {
          ep.partial[(int64_t)blockIdx.z * M * N + idx] = v;
        } else {
          float o = (float)v * (ep.sx[m] * sw);
          if (ep.bias != nullptr) o = o + bias;
          if constexpr ((EPI & EPI_RESID) != 0) o = add_resid<ODT>(ep, idx, o);
          store_out<ODT>(ep.out, idx, o);
        }
      }
    }
  }
}

// ---------------------------------------------------------------------------
// DMA tile kernel: global -> LDS copies by buffer_load_dwordx4 ... lds (no
// register staging). The A part of each k-tile (BM x BK) goes to one of RA LDS
// slots and the B part (BN x BK) to one of RB slots; iteration t issues A(t +
// RA - 1) and B(t + RB - 1), so B runs RB - 1 k-tiles ahead. One wave
// instruction fills 1 KB of LDS, lane l the 16 bytes at 16*l: rows of a slot
// are therefore unpadded (BK bytes) and the 16-byte chunks of row r are stored
// at slot chunk ^ swz(r); swz spreads the rows read by one fragment load over
// distinct banks.
//
// Why the B ring is deeper: a CU fills its LDS at (L1->L2 reads in flight) x
// 128 B / latency, and the TCP holds only about 90 reads in flight. With two
// whole stages of a 256x192x128 tile (the LDS holds no third) the queue of
// copies ran dry at every k-tile boundary (about 70 reads in flight on
// average, 20 B per clock at 4096 x 11008, M = 1024). With A in 2 slots and B
// in 4 (160 KB), the weight rows of the next three k-tiles stay queued across
// the barrier: 87 in flight, 25.5 B per clock, and the loop 11% shorter.
// A resource descriptor with the exact buffer size per operand makes the
// copies 32-bit offsets from one scalar base (about 5% faster than 64-bit
// global_load_lds addresses) and bounds every read by the hardware.
//
// MFMA fragments are double-buffered in registers: the loads for k-slice s+1
// are issued between the MFMAs of k-slice s, and the first k-slice of k-tile
// t+1 is loaded during the last k-slice of k-tile t (after the one barrier per
// k-tile), so LDS latency stays behind the MFMA pipe. sched_group_barrier
// pins that interleave (the scheduler would otherwise sink every load next to
// its first use to save registers).
//
// Epilogue: the accumulators of each 32-row fragment row go through the wave's
// own LDS staging area, then every lane handles 8 consecutive outputs of one
// row: int32 as two 16-byte stores, dequantized values with one scale load per
// row and 16-byte stores of the output type.
//
// Requires K % BK == 0 (K per split too) and 16-byte aligned operands.
// ---------------------------------------------------------------------------
typedef __attribute__((address_space(1))) void gvoid_t;
typedef __attribute__((address_space(3))) void lvoid_t;

// 16 bytes per lane from byte `off` of a raw buffer of `bytes` bytes into LDS
// (buffer_load_dwordx4 ... lds; data format 32-bit, reads past `bytes` give 0).
__device__ __forceinline__ void buf_copy16(const void* base, uint32_t bytes, lvoid_t* dst,
                                           uint32_t off) {
  const __amdgpu_buffer_rsrc_t r =
      __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes, 0x00020000);
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, dst, 16, off, 0, 0, 0);
}

template <int CPR>
__device__ __forceinline__ int chunk_swz(int r) {
  if constexpr (CPR == 4) return ((r >> 1) ^ (r >> 2)) & 3;
  else return (r ^ (r >> 1)) & 7;
}

// s_waitcnt vmcnt(VM) lgkmcnt(LGKM), expcnt left alone (gfx9 encoding).
template <int VM, int LGKM = 15>
__device__ __forceinline__ void wait_cnt() {
  static_assert(VM >= 0 && VM < 64 && LGKM >= 0 && LGKM < 16, "counter range");
  __builtin_amdgcn_s_waitcnt((VM & 15) | ((VM >> 4) << 14) | (0x7 << 4) | (LGKM << 8));
}

// s_barrier without the fence of __syncthreads() (which would also wait for
// every copy in flight). The signal fences keep the compiler from moving
// memory accesses across it; callers wait for what must be complete first.
__device__ __forceinline__ void bare_barrier() {
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
  __builtin_amdgcn_s_barrier();
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
}

// Wait until at most n k-tiles of this wave's copies are still in flight
// (0 <= n <= S - 2), with every LDS read of this wave complete.
template <int LPT, int S, int I = S - 2>
__device__ __forceinline__ void wait_tiles(int n) {
  static_assert(S >= 2 && I * LPT <= 63, "vmcnt holds at most 63 outstanding loads");
  if constexpr (I <= 0) {
    wait_cnt<0, 0>();
  } else {
    if (n >= I) wait_cnt<I * LPT, 0>();
    else wait_tiles<LPT, S, I - 1>(n);
  }
}

// xcd_order (si_common.h): with M-tiles fastest, the tiles that read the same
// weight columns share one XCD's L2.

// 8 consecutive values of type ODT at element idx (16- or 32-byte aligned).
template <int ODT>
__device__ __forceinline__ void load8_out(const void* p, int64_t idx, float* r) {
  if constexpr (ODT == SI_DT_F32) {
    const float4 a = reinterpret_cast<const float4*>(reinterpret_cast<const float*>(p) + idx)[0];
    const float4 b = reinterpret_cast<const float4*>(reinterpret_cast<const float*>(p) + idx)[1];
    r[0] = a.x; r[1] = a.y; r[2] = a.z; r[3] = a.w; r[4] = b.x; r[5] = b.y; r[6] = b.z; r[7] = b.w;
  } else {
    const uint4 w = *reinterpret_cast<const uint4*>(reinterpret_cast<const uint16_t*>(p) + idx);
    const uint32_t ws[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      r[2 * e] = ODT == SI_DT_BF16 ? bf16_bits_to_f32(ws[e] & 0xffffu) : f16_bits_to_f32(ws[e] & 0xffffu);
      r[2 * e + 1] = ODT == SI_DT_BF16 ? bf16_bits_to_f32(ws[e] >> 16) : f16_bits_to_f32(ws[e] >> 16);
    }
  }
}

// A raw buffer over the rows of one 32-row band (band = first byte of its
// first row); offsets within a band stay below 2^32 because N * K < 2^31 and
// K >= 64.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t band_rsrc(void* band) {
  return __builtin_amdgcn_make_buffer_rsrc(wave_uniform(band), (short)0, -1, 0x00020000);
}

// 16 bytes at byte `off` of a band, stored with device scope (sc1): the lines
// are written through to memory as they leave, so less dirty data waits in L2
// for the end-of-kernel writeback (int32 out, 4096 x 11008: M = 1024 49.5 ->
// 48.8 us, M = 256 21.7 -> 21.2 us; 2048 x 4096 x 11008 96.4 -> 95.2 us).
__device__ __forceinline__ void store16_dev(const __amdgpu_buffer_rsrc_t& rs, uint32_t off, v4i v) {
  typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
  __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, v), rs, (int)off, 0, 16);
}

// Plain stores of 8 dequantized outputs (the dequantized tiles are half the
// bytes of int32 ones, and device-scope stores made them 1-2% slower).
template <int ODT>
__device__ __forceinline__ void store8(void* out, int64_t idx, const float* o) {
  if constexpr (ODT == SI_DT_F32) {
    float* p = reinterpret_cast<float*>(out) + idx;
    reinterpret_cast<float4*>(p)[0] = make_float4(o[0], o[1], o[2], o[3]);
    reinterpret_cast<float4*>(p)[1] = make_float4(o[4], o[5], o[6], o[7]);
  } else {
    uint32_t h[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) h[e] = ODT == SI_DT_F16 ? f32_to_f16_bits(o[e]) : f32_to_bf16_bits(o[e]);
    v4i w;
#pragma unroll
    for (int e = 0; e < 4; ++e) w[e] = (int)(h[2 * e] | (h[2 * e + 1] << 16));
    *reinterpret_cast<v4i*>(reinterpret_cast<uint16_t*>(out) + idx) = w;
  }
}

// Stores one 32-row band (FN fragments of 32x32 int32 accumulators) of a
// wave through its own LDS staging area of 16 x (32*FN + 8) words, in two
// passes of 16 rows, as 16-byte row stores: int32 in 4-column pieces (the
// lanes of one store cover whole 128-byte lines: 1024 x 4096 x 11008 51.3 ->
// 49.6 us against 8-column pieces stored as two half-line passes), or
// dequantized in 8-column pieces when EPI is EPI_DEQUANT + 16 * output dtype.
// Accumulator register r of a fragment
// holds row 8*(r/4) + 4*(lane/32) + r%4, column lane%32, so registers
// [8h, 8h+8) hold rows 16h .. 16h+15.
// Residual chunks of one band for one lane: for pass h and chunk slot s, the 8
// values at the element store_frag_row writes there (loaded before any store
// of the tile, so their latency is paid once per tile; each element is read
// by the lane that later writes it, so `out` may alias the residual).
template <int FN>
struct BandResid {
  static constexpr int CPL = (16 * (32 * FN / 8) + 63) / 64;  // chunks per lane per pass
  uint4 r[2][CPL];
};

template <int FN, int ODT>
__device__ __forceinline__ void load_band_resid(BandResid<FN>& br, int m_base, int n_base,
                                                int lane, int M, int N, const EpiArgs& ep) {
  constexpr int CH = 32 * FN / 8;
  constexpr int CPL = BandResid<FN>::CPL;
#pragma unroll
  for (int h = 0; h < 2; ++h)
#pragma unroll
    for (int s = 0; s < CPL; ++s) {
      const int c = lane + 64 * s;
      const int m = m_base + 16 * h + c / CH;
      const int n = n_base + (c % CH) * 8;
      br.r[h][s] = make_uint4(0, 0, 0, 0);
      if (c < 16 * CH && m < M && ep.vec && n + 8 <= N) {
        const int64_t idx = (int64_t)m * N + n;
        if constexpr (ODT == SI_DT_F32) {
          // two halves of 32 bytes do not fit a uint4: the fp32 path reads in the store loop
        } else {
          br.r[h][s] = *reinterpret_cast<const uint4*>(reinterpret_cast<const uint16_t*>(ep.resid) + idx);
        }
      }
    }
}

template <int FN, int EPI>
__device__ __forceinline__ void store_frag_row(const v16i* acc, int m_base, int n_base, int32_t* stg,
                                               int lane, int M, int N, int32_t* dst,
                                               const EpiArgs& ep, const BandResid<FN>* br) {
  constexpr int TN = 32 * FN;
  constexpr int EP = TN + 8;  // staging pitch in words (rows r and r+4 on other banks)
  constexpr int CH = TN / 8;  // 8-wide chunks per staged row
  constexpr int KIND = EPI & 15;
  constexpr int ODT = (EPI >> 4) & 15;
  constexpr bool RES = (EPI & EPI_RESID) != 0;
  const int col = lane & 31;
  const int rq = (lane >> 5) * 4;
#pragma unroll
  for (int h = 0; h < 2; ++h) {
#pragma unroll
    for (int j = 0; j < FN; ++j)
#pragma unroll
      for (int r = 8 * h; r < 8 * h + 8; ++r)
        stg[(8 * (r >> 2) - 16 * h + rq + (r & 3)) * EP + j * 32 + col] = acc[j][r];
    wait_cnt<63, 0>();
    __builtin_amdgcn_wave_barrier();
    if constexpr (KIND != EPI_DEQUANT) {
      // int32 rows: lanes store consecutive 16-byte pieces of a row, so each
      // store instruction writes whole 128-byte lines
      constexpr int CH4 = TN / 4;
      const __amdgpu_buffer_rsrc_t rs = band_rsrc(reinterpret_cast<char*>(dst) + (int64_t)m_base * N * 4);
#pragma unroll
      for (int s = 0; s < (16 * CH4 + 63) / 64; ++s) {
        const int c = lane + 64 * s;
        if (c >= 16 * CH4) continue;
        const int row = c / CH4;
        const int ch = c % CH4;
        const int m = m_base + 16 * h + row;
        const int n = n_base + ch * 4;
        if (m >= M || n >= N) continue;
        const v4i val = *reinterpret_cast<const v4i*>(stg + row * EP + ch * 4);
        const int64_t idx = (int64_t)m * N + n;
        if (ep.vec && n + 4 <= N) {
          store16_dev(rs, ((uint32_t)(16 * h + row) * (uint32_t)N + (uint32_t)n) * 4u, val);
        } else {
          for (int e = 0; e < 4 && n + e < N; ++e) dst[idx + e] = val[e];
        }
      }
      wait_cnt<63, 0>();
      __builtin_amdgcn_wave_barrier();
      continue;
    }
#pragma unroll
    for (int s = 0; s < BandResid<FN>::CPL; ++s) {
      const int c = lane + 64 * s;
      if (c >= 16 * CH) continue;
      const int row = c / CH;
      const int ch = c % CH;
      const int m = m_base + 16 * h + row;
      const int n = n_base + ch * 8;
      if (m >= M || n >= N) continue;
      const int32_t* sp = stg + row * EP + ch * 8;
      const v4i lo = *reinterpret_cast<const v4i*>(sp);
      const v4i hi = *reinterpret_cast<const v4i*>(sp + 4);
      const int32_t v[8] = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
      const int64_t idx = (int64_t)m * N + n;
      const bool full = ep.vec && n + 8 <= N;
      {
        const float sx = ep.sx[m];
        float o[8];
        if (full) {
          const float4 w0 = reinterpret_cast<const float4*>(ep.sw + n)[0];
          const float4 w1 = reinterpret_cast<const float4*>(ep.sw + n)[1];
          const float w[8] = {w0.x, w0.y, w0.z, w0.w, w1.x, w1.y, w1.z, w1.w};
#pragma unroll
          for (int e = 0; e < 8; ++e) o[e] = (float)v[e] * (sx * w[e]);
          if (ep.bias != nullptr) {
            const float4 b0 = reinterpret_cast<const float4*>(ep.bias + n)[0];
            const float4 b1 = reinterpret_cast<const float4*>(ep.bias + n)[1];
            const float bb[8] = {b0.x, b0.y, b0.z, b0.w, b1.x, b1.y, b1.z, b1.w};
#pragma unroll
            for (int e = 0; e < 8; ++e) o[e] = o[e] + bb[e];
          }
          if constexpr (RES) {
            float r[8];
            if constexpr (ODT == SI_DT_F32) {
              load8_out<ODT>(ep.resid, idx, r);
            } else {
              const uint4 w = br->r[h][s];
              const uint32_t ws[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
              for (int e = 0; e < 4; ++e) {
                r[2 * e] = ODT == SI_DT_BF16 ? bf16_bits_to_f32(ws[e] & 0xffffu) : f16_bits_to_f32(ws[e] & 0xffffu);
                r[2 * e + 1] = ODT == SI_DT_BF16 ? bf16_bits_to_f32(ws[e] >> 16) : f16_bits_to_f32(ws[e] >> 16);
              }
            }
#pragma unroll
            for (int e = 0; e < 8; ++e) o[e] = round_to(o[e], ODT) + r[e];
          }
          store8<ODT>(ep.out, idx, o);
        } else {
          for (int e = 0; e < 8 && n + e < N; ++e) {
            float x = (float)v[e] * (sx * ep.sw[n + e]);
            if (ep.bias != nullptr) x = x + ep.bias[n + e];
            if constexpr (RES) x = add_resid<ODT>(ep, idx + e, x);
            store_out<ODT>(ep.out, idx + e, x);
          }
        }
      }
    }
    wait_cnt<63, 0>();
    __builtin_amdgcn_wave_barrier();
  }
}

template <int BM, int BN, int BK, int WM, int WN, int RA, int RB, int EPI>
__global__ __launch_bounds__(64 * WM * WN) void gemm_dma(const int8_t* __restrict__ A,
                                                         const int8_t* __restrict__ B, int M,
                                                         int N, int K, int k_split,
                                                         int32_t* __restrict__ Cout, EpiArgs ep) {
  constexpr int NW = WM * WN;  // 4 waves (one per SIMD) or 8 (two per SIMD)
  static_assert(NW == 4 || NW == 8, "four or eight waves per block");
  static_assert(RA >= 2 && RB >= RA, "A ring no deeper than the B ring");
  constexpr int CPR = BK / 16;
  constexpr int LA = BM * BK / 1024 / NW;  // 1-KB DMA blocks of A per wave per k-tile
  constexpr int LB = BN * BK / 1024 / NW;
  static_assert(LA * 1024 * NW == BM * BK && LB * 1024 * NW == BN * BK, "whole DMA blocks per wave");
  constexpr int LPT = LA + LB;        // vm loads per thread per k-tile
  constexpr int ASZ = BM * BK, BSZ = BN * BK;
  constexpr int LDS_BYTES = RA * ASZ + RB * BSZ;
  constexpr int TM = BM / WM, TN = BN / WN;
  constexpr int FM = TM / 32, FN = TN / 32;
  static_assert(FM * 32 == TM && FN * 32 == TN, "32-row fragments");
  constexpr int KS = BK / 32;
  static_assert(KS % 2 == 0, "fragment buffers alternate per k-slice");
  constexpr int EP = TN + 8;  // epilogue staging pitch in words (rows r and r+4 on other banks)
  static_assert(NW * 16 * EP * 4 <= LDS_BYTES, "epilogue staging fits in the rings");
  static_assert(RA == RB ? (RA - 2) * LPT <= 63
                         : (RB - 2) * LB <= 63 && LB + (RA - 2) * (LA + LB) <= 63,
                "vmcnt range");
  __shared__ __attribute__((aligned(1024))) int8_t lds[LDS_BYTES];
  int8_t* const ldsA = lds;
  int8_t* const ldsB = lds + RA * ASZ;

  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int wm = wave / WN;
  const int wn = wave % WN;
  const int ntiles = (int)gridDim.x;
  const int g = xcd_order((int)(blockIdx.x + blockIdx.z * gridDim.x), ntiles * (int)gridDim.z);
  const int tile = g % ntiles;
  const int split = g / ntiles;
  const int nM = (M + BM - 1) / BM;
  const int m0 = (tile % nM) * BM;
  const int n0 = (tile / nM) * BN;
  const int kb = split * k_split;
  const int ke = min(kb + k_split, K);
  const int nk = (ke - kb) / BK;

  // Byte offset of the 16 bytes this lane copies into each of its DMA blocks
  // (operands are below 2^31 bytes; the host checks).
  const uint32_t abytes = (uint32_t)M * (uint32_t)K, bbytes = (uint32_t)N * (uint32_t)K;
  uint32_t aoff[LA], boff[LB];
#pragma unroll
  for (int i = 0; i < LA; ++i) {
    const int p = (i * NW + wave) * 1024 + 16 * lane;
    const int r = p / BK;
    const int c = ((p % BK) / 16) ^ chunk_swz<CPR>(r);
    const int m = min(m0 + r, M - 1);  // rows past M feed only discarded outputs
    aoff[i] = (uint32_t)m * (uint32_t)K + (uint32_t)(kb + 16 * c);
  }
#pragma unroll
  for (int i = 0; i < LB; ++i) {
    const int p = (i * NW + wave) * 1024 + 16 * lane;
    const int r = p / BK;
    const int c = ((p % BK) / 16) ^ chunk_swz<CPR>(r);
    const int n = min(n0 + r, N - 1);
    boff[i] = (uint32_t)n * (uint32_t)K + (uint32_t)(kb + 16 * c);
  }
  auto issueA = [&](int t) {
    int8_t* st = ldsA + (t % RA) * ASZ;
#pragma unroll
    for (int i = 0; i < LA; ++i)
      buf_copy16(A, abytes, (lvoid_t*)(st + (i * NW + wave) * 1024), aoff[i] + (uint32_t)(t * BK));
  };
  auto issueB = [&](int t) {
    int8_t* st = ldsB + (t % RB) * BSZ;
#pragma unroll
    for (int i = 0; i < LB; ++i)
      buf_copy16(B, bbytes, (lvoid_t*)(st + (i * NW + wave) * 1024), boff[i] + (uint32_t)(t * BK));
  };
  // This wave's copies of A(t+1) and B(t+1) have landed and its LDS reads are
  // complete (called at the end of iteration t; t = -1 before the loop).
  // Copies complete in issue order, so waiting until at most N are in flight
  // is safe whenever at least N were issued after A(t+1); B(t+1) is issued
  // before A(t+1) when RB > RA.
  auto wait_next = [&](int t) {
    if constexpr (RA == RB) {
      // iteration u issued A(u+RA-1), B(u+RA-1): up to RA-2 later k-tiles may fly
      wait_tiles<LPT, RA>(min(nk - 2 - t, RA - 2));
    } else if (t < 0) {
      // prologue issued A(j), B(j) for j < RA-1, then B(RA-1) .. B(RB-2), in
      // k order: B(1) .. B(min(RB-2, nk-1)) came after A(0) and B(0)
      wait_tiles<LB, RB>(min(nk - 1, RB - 2));
    } else if (t + RB - 1 < nk) {
      // A(t+1) was followed by the B k-tile of its iteration and by an A and a
      // B k-tile in each of the RA-2 later iterations
      wait_cnt<LB + (RA - 2) * (LA + LB), 0>();
    } else {
      // near the end: count only the A k-tiles issued after A(t+1)
      wait_tiles<LA, RA>(max(0, min(t + RA - 1, nk - 1) - t - 1));
    }
  };

  v16i acc[FM][FN];
#pragma unroll
  for (int i = 0; i < FM; ++i)
#pragma unroll
    for (int j = 0; j < FN; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0;

  // Fragment rows of this lane and their swizzles (fixed across k-tiles).
  int arow[FM], asw[FM], brow[FN], bsw[FN];
#pragma unroll
  for (int i = 0; i < FM; ++i) {
    const int r = wm * TM + i * 32 + (lane & 31);
    arow[i] = r * BK;
    asw[i] = chunk_swz<CPR>(r);
  }
#pragma unroll
  for (int j = 0; j < FN; ++j) {
    const int r = wn * TN + j * 32 + (lane & 31);
    brow[j] = r * BK;
    bsw[j] = chunk_swz<CPR>(r);
  }
  const int khalf = lane >> 5;
  v4i af[2][FM], bf[2][FN];
  auto load_frags = [&](int t, int ks, v4i* a, v4i* b) {
    const int8_t* sa = ldsA + (t % RA) * ASZ;
    const int8_t* sb = ldsB + (t % RB) * BSZ;
    const int c = 2 * ks + khalf;
#pragma unroll
    for (int i = 0; i < FM; ++i) a[i] = *reinterpret_cast<const v4i*>(sa + arow[i] + 16 * (c ^ asw[i]));
#pragma unroll
    for (int j = 0; j < FN; ++j) b[j] = *reinterpret_cast<const v4i*>(sb + brow[j] + 16 * (c ^ bsw[j]));
  };

  if (nk > 0) {
    // A(0 .. RA-2) and B(0 .. RB-2), in k order, A before B
#pragma unroll
    for (int j = 0; j < RB - 1; ++j) {
      if (j < RA - 1 && j < nk) issueA(j);
      if (j < nk) issueB(j);
    }
    wait_next(-1);
    bare_barrier();
    load_frags(0, 0, af[0], bf[0]);
  }
  for (int t = 0; t < nk; ++t) {
    // The slots of k-tile t-1 are free: every wave passed the barrier of
    // k-tile t-1's last k-slice after its reads of k-tile t-1 had completed.
    if (t + RA - 1 < nk) issueA(t + RA - 1);
    if (t + RB - 1 < nk) issueB(t + RB - 1);
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      const int cur = ks & 1;
      if (ks + 1 < KS) {
        load_frags(t, ks + 1, af[cur ^ 1], bf[cur ^ 1]);
      } else {
        // k-tile t+1: this wave's copies have landed and its reads of k-tile
        // t are complete; after the barrier the same holds for every wave.
        // Unconditional (branch-free, so the loads interleave with the MFMAs
        // below): after the last k-tile it waits for nothing and reads
        // stale slots whose fragments are never used.
        wait_next(t);
        bare_barrier();
        load_frags(t + 1, 0, af[cur ^ 1], bf[cur ^ 1]);
      }
#pragma unroll
      for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(af[cur][i], bf[cur][j], acc[i][j], 0, 0, 0);
      // Interleave: one MFMA, one LDS read, ... then the remaining MFMAs.
      constexpr int NL = FM + FN, NMF = FM * FN, NP = NL < NMF ? NL : NMF;
#pragma unroll
      for (int q = 0; q < NP; ++q) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
        __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
      }
      if constexpr (NMF > NP) __builtin_amdgcn_sched_group_barrier(0x008, NMF - NP, 0);
      if constexpr (NL > NP) __builtin_amdgcn_sched_group_barrier(0x100, NL - NP, 0);
    }
  }

  // ------------------------------------------------------------- epilogue
  __syncthreads();  // every wave is done with the stages
  int32_t* stg = reinterpret_cast<int32_t*>(lds) + wave * (16 * EP);
  int32_t* dst = (EPI & 15) == EPI_PARTIAL ? ep.partial + (int64_t)split * M * N : Cout;
  if constexpr ((EPI & EPI_RESID) != 0) {
    BandResid<FN> br[FM];
#pragma unroll
    for (int i = 0; i < FM; ++i)
      load_band_resid<FN, (EPI >> 4) & 15>(br[i], m0 + wm * TM + i * 32, n0 + wn * TN, lane, M, N, ep);
#pragma unroll
    for (int i = 0; i < FM; ++i)
      store_frag_row<FN, EPI>(acc[i], m0 + wm * TM + i * 32, n0 + wn * TN, stg, lane, M, N, dst,
                              ep, &br[i]);
  } else {
#pragma unroll
    for (int i = 0; i < FM; ++i)
      store_frag_row<FN, EPI>(acc[i], m0 + wm * TM + i * 32, n0 + wn * TN, stg, lane, M, N, dst,
                              ep, nullptr);
  }
}

// ---------------------------------------------------------------------------
// Skinny kernel (M <= 16*MF): each wavefront owns 16 output columns and one
// K range; fragments are loaded straight from global memory.
// Requires K % 64 == 0 and every split range a multiple of 64.
// ---------------------------------------------------------------------------
template <int MF, int EPI>
__global__ __launch_bounds__(256) void gemm_skinny(const int8_t* __restrict__ A,
                                                   const int8_t* __restrict__ B, int M, int N,
                                                   int K, int k_split, int32_t* __restrict__ C,
                                                   EpiArgs ep) {
  constexpr int UNROLL = 4;
  const int lane = threadIdx.x & 63;
  const int nb = blockIdx.x * 4 + (threadIdx.x >> 6);
  const int n = nb * 16 + (lane & 15);
  const int kofs = (lane >> 4) * 16;
  const int kb = blockIdx.y * k_split;
  const int ke = min(kb + k_split, K);
  if (nb * 16 >= N) return;
  const int8_t* brow = B + (int64_t)(n < N ? n : 0) * K + kofs;
  const int8_t* arow[MF];
  bool aok[MF];
#pragma unroll
  for (int i = 0; i < MF; ++i) {
    const int m = i * 16 + (lane & 15);
    aok[i] = m < M;
    arow[i] = A + (int64_t)(aok[i] ? m : 0) * K + kofs;
  }
  const bool bok = n < N;
  v4i acc[MF];
#pragma unroll
  for (int i = 0; i < MF; ++i) acc[i] = v4i{0, 0, 0, 0};
  int k0 = kb;
  for (; k0 + 64 * UNROLL <= ke; k0 += 64 * UNROLL) {
    v4i bf[UNROLL], af[UNROLL][MF];
#pragma unroll
    for (int u = 0; u < UNROLL; ++u) {
      bf[u] = bok ? __builtin_nontemporal_load(reinterpret_cast<const v4i*>(brow + k0 + 64 * u))
                  : v4i{0, 0, 0, 0};
#pragma unroll
      for (int i = 0; i < MF; ++i)
        af[u][i] = aok[i] ? *reinterpret_cast<const v4i*>(arow[i] + k0 + 64 * u) : v4i{0, 0, 0, 0};
    }
#pragma unroll
    for (int u = 0; u < UNROLL; ++u)
#pragma unroll
      for (int i = 0; i < MF; ++i)
        acc[i] = __builtin_amdgcn_mfma_i32_16x16x64_i8(af[u][i], bf[u], acc[i], 0, 0, 0);
  }
  for (; k0 < ke; k0 += 64) {
    const v4i bf = bok ? *reinterpret_cast<const v4i*>(brow + k0) : v4i{0, 0, 0, 0};
#pragma unroll
    for (int i = 0; i < MF; ++i) {
      const v4i af = aok[i] ? *reinterpret_cast<const v4i*>(arow[i] + k0) : v4i{0, 0, 0, 0};
      acc[i] = __builtin_amdgcn_mfma_i32_16x16x64_i8(af, bf, acc[i], 0, 0, 0);
    }
  }
  if (!bok) return;
#pragma unroll
  for (int i = 0; i < MF; ++i) {
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int m = i * 16 + (lane >> 4) * 4 + r;
      if (m < M) epi_store<EPI>(ep, C, M, N, m, n, acc[i][r], blockIdx.y);
    }
  }
}

// ---------------------------------------------------------------------------
// Weight-streaming kernel (M <= 16*MF, bound by reading the weight once): a
// block owns 16*NF output columns and its NW waves split K into NW ranges;
// their int32 partial sums are added in LDS, so nothing but the output leaves
// the block. Fragments use the 16x16x64 layout (lane l holds row or column
// l%16 and k bytes 16*(l/16) .. +15 of a 64-byte k step) and are loaded
// straight into registers in batches of U k steps, two batches in flight:
// one is multiplied while the next streams in.
// Requires K % 64 == 0.
// ---------------------------------------------------------------------------
template <int MF, int NF, int NW, int U, int EPI>
__global__ __launch_bounds__(64 * NW) void gemm_stream(const int8_t* __restrict__ A,
                                                       const int8_t* __restrict__ B, int M, int N,
                                                       int K, int32_t* __restrict__ C, EpiArgs ep) {
  constexpr int RP = 16 * NF + 4;  // LDS pitch (words) of a partial-sum row; rows 4 apart hit other banks
  constexpr int PART = MF * 16 * RP;
  __shared__ int32_t red[NW * PART];
  const int lane = threadIdx.x & 63;
  const int w = threadIdx.x >> 6;
  const int c = lane & 15;
  const int g = lane >> 4;
  const int n0 = blockIdx.x * 16 * NF;
  const int ksteps = K / 64;
  const int q = (ksteps + NW - 1) / NW;
  const int s0 = min(w * q, ksteps);
  const int s1 = min(s0 + q, ksteps);
  const int8_t* bp[NF];
  const int8_t* ap[MF];
#pragma unroll
  for (int j = 0; j < NF; ++j) bp[j] = B + (int64_t)min(n0 + 16 * j + c, N - 1) * K + 16 * g;
#pragma unroll
  for (int i = 0; i < MF; ++i) ap[i] = A + (int64_t)min(16 * i + c, M - 1) * K + 16 * g;

  v4i acc[MF][NF];
#pragma unroll
  for (int i = 0; i < MF; ++i)
#pragma unroll
    for (int j = 0; j < NF; ++j) acc[i][j] = v4i{0, 0, 0, 0};
  v4i b0[U][NF], a0[U][MF], b1[U][NF], a1[U][MF];
  auto load = [&](v4i (&bb)[U][NF], v4i (&aa)[U][MF], int s) {
#pragma unroll
    for (int u = 0; u < U; ++u) {
#pragma unroll
      for (int j = 0; j < NF; ++j)
        bb[u][j] = *reinterpret_cast<const v4i*>(bp[j] + 64 * (s + u));
#pragma unroll
      for (int i = 0; i < MF; ++i) aa[u][i] = *reinterpret_cast<const v4i*>(ap[i] + 64 * (s + u));
    }
  };
  auto mul = [&](v4i (&bb)[U][NF], v4i (&aa)[U][MF]) {
#pragma unroll
    for (int u = 0; u < U; ++u)
#pragma unroll
      for (int i = 0; i < MF; ++i)
#pragma unroll
        for (int j = 0; j < NF; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(aa[u][i], bb[u][j], acc[i][j], 0, 0, 0);
  };
  const int nb = (s1 - s0) / U;  // whole batches of this wave
  if (nb > 0) {
    load(b0, a0, s0);
    int bi = 0;
    for (; bi + 2 < nb; bi += 2) {
      load(b1, a1, s0 + (bi + 1) * U);
      mul(b0, a0);
      load(b0, a0, s0 + (bi + 2) * U);
      mul(b1, a1);
    }
    if (bi + 1 < nb) {  // two batches left: bi (in b0) and bi + 1
      load(b1, a1, s0 + (bi + 1) * U);
      mul(b0, a0);
      mul(b1, a1);
    } else {
      mul(b0, a0);
    }
  }
  for (int s = s0 + nb * U; s < s1; ++s) {
    v4i bb[1][NF], aa[1][MF];
#pragma unroll
    for (int j = 0; j < NF; ++j) bb[0][j] = *reinterpret_cast<const v4i*>(bp[j] + 64 * s);
#pragma unroll
    for (int i = 0; i < MF; ++i) aa[0][i] = *reinterpret_cast<const v4i*>(ap[i] + 64 * s);
#pragma unroll
    for (int i = 0; i < MF; ++i)
#pragma unroll
      for (int j = 0; j < NF; ++j)
        acc[i][j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(aa[0][i], bb[0][j], acc[i][j], 0, 0, 0);
  }

  // Partial sums to LDS: accumulator register r of fragment (i, j) holds row
  // 16i + 4(lane/16) + r, column 16j + lane%16.
  int32_t* mine = red + w * PART;
#pragma unroll
  for (int i = 0; i < MF; ++i)
#pragma unroll
    for (int j = 0; j < NF; ++j)
#pragma unroll
      for (int r = 0; r < 4; ++r) mine[(16 * i + 4 * g + r) * RP + 16 * j + c] = acc[i][j][r];
  __syncthreads();
  constexpr int W = 16 * NF;
  for (int e = threadIdx.x; e < MF * 16 * W; e += 64 * NW) {
    const int m = e / W;
    const int nn = e % W;
    const int n = n0 + nn;
    if (m >= M || n >= N) continue;
    int32_t v = 0;
#pragma unroll
    for (int x = 0; x < NW; ++x) v += red[x * PART + m * RP + nn];
    epi_store<EPI>(ep, C, M, N, m, n, v, 0);
  }
}

// ---------------------------------------------------------------------------
// Row-block streaming kernel (M <= 16*MF, one block per CU): a block owns RB
// <= 16*G consecutive weight rows over the full K, so the weight is read once
// and split evenly over the CUs (4096 x 11008: 43 rows per block, 256 blocks).
// Stage s holds k bytes [256 ks, 256 ks + 256) of the block's weight rows (LDS
// rows 0 .. 16G-1) and of the activation rows (LDS rows 16G .. 16G+16MF-1):
// each copy is one global_load_lds_dwordx4 of 4 rows x 256 contiguous bytes
// (row runs of 256 B keep the HBM bursts whole, where the 64-byte row pieces
// of direct fragment loads do not), chunk p of row r stored at slot p ^ (r &
// 15) so that the 16 rows of one fragment read fall on distinct banks. R
// stages rotate with one barrier per stage; wave w multiplies activation
// fragments w, w + 4, .. against all G weight groups over the whole stage, and
// the finished sums go through LDS once, for row-contiguous stores. Blocks
// start their k loop at different
// stages (the int32 sums do not depend on the order), which spreads the CUs
// of one XCD over different activation lines. The epilogue's scales are
// loaded before the first stage, so no load waits in the tail.
// Requires K % 256 == 0 and 1 <= RB <= 16*G.
// ---------------------------------------------------------------------------
template <int IPW, int I>
__device__ __forceinline__ void wait_stages(int n) {
  if constexpr (I <= 0) {
    wait_cnt<0, 15>();
  } else {
    if (n >= I) wait_cnt<I * IPW, 15>();
    else wait_stages<IPW, I - 1>(n);
  }
}

template <int MF, int G, int R, int EPI>
__global__ __launch_bounds__(256) void gemm_rows(const int8_t* __restrict__ A,
                                                 const int8_t* __restrict__ B, int M, int N, int K,
                                                 int RB, int32_t* __restrict__ C, EpiArgs ep) {
  constexpr int TR = 16 * (G + MF);  // LDS rows per stage
  constexpr int STAGE = TR * 256;
  constexpr int IPW = TR / 16;       // copies per wave per stage
  static_assert((R - 2) * IPW <= 63, "vmcnt holds at most 63 outstanding loads");
  __shared__ __attribute__((aligned(1024))) int8_t lds[R * STAGE];
  const int lane = threadIdx.x & 63;
  const int w = threadIdx.x >> 6;
  const int n0 = blockIdx.x * RB;
  const int nrows = min(RB, N - n0);
  const int stages = K / 256;
  const int rot = (blockIdx.x >> 3) % stages;
  // copy j of wave w fills LDS rows 4(4j + w) .. +3; padding rows re-read the
  // block's last weight row (an L2 hit) instead of another block's rows
  const int8_t* src[IPW];
#pragma unroll
  for (int j = 0; j < IPW; ++j) {
    const int r = 4 * (4 * j + w) + (lane >> 4);
    const int8_t* row = r < 16 * G ? B + (int64_t)(n0 + min(r, nrows - 1)) * K
                                   : A + (int64_t)min(r - 16 * G, M - 1) * K;
    src[j] = row + 16 * ((lane & 15) ^ (r & 15));
  }
  auto issue = [&](int s, int slot) {
    int ks = s + rot;
    ks = ks >= stages ? ks - stages : ks;
    int8_t* dst = lds + slot * STAGE + 1024 * w;
#pragma unroll
    for (int j = 0; j < IPW; ++j)
      __builtin_amdgcn_global_load_lds((gvoid_t*)(src[j] + 256 * ks), (lvoid_t*)(dst + 4096 * j),
                                       16, 0, 0);
  };
  // Outputs in 4-column pieces: item e = threadIdx.x + 256 x is activation row
  // e / PPR and weight rows 4 (e % PPR) .. +3 of the block. With RB a multiple
  // of 4 (the plan's choice) and ep.vec, a piece is one 16-byte (int32, fp32)
  // or 8-byte (fp16, bf16) store; its scales are loaded here, before the
  // first stage, so no load waits in the tail.
  constexpr int PPR = 4 * G;
  constexpr int IPT = (16 * MF * PPR + 255) / 256;
  const int mm = min(M, 16 * MF);
  const bool vec4 = ep.vec && RB % 4 == 0;
  float esx[IPT];
  float4 esw[IPT], eb[IPT];
#pragma unroll
  for (int x = 0; x < IPT; ++x) {
    const int e = threadIdx.x + 256 * x;
    const int m = e / PPR, j0 = 4 * (e - m * PPR);
    esx[x] = 0.0f;
    esw[x] = eb[x] = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    if (EPI == EPI_DEQUANT && m < mm && vec4 && j0 + 4 <= nrows) {
      esx[x] = ep.sx[m];
      esw[x] = *reinterpret_cast<const float4*>(ep.sw + n0 + j0);
      if (ep.bias != nullptr) eb[x] = *reinterpret_cast<const float4*>(ep.bias + n0 + j0);
    }
  }
#pragma unroll
  for (int u = 0; u < R - 1; ++u)
    if (u < stages) issue(u, u);
  const int fr = lane & 15, fc = lane >> 4;
  // The block's sums go through LDS for the row-contiguous stores below. Two
  // ways to split the MFMAs over the four waves:
  // - MF a multiple of 4: wave w owns activation fragments w, w + 4, .. against
  //   every weight group over all four 64-byte k-steps of each stage, so no
  //   partial sums cross waves and the finished sums go to LDS as
  //   [activation row][weight row], pitch TP words (M = 64: 13.0 -> 12.5 us,
  //   M = 128: 18.0 -> 16.6 us against the k-step split);
  // - otherwise wave w multiplies k-step w of each stage for every fragment,
  //   and the four waves' partial sums are added in LDS (with fewer than four
  //   fragments the other split would leave waves idle and run each stage's
  //   MFMAs as one wave's dependent chain: M = 16 9.5 -> 21 us).
  constexpr int TP = 16 * G + 4;       // tile pitch (words)
  constexpr int RP = 16 * MF + 4;      // partial-sum pitch (words)
  constexpr int PART = 16 * G * RP;    // one wave's partial sums
  int32_t* const red = reinterpret_cast<int32_t*>(lds);  // the tile, or the four partials
  int slot = 0;
  if constexpr (MF % 4 == 0) {
    static_assert(16 * MF * TP * 4 <= R * STAGE, "output tile fits in the stages");
    constexpr int IW = MF / 4;
    v4i acc[G][IW];
#pragma unroll
    for (int g = 0; g < G; ++g)
#pragma unroll
      for (int j = 0; j < IW; ++j) acc[g][j] = v4i{0, 0, 0, 0};
    for (int s = 0; s < stages; ++s) {
      wait_stages<IPW, R - 2>(stages - 1 - s);  // stages s+1 .. s+R-2 may stay in flight
      bare_barrier();                            // every wave's copies of stage s landed;
      if (s + R - 1 < stages)                    // every wave is done with stage s-1
        issue(s + R - 1, slot == 0 ? R - 1 : slot - 1);
      const int8_t* sb = lds + slot * STAGE + 256 * fr;
#pragma unroll
      for (int ks = 0; ks < 4; ++ks) {
        const int8_t* base = sb + 16 * ((4 * ks + fc) ^ fr);  // k step ks of a 16-row group
        v4i a[IW], b[G];
#pragma unroll
        for (int j = 0; j < IW; ++j) a[j] = *reinterpret_cast<const v4i*>(base + 4096 * (G + w + 4 * j));
#pragma unroll
        for (int g = 0; g < G; ++g) b[g] = *reinterpret_cast<const v4i*>(base + 4096 * g);
#pragma unroll
        for (int g = 0; g < G; ++g)
#pragma unroll
          for (int j = 0; j < IW; ++j)
            acc[g][j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(a[j], b[g], acc[g][j], 0, 0, 0);
      }
      slot = slot == R - 1 ? 0 : slot + 1;
    }
    __syncthreads();
    // accumulator register r of (g, j): activation row 16 (w + 4j) + 4 (lane / 16)
    // + r, weight row 16g + lane % 16
#pragma unroll
    for (int g = 0; g < G; ++g)
#pragma unroll
      for (int j = 0; j < IW; ++j)
#pragma unroll
        for (int r = 0; r < 4; ++r)
          red[(16 * (w + 4 * j) + 4 * fc + r) * TP + 16 * g + fr] = acc[g][j][r];
  } else {
    const int foff = 256 * fr + 16 * ((4 * w + fc) ^ fr);  // k step w of a 16-row group
    v4i acc[G][MF];
#pragma unroll
    for (int g = 0; g < G; ++g)
#pragma unroll
      for (int i = 0; i < MF; ++i) acc[g][i] = v4i{0, 0, 0, 0};
    for (int s = 0; s < stages; ++s) {
      wait_stages<IPW, R - 2>(stages - 1 - s);  // stages s+1 .. s+R-2 may stay in flight
      bare_barrier();                            // every wave's copies of stage s landed;
      if (s + R - 1 < stages)                    // every wave is done with stage s-1
        issue(s + R - 1, slot == 0 ? R - 1 : slot - 1);
      const int8_t* base = lds + slot * STAGE + foff;
      v4i a[MF], b[G];
#pragma unroll
      for (int i = 0; i < MF; ++i) a[i] = *reinterpret_cast<const v4i*>(base + 4096 * (G + i));
#pragma unroll
      for (int g = 0; g < G; ++g) b[g] = *reinterpret_cast<const v4i*>(base + 4096 * g);
#pragma unroll
      for (int g = 0; g < G; ++g)
#pragma unroll
        for (int i = 0; i < MF; ++i)
          acc[g][i] = __builtin_amdgcn_mfma_i32_16x16x64_i8(a[i], b[g], acc[g][i], 0, 0, 0);
      slot = slot == R - 1 ? 0 : slot + 1;
    }
    __syncthreads();
    // accumulator register r of (g, i): activation row 16i + 4(lane/16) + r,
    // weight row 16g + lane%16; wave w's partial sums at red + w * PART, added
    // by the stores below
    static_assert(4 * PART * 4 <= R * STAGE, "reduction area");
#pragma unroll
    for (int g = 0; g < G; ++g)
#pragma unroll
      for (int i = 0; i < MF; ++i)
#pragma unroll
        for (int r = 0; r < 4; ++r)
          red[w * PART + (16 * g + fr) * RP + 16 * i + 4 * fc + r] = acc[g][i][r];
  }
  __syncthreads();
#pragma unroll
  for (int x = 0; x < IPT; ++x) {
    const int e = threadIdx.x + 256 * x;
    const int m = e / PPR, j0 = 4 * (e - m * PPR);
    if (m >= mm || j0 >= nrows) continue;
    int32_t v[4];
    if constexpr (MF % 4 == 0) {
      const v4i tv = *reinterpret_cast<const v4i*>(red + m * TP + j0);
#pragma unroll
      for (int j = 0; j < 4; ++j) v[j] = tv[j];
    } else {
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        v[j] = 0;
#pragma unroll
        for (int y = 0; y < 4; ++y) v[j] += red[y * PART + (j0 + j) * RP + m];
      }
    }
    const int64_t idx = (int64_t)m * N + n0 + j0;
    if (!vec4 || j0 + 4 > nrows) {  // ragged last piece or unaligned operands
      for (int j = 0; j < 4 && j0 + j < nrows; ++j) epi_store<EPI>(ep, C, M, N, m, n0 + j0 + j, v[j], 0);
      continue;
    }
    if (EPI != EPI_DEQUANT) {  // device scope, as in the tiles' int32 epilogue (M = 128: 16.5 -> 15.8 us)
      store16_dev(band_rsrc(C + n0), ((uint32_t)m * (uint32_t)N + (uint32_t)j0) * 4u,
                  v4i{v[0], v[1], v[2], v[3]});
      continue;
    }
    const float w[4] = {esw[x].x, esw[x].y, esw[x].z, esw[x].w};
    const float bb[4] = {eb[x].x, eb[x].y, eb[x].z, eb[x].w};
    float o[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      o[j] = (float)v[j] * (esx[x] * w[j]);
      if (ep.bias != nullptr) o[j] = o[j] + bb[j];
    }
    if (ep.out_dtype == SI_DT_F32) {
      float* out = reinterpret_cast<float*>(ep.out) + idx;
      if (ep.resid != nullptr) {
        const float4 r = *reinterpret_cast<const float4*>(reinterpret_cast<const float*>(ep.resid) + idx);
        o[0] += r.x; o[1] += r.y; o[2] += r.z; o[3] += r.w;
      }
      *reinterpret_cast<float4*>(out) = make_float4(o[0], o[1], o[2], o[3]);
    } else {
      const bool f16 = ep.out_dtype == SI_DT_F16;
      if (ep.resid != nullptr) {
        const uint2 r = *reinterpret_cast<const uint2*>(reinterpret_cast<const uint16_t*>(ep.resid) + idx);
        const uint32_t rh[4] = {r.x & 0xffffu, r.x >> 16, r.y & 0xffffu, r.y >> 16};
#pragma unroll
        for (int j = 0; j < 4; ++j)
          o[j] = round_to(o[j], ep.out_dtype) + (f16 ? f16_bits_to_f32(rh[j]) : bf16_bits_to_f32(rh[j]));
      }
      uint32_t h[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) h[j] = f16 ? f32_to_f16_bits(o[j]) : f32_to_bf16_bits(o[j]);
      *reinterpret_cast<uint2*>(reinterpret_cast<uint16_t*>(ep.out) + idx) =
          make_uint2(h[0] | (h[1] << 16), h[2] | (h[3] << 16));
    }
  }
}

// Sum split-K partials (exact integer adds) and store int32 or dequantized.
__global__ __launch_bounds__(256) void gemm_finalize(const int32_t* __restrict__ partial,
                                                     int splits, int64_t M, int64_t N,
                                                     int32_t* __restrict__ C, EpiArgs ep,
                                                     int dequant) {
  const int64_t total = M * N;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total;
       i += (int64_t)gridDim.x * blockDim.x) {
    int32_t acc = 0;
    for (int s = 0; s < splits; ++s) acc += partial[(int64_t)s * total + i];
    if (!dequant) {
      C[i] = acc;
    } else {
      const int64_t m = i / N;
      const int64_t n = i - m * N;
      store_dequant(ep, i, acc, ep.sx[m], ep.sw[n], ep.bias != nullptr ? ep.bias[n] : 0.0f);
    }
  }
}

// Any-shape fallback (K not a multiple of 16): one thread per output.
__global__ __launch_bounds__(256) void gemm_i8_scalar(const int8_t* __restrict__ A,
                                                     const int8_t* __restrict__ B, int64_t M,
                                                     int64_t N, int64_t K, int32_t* __restrict__ C,
                                                     EpiArgs ep, int dequant) {
  const int64_t total = M * N;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total;
       i += (int64_t)gridDim.x * blockDim.x) {
    const int64_t m = i / N;
    const int64_t n = i - m * N;
    int32_t acc = 0;
    for (int64_t k = 0; k < K; ++k) acc += (int32_t)A[m * K + k] * (int32_t)B[n * K + k];
    if (!dequant) {
      C[i] = acc;
    } else {
      store_dequant(ep, i, acc, ep.sx[m], ep.sw[n], ep.bias != nullptr ? ep.bias[n] : 0.0f);
    }
  }
}

// ---------------------------------------------------------------------------
// Launch plans
// ---------------------------------------------------------------------------
enum Kind { K_SCALAR = 0, K_SKINNY = 1, K_TILE_128x128 = 3, K_DMA_256x256 = 6,
            K_DMA_128x256 = 7, K_DMA_128x128 = 8, K_DMA_256x128 = 9, K_DMA_256x192 = 10,
            K_DMA_256x64 = 11, K_DMA_256x128_K128 = 12,
            // eight waves per block (two per SIMD)
            K_DMA8_256x256 = 13, K_DMA8_256x256_K128 = 14, K_DMA8_256x192_K128 = 15,
            K_DMA8_256x128 = 16, K_DMA8_128x256 = 17,
            K_STREAM_N64 = 25, K_STREAM_N64_W8 = 27,
            // eight waves on a 128x128 tile (4x2 and 2x4 wave grids)
            K_DMA8_128x128_42 = 30, K_DMA8_128x128_24 = 31,
            // weight streaming with 32 / 16 output columns per block
            K_STREAM_N32 = 32, K_STREAM_N16 = 33, K_STREAM_N32_W8 = 34, K_STREAM_N16_W8 = 35,
            // 64-row tiles of the small-M choice (choose_fill): less row padding and
            // more blocks than 128x128 when few rows share the weight
            K_DMA_64x64 = 38, K_DMA_64x128 = 39,
            // one block per CU over ceil(N / 256) weight rows (gemm_rows)
            K_ROWS = 40,
            // four waves over a 128x96 tile (each 32 rows x 96 columns)
            K_DMA_128x96 = 41 };

struct Plan {
  int kind;
  int mf;       // skinny: 16-row fragments
  int splits;
  int k_split;  // k per split (multiple of the kernel's k step)
  int bm, bn, bk;
};

// Tile and split-K overrides set by si_tune_gemm_plan (tests and tile
// sweeps); -1 / 0 = automatic choice.
std::atomic<int> g_forced_kind{-1};
std::atomic<int> g_forced_splits{0};
int forced_kind() { return g_forced_kind.load(std::memory_order_relaxed); }
int forced_splits() { return g_forced_splits.load(std::memory_order_relaxed); }

// Tile and split-K choice for 16 < M <= 128 with K % 128 == 0 (and up to
// M = 512 where the larger tiles would leave most CUs idle), where each CU
// holds at most one block and a block's time is set by how fast its CU can
// pull A and B rows out of L2 (about 63 GB/s per CU with 4 waves), plus a
// fixed 6.7 us per wave of blocks; split K adds the int32 partial round trip
// through gemm_finalize (2 us + bytes at ~4 TB/s). Fitted on 4096 x 11008,
// 11008 x 4096 and 4096 x 22016 at M = 24..192, where it reproduces the
// measured times within ~10%. Returns the kind and sets *splits.
int choose_fill(int64_t M, int64_t N, int64_t K, int* splits) {
  struct Cand { int kind, bm, bn; };
  const Cand cands[3] = {{K_DMA_64x64, 64, 64}, {K_DMA_64x128, 64, 128},
                         {K_DMA8_128x128_24, 128, 128}};
  const int64_t kt = K / 128;
  double best = 0.0;
  int kind = K_DMA8_128x128_24;
  *splits = 1;
  for (const Cand& c : cands) {
    for (int s = 1; s <= 8; s *= 2) {
      if (s > 1 && kt / s < 16) break;  // shorter K loops lose more than the model says
      const int64_t per = ceil_div(kt, s);
      const int64_t blocks = ceil_div(M, c.bm) * ceil_div(N, c.bn) * ceil_div(kt, per);
      double t = (double)ceil_div(blocks, 256) *
                 (6.7 + 15.9e-6 * (double)(c.bm + c.bn) * (double)(per * 128));
      if (s > 1) t += 2.0 + (double)(s + 1) * (double)M * (double)N * 4.0 / 4.0e6;
      if (best == 0.0 || t < best * (1.0 - 1e-9)) { best = t; kind = c.kind; *splits = s; }
    }
  }
  return kind;
}

Plan choose(int64_t M, int64_t N, int64_t K) {
  Plan p{K_SCALAR, 0, 1, (int)K, 0, 0, 0};
  const bool big = M >= ((int64_t)1 << 31) || N >= ((int64_t)1 << 31) || K >= ((int64_t)1 << 31);
  if (K % 16 != 0 || M == 0 || N == 0 || big) return p;
  int kind;
  int fill_splits = 0;
  const int64_t rows_per_cu = ceil_div(N, 256);
  if (forced_kind() >= 0) {
    kind = forced_kind();
  } else if (K % 256 == 0 && rows_per_cu >= 16 && rows_per_cu <= 48 &&
             (M <= 32 || (M <= 128 && rows_per_cu >= 17))) {
    // Each CU streams its own ceil(N / 256) weight rows once: 11008 x 4096 at
    // M = 16 / 32: 14.1 / 14.7 -> 10.2 / 11.3 us; 4096 x 11008: 14.0 / 15.0 ->
    // 13.6 / 14.5 us. With 17-48 rows per CU this beats the 64-row tiles up to
    // M = 128 (4096 -> 11008 at M = 40 / 64 / 96 / 128: 13.5 / 14.5 / 17.2 /
    // 18.9 -> 11.1 / 13.2 / 16.1 / 18.7 us; 4096 -> 8192 at M = 64: 11.4 -> 9.6
    // us); with 16 rows per CU (N = 4096) the activation rows outweigh the
    // weight's from M = 33 (M = 96: 18.5 against 23.7 us for the tiles).
    kind = K_ROWS;
  } else if (K % 128 == 0 && M <= 128 &&
             (M > 16 || (M > 8 && ceil_div(N, 64) >= 128 && ceil_div(N, 64) < 256))) {
    // From 9 rows, where the stream kernel would use 64-column blocks (128..255
    // of them), 64x64 tiles are faster: 16 x 11008 x 4096 14.2 -> 13.1 us. With
    // 16- or 32-column stream blocks (other N) streaming stays ahead to M = 16.
    kind = choose_fill(M, N, K, &fill_splits);
  } else if (M <= 32 && K % 64 == 0) {
    // Weight streaming; the column width per block sets how many CUs stream.
    // M = 16: N = 11008 -> 64 columns (172 blocks, 12 us); N = 4096 -> 16
    // columns, 8 waves (256 blocks: 12 us, 26.5 us with 64 columns); N = 22016
    // -> 32 columns (688 blocks: 23.5 us, 27 us with 64).
    const int64_t b64 = ceil_div(N, 64);
    kind = b64 < 128 ? K_STREAM_N16_W8 : (b64 < 256 ? K_STREAM_N64 : K_STREAM_N32);
  } else if (K % 128 == 0) {
    // One tile per CU per wave of tiles. Estimated time = waves of 256 tiles
    // x (tile area / the tile's measured speed relative to 256x256); the
    // smallest wins. 4096 x 11008: M = 129..256 -> 128x96 (230 tiles; M = 256:
    // 23.8 -> 22.0 us against 128x128), M = 384..512 -> 256x128, M = 640 ->
    // 128x128, M = 1024 -> 256x192; 2048 x 22016 x 4096 -> 256x256 (k step
    // 128: 206 -> 199 us against 64); 2048 x 4096 x 11008 -> 256x128. The
    // 128x96 tile only up to 256 rows and where its grid is one wave filling
    // at least 192 CUs, as measured (at M = 320 its two waves lose to 256x128,
    // 37 against 34 us; grids filling fewer CUs belong to the fill model).
    struct Cand { int kind, bm, bn; double speed; bool one_wave; };
    const Cand cands[5] = {{K_DMA8_256x192_K128, 256, 192, 0.91, false},
                           {K_DMA8_256x256_K128, 256, 256, 1.0, false},
                           {K_DMA_256x128_K128, 256, 128, 0.81, false},
                           {K_DMA8_128x128_24, 128, 128, 0.78, false},
                           {K_DMA_128x96, 128, 96, 0.63, true}};
    double best = 0.0;
    int64_t best_tiles = 0;
    kind = K_DMA8_256x192_K128;
    for (const Cand& c : cands) {
      const int64_t tiles = ceil_div(M, c.bm) * ceil_div(N, c.bn);
      if (c.one_wave && (tiles > 256 || tiles < 192 || M > 256)) continue;
      const double t = (double)ceil_div(tiles, 256) * c.bm * c.bn / c.speed;
      if (best == 0.0 || t < best * (1.0 - 1e-9)) { best = t; kind = c.kind; best_tiles = tiles; }
    }
    // A grid that leaves over half the CUs idle (the 4096-column down
    // projection: 64-128 tiles up to M = 512) goes to the fill model, which
    // splits K: 256 x 4096 x 11008 52.3 -> 28.1 us, 512 rows 51.5 -> 41.7 us.
    if (best_tiles <= 128 && M <= 512) kind = choose_fill(M, N, K, &fill_splits);
  } else if (K % 64 == 0) {
    kind = K_DMA_256x192;
  } else {
    kind = K_TILE_128x128;
  }
  if (kind == K_ROWS) {
    if (K % 256 == 0 && rows_per_cu <= 48 && (M <= 32 || (M <= 128 && rows_per_cu >= 17))) {
      p.kind = K_ROWS;
      p.mf = (int)ceil_div(M, 16);
      p.bn = (int)(ceil_div(rows_per_cu, 4) * 4);  // whole 4-column output pieces per block
      return p;
    }
    kind = K_TILE_128x128;
  }
  if (kind == K_SKINNY) {
    if (M > 64 || K % 64 != 0) kind = K_TILE_128x128;
  }
  if (kind == K_STREAM_N64 || kind == K_STREAM_N64_W8 || kind == K_STREAM_N32 ||
      kind == K_STREAM_N16 || kind == K_STREAM_N32_W8 || kind == K_STREAM_N16_W8) {
    if (M > 64 || K % 64 != 0) {
      kind = K_TILE_128x128;
    } else {
      p.kind = kind;
      p.mf = (int)ceil_div(M, 16);
      return p;
    }
  }
  p.kind = kind;
  if (kind == K_SKINNY) {
    p.mf = (int)ceil_div(M, 16);
    const int64_t waves = ceil_div(N, 16);
    const int64_t ksteps = K / 64;
    int splits = 1;
    // enough wavefronts to stream the weight (~8 per SIMD), >= 8 k steps each
    while (waves * splits < 8192 && ksteps / (splits * 2) >= 8) splits *= 2;
    p.splits = splits;
    p.k_split = (int)(ceil_div(ksteps, splits) * 64);
    p.splits = (int)ceil_div(K, p.k_split);
    return p;
  }
  switch (kind) {
    case K_DMA_256x256: p.bm = 256; p.bn = 256; p.bk = 64; break;
    case K_DMA_128x256: p.bm = 128; p.bn = 256; p.bk = 64; break;
    case K_DMA_256x128: p.bm = 256; p.bn = 128; p.bk = 64; break;
    case K_DMA_128x128: p.bm = 128; p.bn = 128; p.bk = 128; break;
    case K_DMA_256x192: p.bm = 256; p.bn = 192; p.bk = 64; break;
    case K_DMA_256x64: p.bm = 256; p.bn = 64; p.bk = 128; break;
    case K_DMA_256x128_K128: p.bm = 256; p.bn = 128; p.bk = 128; break;
    case K_DMA8_256x256: p.bm = 256; p.bn = 256; p.bk = 64; break;
    case K_DMA8_256x256_K128: p.bm = 256; p.bn = 256; p.bk = 128; break;
    case K_DMA8_256x192_K128: p.bm = 256; p.bn = 192; p.bk = 128; break;
    case K_DMA8_256x128: p.bm = 256; p.bn = 128; p.bk = 64; break;
    case K_DMA8_128x256: p.bm = 128; p.bn = 256; p.bk = 64; break;
    case K_DMA8_128x128_42: p.bm = 128; p.bn = 128; p.bk = 128; break;
    case K_DMA8_128x128_24: p.bm = 128; p.bn = 128; p.bk = 128; break;
    case K_DMA_64x64: p.bm = 64; p.bn = 64; p.bk = 128; break;
    case K_DMA_64x128: p.bm = 64; p.bn = 128; p.bk = 128; break;
    case K_DMA_128x96: p.bm = 128; p.bn = 96; p.bk = 128; break;
    default: p.kind = K_TILE_128x128; p.bm = 128; p.bn = 128; p.bk = 128; break;
  }
  if (K % p.bk != 0 && p.bk == 128 && K % 64 == 0 && p.kind != K_TILE_128x128) {
    p.kind = K_DMA_256x128;  // same family, k step 64
    p.bm = 256; p.bn = 128; p.bk = 64;
  }
  if (K % p.bk != 0) {  // fall back to a k step that divides K
    p.kind = K_TILE_128x128;
    p.bm = 128; p.bn = 128; p.bk = K % 128 == 0 ? 128 : 32;
    if (K % 32 != 0) { p.kind = K_SCALAR; return p; }
  }
  // gemm_dma addresses each operand with 32-bit byte offsets.
  if (p.kind != K_TILE_128x128 && (M * K >= ((int64_t)1 << 31) || N * K >= ((int64_t)1 << 31))) {
    p.kind = K_TILE_128x128;
    p.bm = 128; p.bn = 128; p.bk = K % 128 == 0 ? 128 : 32;
    if (K % 32 != 0) { p.kind = K_SCALAR; return p; }
  }
  p.splits = 1;
  p.k_split = (int)K;
  int want = forced_splits();
  if (want <= 0 && fill_splits > 0) want = fill_splits;
  if (want > 1 && p.kind != K_TILE_128x128) {
    const int64_t kt = K / p.bk;
    const int64_t per = ceil_div(kt, want);
    p.k_split = (int)(per * p.bk);
    p.splits = (int)ceil_div(kt, per);
  }
  return p;
}

size_t workspace_for(int64_t M, int64_t N, int64_t K) {
  const Plan p = choose(M, N, K);
  return p.splits > 1 ? (size_t)p.splits * (size_t)M * (size_t)N * sizeof(int32_t) : 0;
}

template <int EPI>
void launch_tile(const Plan& p, const int8_t* a, const int8_t* b, int M, int N, int K, int32_t* c,
                 const EpiArgs& ep, hipStream_t st) {
  const dim3 block(256);
  if (p.kind == K_TILE_128x128) {
    const dim3 grid((unsigned)ceil_div(N, p.bn), (unsigned)ceil_div(M, p.bm), (unsigned)p.splits);
    if (p.bk == 32) gemm_tile<128, 128, 32, 2, 2, EPI><<<grid, block, 0, st>>>(a, b, M, N, K, p.k_split, c, ep);
    else gemm_tile<128, 128, 128, 2, 2, EPI><<<grid, block, 0, st>>>(a, b, M, N, K, p.k_split, c, ep);
    return;
  }
  // DMA kernels: one linear grid dimension over the tiles (renumbered per XCD
  // inside the kernel), splits in z.
  const dim3 grid((unsigned)(ceil_div(M, p.bm) * ceil_div(N, p.bn)), 1, (unsigned)p.splits);
#define SI_DMA(BM_, BN_, BK_, WM_, WN_, S_) SI_DMA2(BM_, BN_, BK_, WM_, WN_, S_, S_)
#define SI_DMA2(BM_, BN_, BK_, WM_, WN_, RA_, RB_)                                                \
  gemm_dma<BM_, BN_, BK_, WM_, WN_, RA_, RB_, EPI><<<grid, dim3(64 * WM_ * WN_), 0, st>>>( \
      a, b, M, N, K, p.k_split, c, ep)
  switch (p.kind) {
    case K_DMA_256x256: SI_DMA(256, 256, 64, 2, 2, 4); break;
    case K_DMA_128x256: SI_DMA(128, 256, 64, 2, 2, 4); break;
    case K_DMA_256x128: SI_DMA(256, 128, 64, 2, 2, 4); break;
    case K_DMA_128x128: SI_DMA(128, 128, 128, 2, 2, 4); break;
    case K_DMA_256x192: SI_DMA(256, 192, 64, 2, 2, 4); break;
    case K_DMA_256x64: SI_DMA(256, 64, 128, 4, 1, 3); break;
    case K_DMA_256x128_K128: SI_DMA2(256, 128, 128, 2, 2, 2, 6); break;
    case K_DMA8_256x256: SI_DMA(256, 256, 64, 4, 2, 4); break;
    case K_DMA8_256x256_K128: SI_DMA2(256, 256, 128, 4, 2, 2, 3); break;
    case K_DMA8_256x192_K128: SI_DMA2(256, 192, 128, 4, 2, 2, 4); break;
    case K_DMA8_256x128: SI_DMA(256, 128, 64, 4, 2, 4); break;
    case K_DMA8_128x128_42: SI_DMA(128, 128, 128, 4, 2, 4); break;
    case K_DMA8_128x128_24: SI_DMA(128, 128, 128, 2, 4, 4); break;
    case K_DMA_64x64: SI_DMA(64, 64, 128, 2, 2, 4); break;
    case K_DMA_64x128: SI_DMA(64, 128, 128, 2, 2, 4); break;
    case K_DMA_128x96: SI_DMA(128, 96, 128, 4, 1, 4); break;
    default: SI_DMA(128, 256, 64, 2, 4, 4); break;
  }
#undef SI_DMA
#undef SI_DMA2
}

template <int MF, int EPI>
void launch_stream(const Plan& p, const int8_t* a, const int8_t* b, int M, int N, int K, int32_t* c,
                   const EpiArgs& ep, hipStream_t st) {
#define SI_STREAM(NF_, NW_, U_)                                                           \
  gemm_stream<MF, NF_, NW_, U_, EPI><<<dim3((unsigned)ceil_div(N, 16 * NF_)), dim3(64 * NW_), 0, st>>>( \
      a, b, M, N, K, c, ep)
  switch (p.kind) {
    case K_STREAM_N64_W8: SI_STREAM(4, 8, 2); break;
    case K_STREAM_N32: SI_STREAM(2, 4, 4); break;
    case K_STREAM_N16: SI_STREAM(1, 4, 4); break;
    case K_STREAM_N32_W8: SI_STREAM(2, 8, 2); break;
    case K_STREAM_N16_W8: SI_STREAM(1, 8, 2); break;
    default: SI_STREAM(4, 4, 4);
  }
#undef SI_STREAM
}

template <int MF, int EPI>
void launch_rows(const Plan& p, const int8_t* a, const int8_t* b, int M, int N, int K, int32_t* c,
                 const EpiArgs& ep, hipStream_t st) {
  const dim3 grid((unsigned)ceil_div(N, p.bn));
  const int G = (p.bn + 15) / 16;
  // 16-row stages are small (8-12 KB): six of them keep about as many bytes in
  // flight as four of the 48-row stages (16 x 4096 x 11008: 12.9 -> 11.8 us,
  // 32 rows 13.6 -> 13.1 us). 16 weight rows per CU only up to 32 activation
  // rows (choose); wider stages take four slots, or three where four would not
  // fit in 160 KB of LDS.
  if constexpr (MF <= 2) {
    if (G == 1) {
      gemm_rows<MF, 1, 6, EPI><<<grid, 256, 0, st>>>(a, b, M, N, K, p.bn, c, ep);
      return;
    }
  }
  constexpr int R2 = 16 * (2 + MF) * 256 * 4 <= 160 * 1024 ? 4 : 3;
  constexpr int R3 = 16 * (3 + MF) * 256 * 4 <= 160 * 1024 ? 4 : 3;
  if (G <= 2) gemm_rows<MF, 2, R2, EPI><<<grid, 256, 0, st>>>(a, b, M, N, K, p.bn, c, ep);
  else gemm_rows<MF, 3, R3, EPI><<<grid, 256, 0, st>>>(a, b, M, N, K, p.bn, c, ep);
}

template <int EPI>
void launch(const Plan& p, const int8_t* a, const int8_t* b, int M, int N, int K, int32_t* c,
            const EpiArgs& ep, hipStream_t st) {
  const dim3 block(256);
  if (p.kind == K_ROWS) {
    switch (p.mf) {
      case 1: launch_rows<1, EPI>(p, a, b, M, N, K, c, ep, st); break;
      case 2: launch_rows<2, EPI>(p, a, b, M, N, K, c, ep, st); break;
      case 3: launch_rows<3, EPI>(p, a, b, M, N, K, c, ep, st); break;
      case 4: launch_rows<4, EPI>(p, a, b, M, N, K, c, ep, st); break;
      case 5: launch_rows<5, EPI>(p, a, b, M, N, K, c, ep, st); break;
      case 6: launch_rows<6, EPI>(p, a, b, M, N, K, c, ep, st); break;
      case 7: launch_rows<7, EPI>(p, a, b, M, N, K, c, ep, st); break;
      default: launch_rows<8, EPI>(p, a, b, M, N, K, c, ep, st);
    }
    return;
  }
  if (p.kind == K_STREAM_N64 || p.kind == K_STREAM_N64_W8 || p.kind == K_STREAM_N32 ||
      p.kind == K_STREAM_N16 || p.kind == K_STREAM_N32_W8 || p.kind == K_STREAM_N16_W8) {
    switch (p.mf) {
      case 1: launch_stream<1, EPI>(p, a, b, M, N, K, c, ep, st); break;
      case 2: launch_stream<2, EPI>(p, a, b, M, N, K, c, ep, st); break;
      case 3: launch_stream<3, EPI>(p, a, b, M, N, K, c, ep, st); break;
      default: launch_stream<4, EPI>(p, a, b, M, N, K, c, ep, st);
    }
    return;
  }
  if (p.kind == K_SKINNY) {
    const dim3 grid((unsigned)ceil_div(ceil_div(N, 16), 4), (unsigned)p.splits);
    switch (p.mf) {
      case 1: gemm_skinny<1, EPI><<<grid, block, 0, st>>>(a, b, M, N, K, p.k_split, c, ep); break;
      case 2: gemm_skinny<2, EPI><<<grid, block, 0, st>>>(a, b, M, N, K, p.k_split, c, ep); break;
      case 3: gemm_skinny<3, EPI><<<grid, block, 0, st>>>(a, b, M, N, K, p.k_split, c, ep); break;
      default: gemm_skinny<4, EPI><<<grid, block, 0, st>>>(a, b, M, N, K, p.k_split, c, ep);
    }
    return;
  }
  if (EPI != EPI_DEQUANT) {
    launch_tile<EPI>(p, a, b, M, N, K, c, ep, st);
  } else if (ep.resid != nullptr) {
    if (ep.out_dtype == SI_DT_F32)
      launch_tile<EPI_DEQUANT + 16 * SI_DT_F32 + EPI_RESID>(p, a, b, M, N, K, c, ep, st);
    else if (ep.out_dtype == SI_DT_F16)
      launch_tile<EPI_DEQUANT + 16 * SI_DT_F16 + EPI_RESID>(p, a, b, M, N, K, c, ep, st);
    else
      launch_tile<EPI_DEQUANT + 16 * SI_DT_BF16 + EPI_RESID>(p, a, b, M, N, K, c, ep, st);
  } else if (ep.out_dtype == SI_DT_F32) {
    launch_tile<EPI_DEQUANT + 16 * SI_DT_F32>(p, a, b, M, N, K, c, ep, st);
  } else if (ep.out_dtype == SI_DT_F16) {
    launch_tile<EPI_DEQUANT + 16 * SI_DT_F16>(p, a, b, M, N, K, c, ep, st);
  } else {
    launch_tile<EPI_DEQUANT + 16 * SI_DT_BF16>(p, a, b, M, N, K, c, ep, st);
  }
}

int run_gemm(const int8_t* a, const int8_t* b, int64_t M, int64_t N, int64_t K, int32_t* c,
             EpiArgs ep, bool dequant, void* ws, size_t ws_bytes, hipStream_t st, const char* who) {
  if (M == 0 || N == 0) return SI_OK;
  const Plan p = choose(M, N, K);
  {
    uintptr_t bits = reinterpret_cast<uintptr_t>(c) | reinterpret_cast<uintptr_t>(ep.out) |
                     reinterpret_cast<uintptr_t>(ep.sw) | reinterpret_cast<uintptr_t>(ep.bias) |
                     reinterpret_cast<uintptr_t>(ep.resid) | reinterpret_cast<uintptr_t>(ws);
    // The int32 epilogues' device-scope buffer stores address a band of at
    // most 128 output rows by a 32-bit byte offset (< 512 N): wider outputs
    // take the per-element stores.
    ep.vec = (N % 8 == 0 && (bits & 15) == 0 && N < ((int64_t)1 << 22)) ? 1 : 0;
  }
  if (p.kind == K_SCALAR) {
    const int64_t blocks = std::min<int64_t>(ceil_div(M * N, 256), 65536);
    gemm_i8_scalar<<<(unsigned)blocks, 256, 0, st>>>(a, b, M, N, K, c, ep, dequant ? 1 : 0);
    return check_launch(who);
  }
  if (ceil_div(M, p.bm > 0 ? p.bm : 1) >= 65536 || p.splits >= 65536) {
    set_error("%s: shape too large", who);
    return SI_ERR_INVALID;
  }
  const int Mi = (int)M, Ni = (int)N, Ki = (int)K;
  if (p.splits == 1) {
    if (dequant) launch<EPI_DEQUANT>(p, a, b, Mi, Ni, Ki, c, ep, st);
    else launch<EPI_I32>(p, a, b, Mi, Ni, Ki, c, ep, st);
    return check_launch(who);
  }
  const size_t need = workspace_for(M, N, K);
  if (ws == nullptr || ws_bytes < need) {
    set_error("%s: workspace too small (%zu < %zu bytes)", who, ws_bytes, need);
    return SI_ERR_INVALID;
  }
  ep.partial = reinterpret_cast<int32_t*>(ws);
  launch<EPI_PARTIAL>(p, a, b, Mi, Ni, Ki, c, ep, st);
  if (int rc = check_launch(who)) return rc;
  const int64_t blocks = std::min<int64_t>(ceil_div(M * N, 256), 65536);
  gemm_finalize<<<(unsigned)blocks, 256, 0, st>>>(ep.partial, p.splits, M, N, c, ep,
                                                 dequant ? 1 : 0);
  return check_launch(who);
}

}  // namespace
}  // namespace si

using namespace si;

extern "C" void si_tune_gemm_plan(int kind, int splits) {
  g_forced_kind.store(kind < 0 ? -1 : kind, std::memory_order_relaxed);
  g_forced_splits.store(splits > 0 ? splits : 0, std::memory_order_relaxed);
}

extern "C" size_t si_gemm_workspace_bytes(int64_t M, int64_t N, int64_t K) {
  if (M <= 0 || N <= 0 || K <= 0) return 0;
  return workspace_for(M, N, K);
}

extern "C" int si_gemm_i8i8_i32(const int8_t* a, const int8_t* b, int64_t M, int64_t N, int64_t K,
                                int32_t* c, void* workspace, size_t workspace_bytes,
                                si_stream_t stream) {
  clear_error();
  SI_CHECK_ARG(M >= 0 && N >= 0 && K > 0, "si_gemm_i8i8_i32: bad shape");
  if (M == 0 || N == 0) return SI_OK;
  SI_CHECK_ARG(a && b && c, "si_gemm_i8i8_i32: NULL argument");
  SI_CHECK_ARG(((reinterpret_cast<uintptr_t>(a) | reinterpret_cast<uintptr_t>(b)) & 15) == 0,
               "si_gemm_i8i8_i32: operands must be 16-byte aligned");
  EpiArgs ep{nullptr, nullptr, nullptr, nullptr, 0, nullptr};
  return run_gemm(a, b, M, N, K, c, ep, false, workspace, workspace_bytes, as_stream(stream),
                  "si_gemm_i8i8_i32");
}

namespace {
int gemm_dequant(const int8_t* a, const float* sx, const int8_t* b, const float* sw,
                 const float* bias, const void* resid, int64_t M, int64_t N, int64_t K, void* out,
                 int out_dtype, void* workspace, size_t workspace_bytes, si_stream_t stream,
                 const char* who) {
  SI_CHECK_ARG(dtype_ok(out_dtype), "%s: unsupported out dtype %d", who, out_dtype);
  SI_CHECK_ARG(M >= 0 && N >= 0 && K > 0, "%s: bad shape", who);
  if (M == 0 || N == 0) return SI_OK;
  SI_CHECK_ARG(a && sx && b && sw && out, "%s: NULL argument", who);
  SI_CHECK_ARG(((reinterpret_cast<uintptr_t>(a) | reinterpret_cast<uintptr_t>(b)) & 15) == 0,
               "%s: operands must be 16-byte aligned", who);
  EpiArgs ep{sx, sw, bias, out, out_dtype, nullptr, 0, resid};
  return run_gemm(a, b, M, N, K, nullptr, ep, true, workspace, workspace_bytes,
                  as_stream(stream), who);
}
}  // namespace

extern "C" int si_gemm_i8_dequant(const int8_t* a, const float* sx, const int8_t* b,
                                  const float* sw, const float* bias, int64_t M, int64_t N,
                                  int64_t K, void* out, int out_dtype, void* workspace,
                                  size_t workspace_bytes, si_stream_t stream) {
  clear_error();
  return gemm_dequant(a, sx, b, sw, bias, nullptr, M, N, K, out, out_dtype, workspace,
                      workspace_bytes, stream, "si_gemm_i8_dequant");
}

extern "C" int si_gemm_i8_dequant_add(const int8_t* a, const float* sx, const int8_t* b,
                                      const float* sw, const float* bias, const void* residual,
                                      int64_t M, int64_t N, int64_t K, void* out, int out_dtype,
                                      void* workspace, size_t workspace_bytes,
                                      si_stream_t stream) {
  clear_error();
  SI_CHECK_ARG(residual != nullptr || M == 0 || N == 0, "si_gemm_i8_dequant_add: NULL residual");
  return gemm_dequant(a, sx, b, sw, bias, residual, M, N, K, out, out_dtype, workspace,
                      workspace_bytes, stream, "si_gemm_i8_dequant_add");
}

extern "C" size_t si_int8_linear_workspace_bytes(int64_t M, int64_t K, int64_t N) {
  if (M <= 0 || K <= 0 || N <= 0) return 0;
  const size_t q = ((size_t)M * (size_t)K + 255) & ~(size_t)255;
  const size_t s = ((size_t)M * sizeof(float) + 255) & ~(size_t)255;
  return q + s + workspace_for(M, N, K);
}

extern "C" int si_int8_linear_forward(const void* x, int dtype, int64_t M, int64_t K, int64_t N,
                                      const int8_t* qweight, const float* sw, const float* bias,
                                      void* out, void* workspace, size_t workspace_bytes,
                                      si_stream_t stream) {
  clear_error();
  SI_CHECK_ARG(dtype_ok(dtype), "si_int8_linear_forward: unsupported dtype %d", dtype);
  SI_CHECK_ARG(M >= 0 && K > 0 && N > 0, "si_int8_linear_forward: bad shape");
  if (M == 0) return SI_OK;
  SI_CHECK_ARG(x && qweight && sw && out, "si_int8_linear_forward: NULL argument");
  const size_t need = si_int8_linear_workspace_bytes(M, K, N);
  SI_CHECK_ARG(workspace != nullptr && workspace_bytes >= need,
               "si_int8_linear_forward: workspace too small (%zu < %zu bytes)", workspace_bytes,
               need);
  int8_t* q = reinterpret_cast<int8_t*>(workspace);
  const size_t qbytes = ((size_t)M * (size_t)K + 255) & ~(size_t)255;
  float* sx = reinterpret_cast<float*>(reinterpret_cast<char*>(workspace) + qbytes);
  const size_t sbytes = ((size_t)M * sizeof(float) + 255) & ~(size_t)255;
  void* gws = reinterpret_cast<char*>(workspace) + qbytes + sbytes;
  if (int rc = si_act_quant_i8(x, dtype, M, K, q, sx, stream)) return rc;
  return si_gemm_i8_dequant(q, sx, qweight, sw, bias, M, N, K, out, dtype, gws,
                            workspace_bytes - qbytes - sbytes, stream);
}

extern "C" int si_int8_linear_forward_add(const void* x, int dtype, int64_t M, int64_t K, int64_t N,
                                          const int8_t* qweight, const float* sw,
                                          const float* bias, const void* residual, void* out,
                                          void* workspace, size_t workspace_bytes,
                                          si_stream_t stream) {
  clear_error();
  SI_CHECK_ARG(dtype_ok(dtype), "si_int8_linear_forward_add: unsupported dtype %d", dtype);
  SI_CHECK_ARG(M >= 0 && K > 0 && N > 0, "si_int8_linear_forward_add: bad shape");
  if (M == 0) return SI_OK;
  SI_CHECK_ARG(x && qweight && sw && out && residual, "si_int8_linear_forward_add: NULL argument");
  const size_t need = si_int8_linear_workspace_bytes(M, K, N);
  SI_CHECK_ARG(workspace != nullptr && workspace_bytes >= need,
               "si_int8_linear_forward_add: workspace too small (%zu < %zu bytes)",
               workspace_bytes, need);
  int8_t* q = reinterpret_cast<int8_t*>(workspace);
  const size_t qbytes = ((size_t)M * (size_t)K + 255) & ~(size_t)255;
  float* sx = reinterpret_cast<float*>(reinterpret_cast<char*>(workspace) + qbytes);
  const size_t sbytes = ((size_t)M * sizeof(float) + 255) & ~(size_t)255;
  void* gws = reinterpret_cast<char*>(workspace) + qbytes + sbytes;
  if (int rc = si_act_quant_i8(x, dtype, M, K, q, sx, stream)) return rc;
  return gemm_dequant(q, sx, qweight, sw, bias, residual, M, N, K, out, dtype, gws,
                      workspace_bytes - qbytes - sbytes, stream, "si_int8_linear_forward_add");
}

// ---------------------------------------------------------------------------
// si_int8_linear_forward_noalloc: si_int8_linear_forward with its workspace
// (quantized activations, their scales, split-K partials) in `scratch`, a
// file-scope device array, instead of caller memory, for callers that cannot
// allocate. Every device holds its own copy until the process ends. The host
// never passes the array's name to a kernel: it looks the array's device
// address up once per device (hipGetSymbolAddress, with that device current)
// and uses that address. No entry here allocates device memory.
// ---------------------------------------------------------------------------
namespace si {
namespace {

constexpr size_t kScratchBytes = SI_INT8_LINEAR_SCRATCH_BYTES;
static __device__ __align__(256) unsigned char scratch[kScratchBytes];

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch[kMaxDevices] = {};

// The current device's copy of `scratch`, or nullptr (error set).
void* scratch_here(const char* who) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess || dev < 0 || dev >= kMaxDevices) {
    set_error("%s: no usable current device (%s, device %d)", who, hipGetErrorString(e), dev);
    return nullptr;
  }
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_scratch[dev] == nullptr) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || p == nullptr) {
      set_error("%s: hipGetSymbolAddress of the scratch array failed on device %d: %s", who,
                dev, hipGetErrorString(e));
      return nullptr;
    }
    g_scratch[dev] = p;
  }
  return g_scratch[dev];
}

}  // namespace
}  // namespace si

extern "C" int si_int8_linear_forward_noalloc(const void* x, int dtype, int64_t M, int64_t K,
                                              int64_t N, const int8_t* qweight, const float* sw,
                                              const float* bias, void* out, si_stream_t stream) {
  clear_error();
  SI_CHECK_ARG(dtype_ok(dtype), "si_int8_linear_forward_noalloc: unsupported dtype %d", dtype);
  SI_CHECK_ARG(M >= 0 && K > 0 && N > 0, "si_int8_linear_forward_noalloc: bad shape");
  if (M == 0) return SI_OK;
  SI_CHECK_ARG(x && qweight && sw && out, "si_int8_linear_forward_noalloc: NULL argument");
  const size_t need = si_int8_linear_workspace_bytes(M, K, N);
  SI_CHECK_ARG(need <= kScratchBytes,
               "si_int8_linear_forward_noalloc: this shape needs %zu bytes of workspace, more "
               "than the %zu-byte scratch; use si_int8_linear_forward with a workspace",
               need, kScratchBytes);
  void* ws = scratch_here("si_int8_linear_forward_noalloc");
  if (ws == nullptr) return SI_ERR_HIP;
  return si_int8_linear_forward(x, dtype, M, K, N, qweight, sw, bias, out, ws, kScratchBytes,
                                stream);
}
