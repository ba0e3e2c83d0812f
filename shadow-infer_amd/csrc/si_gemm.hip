// int8 x int8 -> int32 GEMM on gfx950 MFMA (v_mfma_i32_16x16x64_i8) with the
// INT8Linear dequant epilogue (ffn_optimizer/int8_linear.py:102-115).
//
// Operands: A = quantized activations [M, K] (K contiguous), B = qweight
// [K, N] (N contiguous, the reference's stored layout). MFMA wants K-contiguous
// fragments for both operands, so the B tile is transposed while it is staged:
// each thread loads a 4(k) x 16(n) byte block with four 16-byte loads,
// transposes it in registers with byte permutes and writes 16 dwords of
// 4 consecutive k to the LDS tile Bs[n][k].
//
// Fragment layout of v_mfma_i32_16x16x64_i8: lane l holds row (l % 16) of A
// and column (l % 16) of B, each as 16 consecutive k values starting at
// 16 * (l / 16); the accumulator lane l holds C[4*(l/16) + r][l % 16], r < 4.
// The k order inside a fragment only has to agree between A and B, which it
// does by construction, so the int32 sum is exact for any order.
//
// Split-K: when the (M, N) tile grid alone cannot fill the 256 CUs, K is split
// over blockIdx.z; each split writes an int32 partial and a second kernel adds
// the partials (integer adds, so the result does not depend on the order) and
// applies the epilogue.
#include "si_common.h"

namespace si {
namespace {

typedef int v4i __attribute__((ext_vector_type(4)));

constexpr int BK = 64;         // k per staged tile = one MFMA k-step
constexpr int LDK = BK + 16;   // LDS row pitch in bytes (padding against bank conflicts)

enum Epi { EPI_I32 = 0, EPI_PARTIAL = 1, EPI_DEQUANT = 2 };

struct EpiArgs {
  const float* sx;
  const float* sw;
  const float* bias;
  void* out;
  int out_dtype;
  int32_t* partial;  // [splits, M, N] when EPI_PARTIAL
};

// out = T(float(acc) * (sx * sw) [+ bias]) with the reference's rounding order.
__device__ __forceinline__ void store_dequant(const EpiArgs& ep, int64_t idx, int32_t acc, float sx,
                                              float sw, float bias) {
  const float sc = sx * sw;
  float o = (float)acc * sc;
  if (ep.bias != nullptr) o = o + bias;
  store_any(ep.out, ep.out_dtype, idx, o);
}

// 4x4 byte transpose: in[r] holds bytes (k=r, n=0..3); out[c] holds (n=c, k=0..3).
__device__ __forceinline__ void transpose4x4(const uint32_t in[4], uint32_t out[4]) {
  // Interleave pairs of rows, then pairs of pairs (v_perm_b32 selects bytes of {a, b}).
  const uint32_t t01_lo = __builtin_amdgcn_perm(in[1], in[0], 0x05010400u);  // k0n0 k1n0 k0n1 k1n1
  const uint32_t t01_hi = __builtin_amdgcn_perm(in[1], in[0], 0x07030602u);  // k0n2 k1n2 k0n3 k1n3
  const uint32_t t23_lo = __builtin_amdgcn_perm(in[3], in[2], 0x05010400u);
  const uint32_t t23_hi = __builtin_amdgcn_perm(in[3], in[2], 0x07030602u);
  out[0] = __builtin_amdgcn_perm(t23_lo, t01_lo, 0x05040100u);  // n0: k0 k1 k2 k3
  out[1] = __builtin_amdgcn_perm(t23_lo, t01_lo, 0x07060302u);  // n1
  out[2] = __builtin_amdgcn_perm(t23_hi, t01_hi, 0x05040100u);  // n2
  out[3] = __builtin_amdgcn_perm(t23_hi, t01_hi, 0x07060302u);  // n3
}

// Requirements (checked on the host): K % 16 == 0, N % 16 == 0, k_split % BK == 0.
template <int BM, int BN, int WM, int WN, int EPI>
__global__ __launch_bounds__(256) void gemm_i8_mfma(const int8_t* __restrict__ A,
                                                   const int8_t* __restrict__ B, int64_t M,
                                                   int64_t N, int64_t K, int64_t k_split,
                                                   int32_t* __restrict__ C, EpiArgs ep) {
  static_assert(WM * WN == 4, "four waves per block");
  constexpr int TM = BM / WM;  // rows per wave
  constexpr int TN = BN / WN;  // cols per wave
  constexpr int FM = TM / 16;
  constexpr int FN = TN / 16;
  __shared__ __attribute__((aligned(16))) uint8_t As[BM * LDK];
  __shared__ __attribute__((aligned(16))) uint8_t Bs[BN * LDK];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int wm = wave / WN;
  const int wn = wave % WN;
  const int64_t m0 = (int64_t)blockIdx.y * BM;
  const int64_t n0 = (int64_t)blockIdx.x * BN;
  const int64_t kb = (int64_t)blockIdx.z * k_split;
  const int64_t ke = kb + k_split < K ? kb + k_split : K;

  v4i acc[FM][FN];
#pragma unroll
  for (int i = 0; i < FM; ++i)
#pragma unroll
    for (int j = 0; j < FN; ++j) acc[i][j] = v4i{0, 0, 0, 0};

  for (int64_t k0 = kb; k0 < ke; k0 += BK) {
    // ---- stage A: BM rows x 64 bytes, 16-byte vectors ----
    for (int i = tid; i < BM * 4; i += 256) {
      const int r = i >> 2;
      const int q = i & 3;
      const int64_t m = m0 + r;
      const int64_t k = k0 + q * 16;
      uint4 v = make_uint4(0, 0, 0, 0);
      if (m < M && k < ke) v = *reinterpret_cast<const uint4*>(A + m * K + k);
      *reinterpret_cast<uint4*>(As + r * LDK + q * 16) = v;
    }
    // ---- stage B: 64 x BN bytes as 4x16 blocks, transposed to Bs[n][k] ----
    for (int i = tid; i < 16 * (BN / 16); i += 256) {
      const int kq = i / (BN / 16);  // 0..15: 4-row group
      const int nq = i % (BN / 16);  // 16-column group
      const int64_t k = k0 + kq * 4;
      const int64_t n = n0 + nq * 16;
      uint4 rows[4];
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        rows[r] = make_uint4(0, 0, 0, 0);
        if (n < N && k + r < ke) rows[r] = *reinterpret_cast<const uint4*>(B + (k + r) * N + n);
      }
      const uint32_t* rw = reinterpret_cast<const uint32_t*>(rows);
#pragma unroll
      for (int c = 0; c < 4; ++c) {  // 4 columns per dword
        const uint32_t in[4] = {rw[0 * 4 + c], rw[1 * 4 + c], rw[2 * 4 + c], rw[3 * 4 + c]};
        uint32_t out[4];
        transpose4x4(in, out);
#pragma unroll
        for (int j = 0; j < 4; ++j)
          *reinterpret_cast<uint32_t*>(Bs + (nq * 16 + c * 4 + j) * LDK + kq * 4) = out[j];
      }
    }
    __syncthreads();
    // ---- MFMA ----
    v4i af[FM], bf[FN];
    const int fr = lane & 15;
    const int fk = (lane >> 4) * 16;
#pragma unroll
    for (int i = 0; i < FM; ++i)
      af[i] = *reinterpret_cast<const v4i*>(As + (wm * TM + i * 16 + fr) * LDK + fk);
#pragma unroll
    for (int j = 0; j < FN; ++j)
      bf[j] = *reinterpret_cast<const v4i*>(Bs + (wn * TN + j * 16 + fr) * LDK + fk);
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
      for (int j = 0; j < FN; ++j)
        acc[i][j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(af[i], bf[j], acc[i][j], 0, 0, 0);
    __syncthreads();
  }

  // ---- epilogue ----
  const int col = lane & 15;
  const int rq = (lane >> 4) * 4;
#pragma unroll
  for (int i = 0; i < FM; ++i) {
#pragma unroll
    for (int j = 0; j < FN; ++j) {
      const int64_t n = n0 + wn * TN + j * 16 + col;
      if (n >= N) continue;
      float sw = 0.0f, bias = 0.0f;
      if (EPI == EPI_DEQUANT) {
        sw = ep.sw[n];
        if (ep.bias != nullptr) bias = ep.bias[n];
      }
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int64_t m = m0 + wm * TM + i * 16 + rq + r;
        if (m >= M) continue;
        const int32_t v = acc[i][j][r];
        if (EPI == EPI_I32) {
          C[m * N + n] = v;
        } else if (EPI == EPI_PARTIAL) {
          ep.partial[((int64_t)blockIdx.z * M + m) * N + n] = v;
        } else {
          store_dequant(ep, m * N + n, v, ep.sx[m], sw, bias);
        }
      }
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

// Any-shape fallback (K or N not a multiple of 16): one thread per output.
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
    for (int64_t k = 0; k < K; ++k) acc += (int32_t)A[m * K + k] * (int32_t)B[k * N + n];
    if (!dequant) {
      C[i] = acc;
    } else {
      store_dequant(ep, i, acc, ep.sx[m], ep.sw[n], ep.bias != nullptr ? ep.bias[n] : 0.0f);
    }
  }
}

struct Plan {
  int kind;     // 0 scalar, 1: BM16, 2: BM64, 3: BM128
  int splits;
  int64_t k_split;
};

Plan choose(int64_t M, int64_t N, int64_t K) {
  Plan p{0, 1, K};
  if (K % 16 != 0 || N % 16 != 0 || M == 0) return p;
  int bm;
  if (M <= 16) { p.kind = 1; bm = 16; }
  else if (M <= 256) { p.kind = 2; bm = 64; }
  else { p.kind = 3; bm = 128; }
  const int64_t tiles = ceil_div(M, bm) * ceil_div(N, 128);
  const int64_t kt = ceil_div(K, BK);  // k tiles
  // Split K while the tile grid is small, each split keeps >= 4 k tiles, and
  // the partial sums (written and re-read, 8 bytes per output per split) stay
  // within a small fraction of the K*N weight bytes.
  int splits = 1;
  while (tiles * splits < 512 && splits < 8 && kt / (splits * 2) >= 4 &&
         (int64_t)(splits * 2) * M * 16 <= K)
    splits *= 2;
  p.splits = splits;
  p.k_split = ceil_div(kt, splits) * BK;
  p.splits = (int)ceil_div(K, p.k_split);
  return p;
}

size_t workspace_for(int64_t M, int64_t N, int64_t K) {
  const Plan p = choose(M, N, K);
  return p.splits > 1 ? (size_t)p.splits * (size_t)M * (size_t)N * sizeof(int32_t) : 0;
}

template <int EPI>
void launch_tiles(const Plan& p, const int8_t* a, const int8_t* b, int64_t M, int64_t N, int64_t K,
                  int32_t* c, const EpiArgs& ep, hipStream_t st) {
  dim3 block(256);
  switch (p.kind) {
    case 1: {
      dim3 grid((unsigned)ceil_div(N, 128), (unsigned)ceil_div(M, 16), (unsigned)p.splits);
      gemm_i8_mfma<16, 128, 1, 4, EPI><<<grid, block, 0, st>>>(a, b, M, N, K, p.k_split, c, ep);
      break;
    }
    case 2: {
      dim3 grid((unsigned)ceil_div(N, 128), (unsigned)ceil_div(M, 64), (unsigned)p.splits);
      gemm_i8_mfma<64, 128, 1, 4, EPI><<<grid, block, 0, st>>>(a, b, M, N, K, p.k_split, c, ep);
      break;
    }
    default: {
      dim3 grid((unsigned)ceil_div(N, 128), (unsigned)ceil_div(M, 128), (unsigned)p.splits);
      gemm_i8_mfma<128, 128, 2, 2, EPI><<<grid, block, 0, st>>>(a, b, M, N, K, p.k_split, c, ep);
    }
  }
}

int run_gemm(const int8_t* a, const int8_t* b, int64_t M, int64_t N, int64_t K, int32_t* c,
             EpiArgs ep, bool dequant, void* ws, size_t ws_bytes, hipStream_t st, const char* who) {
  if (M == 0 || N == 0) return SI_OK;
  const Plan p = choose(M, N, K);
  if (p.kind == 0) {
    const int64_t total = M * N;
    const int64_t blocks = std::min<int64_t>(ceil_div(total, 256), 65536);
    gemm_i8_scalar<<<(unsigned)blocks, 256, 0, st>>>(a, b, M, N, K, c, ep, dequant ? 1 : 0);
    return check_launch(who);
  }
  if (p.splits == 1) {
    if (dequant) launch_tiles<EPI_DEQUANT>(p, a, b, M, N, K, c, ep, st);
    else launch_tiles<EPI_I32>(p, a, b, M, N, K, c, ep, st);
    return check_launch(who);
  }
  const size_t need = workspace_for(M, N, K);
  if (ws == nullptr || ws_bytes < need) {
    set_error("%s: workspace too small (%zu < %zu bytes)", who, ws_bytes, need);
    return SI_ERR_INVALID;
  }
  ep.partial = reinterpret_cast<int32_t*>(ws);
  launch_tiles<EPI_PARTIAL>(p, a, b, M, N, K, c, ep, st);
  if (int rc = check_launch(who)) return rc;
  const int64_t blocks = std::min<int64_t>(ceil_div(M * N, 256), 65536);
  gemm_finalize<<<(unsigned)blocks, 256, 0, st>>>(ep.partial, p.splits, M, N, c, ep,
                                                 dequant ? 1 : 0);
  return check_launch(who);
}

}  // namespace
}  // namespace si

using namespace si;

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
  EpiArgs ep{nullptr, nullptr, nullptr, nullptr, 0, nullptr};
  return run_gemm(a, b, M, N, K, c, ep, false, workspace, workspace_bytes, as_stream(stream),
                  "si_gemm_i8i8_i32");
}

extern "C" int si_gemm_i8_dequant(const int8_t* a, const float* sx, const int8_t* b,
                                  const float* sw, const float* bias, int64_t M, int64_t N,
                                  int64_t K, void* out, int out_dtype, void* workspace,
                                  size_t workspace_bytes, si_stream_t stream) {
  clear_error();
  SI_CHECK_ARG(dtype_ok(out_dtype), "si_gemm_i8_dequant: unsupported out dtype %d", out_dtype);
  SI_CHECK_ARG(M >= 0 && N >= 0 && K > 0, "si_gemm_i8_dequant: bad shape");
  if (M == 0 || N == 0) return SI_OK;
  SI_CHECK_ARG(a && sx && b && sw && out, "si_gemm_i8_dequant: NULL argument");
  EpiArgs ep{sx, sw, bias, out, out_dtype, nullptr};
  return run_gemm(a, b, M, N, K, nullptr, ep, true, workspace, workspace_bytes,
                  as_stream(stream), "si_gemm_i8_dequant");
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
