// Device-side KV precision admission for gfx950: the rate-distortion
// sensitivity proxy and the closed-form budget solver of
// shadowinfer/shadowkv/rd_allocator.py (kv_sensitivity :47-61,
// predict_codes_bytes :173-188, admit_codes :190-318).
//
// admit_codes ranks eligible token-heads by ascending score (importance x
// sensitivity, stable on the token-major index), walks the ranking with
// prefix sums of the bytes each entry saves, and cuts at the first prefix
// that covers the excess over the budget (a partial downgrade for the entry
// at the cut), then optionally evicts a second prefix. Only the cut entry
// matters, so the device never sorts: a weighted radix select over the
// score keys (four 8-bit digits, most significant first) finds the key of
// the cut entry, a scan over the entries with that key (in index order, as a
// stable sort leaves them) finds the entry itself, and one pass rewrites the
// codes of everything ranked before it. Every step is an integer sum, so the
// cut is exact.
#include "si_common.h"

namespace si {
namespace {

constexpr int ADM_THREADS = 256;
constexpr int TIE_CHUNK = 2048;  // entries per block of the tie scan
constexpr int MODE_DOWN = 0;     // ladder downgrade (fp32 -> fp16 -> int8 -> int4)
constexpr int MODE_EVICT = 1;    // eviction of the remaining bytes

struct AdmCosts {
  long long cost[5];   // bytes of one token-head per code (K + V with scales)
  long long delta[3];  // cost[c] - cost[c + 1]
};

struct AdmState {
  unsigned long long pred[3];  // total bytes after prep, downgrade, eviction
  unsigned long long ncand;    // eligible entries
  unsigned long long evicted;  // entries newly evicted
  unsigned long long R;        // weight the cut still has to cover
  unsigned long long rem;      // excess left when the ranking reaches the cut entry
  long long budget;            // bytes allowed (may be negative)
  int use_budget;              // 0: no budget, nothing is admitted
  long long b_idx;             // flat index of the cut entry
  unsigned int prefix;         // key bits fixed so far; the cut key after four digits
  int active;                  // the current selection runs
  int all;                     // the whole ranking is inside the cut
  int bad;                     // codes outside 0..4 were seen
};

// Bytes an entry of code c frees when taken down the ladder to int4.
__device__ __forceinline__ long long ladder_savings(const AdmCosts& cs, int c) {
  long long s = 0;
  for (int x = c; x < 3; ++x) s += cs.delta[x];
  return c >= 0 ? s : 0;
}

__device__ __forceinline__ unsigned long long weight(const AdmCosts& cs, int mode, int c) {
  if (c < 0 || c > 4) return 0;
  return (unsigned long long)(mode == MODE_DOWN ? ladder_savings(cs, c) : cs.cost[c]);
}

// Order-preserving key of an fp32 score: ascending keys = ascending scores,
// -0 == +0, NaN above +inf (torch.argsort puts NaN last).
__device__ __forceinline__ unsigned int score_key(float x) {
  if (x != x) return 0xffffffffu;
  if (x == 0.0f) x = 0.0f;
  const unsigned int u = __float_as_uint(x);
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

template <typename T>
__device__ __forceinline__ T block_sum(T v, T* red) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  const int wave = threadIdx.x >> 6, nw = blockDim.x >> 6;
  __syncthreads();
  if ((threadIdx.x & 63) == 0) red[wave] = v;
  __syncthreads();
  T s = 0;
  for (int w = 0; w < nw; ++w) s += red[w];
  return s;
}

__global__ void adm_init(AdmState* st, unsigned long long* hist, long long budget, int use_budget) {
  for (int i = threadIdx.x; i < 256; i += blockDim.x) hist[i] = 0;
  if (threadIdx.x == 0) {
    st->pred[0] = st->pred[1] = st->pred[2] = 0;
    st->ncand = st->evicted = st->R = st->rem = 0;
    st->budget = budget;
    st->use_budget = use_budget;
    st->b_idx = -1;
    st->prefix = 0;
    st->active = st->all = st->bad = 0;
  }
}

// Copies the codes, sums their bytes, and computes each entry's score key and
// eligibility (not a sink token, not protected).
__global__ __launch_bounds__(ADM_THREADS) void adm_prep(
    const int8_t* __restrict__ codes_in, int8_t* __restrict__ codes, int64_t n, int64_t H,
    const float* __restrict__ imp, const float* __restrict__ sens,
    const uint8_t* __restrict__ prot, int64_t sink, AdmCosts cs, unsigned int* __restrict__ key,
    uint8_t* __restrict__ cand, AdmState* st) {
  __shared__ unsigned long long red[ADM_THREADS / 64];
  unsigned long long bytes = 0, nc = 0;
  int bad = 0;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
       i += (int64_t)gridDim.x * blockDim.x) {
    const int c = codes_in[i];
    codes[i] = (int8_t)c;
    if (c < 0 || c > 4) bad = 1;
    else bytes += (unsigned long long)cs.cost[c];
    const bool elig = i / H >= sink && !(prot != nullptr && prot[i] != 0);
    const float s = sens != nullptr ? imp[i] * sens[i] : imp[i];
    key[i] = score_key(s);
    cand[i] = elig ? 1 : 0;
    nc += elig ? 1 : 0;
  }
  bytes = block_sum(bytes, red);
  nc = block_sum(nc, red);
  const int any_bad = __syncthreads_or(bad);
  if (threadIdx.x == 0) {
    atomicAdd(&st->pred[0], bytes);
    atomicAdd(&st->ncand, nc);
    if (any_bad) atomicOr(&st->bad, 1);
  }
}

// Starts a selection: the downgrade cuts the excess of the initial bytes over
// the budget, the eviction the excess left after the downgrade.
__global__ void adm_sel_begin(AdmState* st, int mode, int allow_evict) {
  if (threadIdx.x != 0) return;
  const long long budget = st->budget;
  const long long p = (long long)(mode == MODE_DOWN ? st->pred[0] : st->pred[1]);
  int active = st->use_budget && st->ncand > 0 && st->bad == 0 && p > budget;
  if (mode == MODE_EVICT && !allow_evict) active = 0;
  st->active = active;
  st->all = 0;
  st->prefix = 0;
  st->b_idx = -1;
  st->rem = 0;
  st->R = active ? (unsigned long long)p - (unsigned long long)budget : 0;
}

// Weight histogram of one 8-bit key digit over the candidates whose higher
// digits equal the ones already fixed.
__global__ __launch_bounds__(ADM_THREADS) void adm_hist(
    int mode, int digit, const unsigned int* __restrict__ key, const uint8_t* __restrict__ cand,
    const int8_t* __restrict__ codes, int64_t n, AdmCosts cs, unsigned long long* __restrict__ hist,
    const AdmState* st) {
  if (!st->active || st->all) return;
  __shared__ unsigned long long lh[256];
  for (int b = threadIdx.x; b < 256; b += blockDim.x) lh[b] = 0;
  __syncthreads();
  const unsigned int prefix = st->prefix;
  const int sh = 8 * digit;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
       i += (int64_t)gridDim.x * blockDim.x) {
    if (!cand[i]) continue;
    const unsigned int k = key[i];
    if (digit < 3 && (k >> (sh + 8)) != prefix) continue;
    const unsigned long long w = weight(cs, mode, codes[i]);
    if (w != 0) atomicAdd(&lh[(k >> sh) & 255u], w);
  }
  __syncthreads();
  for (int b = threadIdx.x; b < 256; b += blockDim.x)
    if (lh[b] != 0) atomicAdd(&hist[b], lh[b]);
}

// Picks the digit whose bucket holds the cut (the first bucket where the
// running weight reaches R), and clears the histogram for the next digit.
// One block of 256 threads.
__global__ __launch_bounds__(256) void adm_pick(int digit, unsigned long long* hist, AdmState* st) {
  if (!st->active || st->all) return;
  __shared__ unsigned long long cum[256];
  const int b = threadIdx.x;
  cum[b] = hist[b];
  __syncthreads();
  for (int o = 1; o < 256; o <<= 1) {
    const unsigned long long add = b >= o ? cum[b - o] : 0;
    __syncthreads();
    cum[b] += add;
    __syncthreads();
  }
  hist[b] = 0;
  const unsigned long long R = st->R;
  if (digit == 3 && cum[255] < R) {  // every candidate together saves less than the excess
    if (b == 0) st->all = 1;
    return;
  }
  const unsigned long long before = b > 0 ? cum[b - 1] : 0;
  if (cum[b] >= R && before < R) {
    st->prefix = (st->prefix << 8) | (unsigned int)b;
    st->R = R - before;
  }
}

// Per-chunk weight of the candidates whose key equals the cut key.
__global__ __launch_bounds__(ADM_THREADS) void adm_tie_sum(
    int mode, const unsigned int* __restrict__ key, const uint8_t* __restrict__ cand,
    const int8_t* __restrict__ codes, int64_t n, AdmCosts cs, unsigned long long* __restrict__ blk,
    const AdmState* st) {
  if (!st->active || st->all) return;
  __shared__ unsigned long long red[ADM_THREADS / 64];
  const unsigned int tau = st->prefix;
  const int64_t base = (int64_t)blockIdx.x * TIE_CHUNK;
  unsigned long long s = 0;
  for (int64_t i = base + threadIdx.x; i < min(base + TIE_CHUNK, n); i += blockDim.x)
    if (cand[i] && key[i] == tau) s += weight(cs, mode, codes[i]);
  s = block_sum(s, red);
  if (threadIdx.x == 0) blk[blockIdx.x] = s;
}

// Inclusive scan of 1024 values held one per thread; returns this thread's sum.
__device__ __forceinline__ unsigned long long scan1024(unsigned long long v, unsigned long long* sh) {
  const int t = threadIdx.x;
  sh[t] = v;
  __syncthreads();
  for (int o = 1; o < 1024; o <<= 1) {
    const unsigned long long add = t >= o ? sh[t - o] : 0;
    __syncthreads();
    sh[t] += add;
    __syncthreads();
  }
  const unsigned long long r = sh[t];
  __syncthreads();
  return r;
}

// Finds the cut entry among the candidates with the cut key, in index order:
// the chunk whose running weight reaches R, then the entry inside it.
// One block of 1024 threads.
__global__ __launch_bounds__(1024) void adm_tie_pick(
    int mode, const unsigned int* __restrict__ key, const uint8_t* __restrict__ cand,
    const int8_t* __restrict__ codes, int64_t n, AdmCosts cs, const unsigned long long* __restrict__ blk,
    int64_t nblk, AdmState* st) {
  if (!st->active || st->all) return;
  __shared__ unsigned long long sh[1024];
  __shared__ long long found;
  __shared__ unsigned long long carry;
  const int t = threadIdx.x;
  const unsigned int tau = st->prefix;
  unsigned long long R = st->R;
  if (t == 0) { found = -1; carry = 0; }
  __syncthreads();
  // 1. the chunk
  for (int64_t c0 = 0; c0 < nblk; c0 += 1024) {
    const int64_t c = c0 + t;
    const unsigned long long v = c < nblk ? blk[c] : 0;
    const unsigned long long inc = scan1024(v, sh) + carry;
    const unsigned long long exc = inc - v;
    if (c < nblk && inc >= R && exc < R) found = c;
    __syncthreads();
    if (found >= 0) {
      if (c == found) { R -= exc; carry = R; }  // weight left inside the chunk
      break;
    }
    if (t == 1023) carry = inc;
    __syncthreads();
  }
  __syncthreads();
  if (found < 0) return;  // cannot happen: the digits guarantee enough weight
  R = carry;
  const int64_t base = found * TIE_CHUNK;
  // 2. the entry: two consecutive entries per thread keep index order
  const int64_t i0 = base + 2 * t;
  unsigned long long w0 = 0, w1 = 0;
  if (i0 < n && cand[i0] && key[i0] == tau) w0 = weight(cs, mode, codes[i0]);
  if (i0 + 1 < n && cand[i0 + 1] && key[i0 + 1] == tau) w1 = weight(cs, mode, codes[i0 + 1]);
  const unsigned long long inc = scan1024(w0 + w1, sh);
  const unsigned long long exc = inc - w0 - w1;
  if (exc < R && exc + w0 >= R) {
    st->b_idx = i0;
    st->rem = R - exc;
  } else if (exc + w0 < R && inc >= R) {
    st->b_idx = i0 + 1;
    st->rem = R - exc - w0;
  }
}

// Rewrites the codes of the candidates ranked before the cut (and the cut
// entry), then sums the new total bytes.
__global__ __launch_bounds__(ADM_THREADS) void adm_apply(
    int mode, const unsigned int* __restrict__ key, const uint8_t* __restrict__ cand,
    int8_t* __restrict__ codes, int64_t n, AdmCosts cs, AdmState* st, int slot) {
  __shared__ unsigned long long red[ADM_THREADS / 64];
  const int active = st->active;
  const int all = st->all;
  const unsigned int tau = st->prefix;
  const long long b_idx = st->b_idx;
  const long long rem = (long long)st->rem;
  unsigned long long bytes = 0, ev = 0;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
       i += (int64_t)gridDim.x * blockDim.x) {
    int c = codes[i];
    if (active && cand[i]) {
      const unsigned int k = key[i];
      const bool before = all || k < tau || (k == tau && i < b_idx);
      const bool at = !all && i == b_idx;
      const int c0 = c;
      if (mode == MODE_DOWN) {
        if (before) {
          if (c != 4) c = 3;
        } else if (at && c != 4) {
          const long long s1 = c < 3 ? cs.delta[c] : 0;
          const int n1 = c < 3 ? c + 1 : c;
          const long long s2 = n1 < 3 ? cs.delta[n1] : 0;
          const int n2 = n1 < 3 ? n1 + 1 : n1;
          c = rem <= s1 ? n1 : rem <= s1 + s2 ? n2 : 3;
        }
      } else if (before || at) {
        if (c != 4) ++ev;
        c = 4;
      }
      if (c != c0) codes[i] = (int8_t)c;
    }
    if (c >= 0 && c <= 4) bytes += (unsigned long long)cs.cost[c];
  }
  bytes = block_sum(bytes, red);
  ev = block_sum(ev, red);
  if (threadIdx.x == 0) {
    atomicAdd(&st->pred[slot], bytes);
    if (ev) atomicAdd(&st->evicted, ev);
  }
}

__global__ void adm_finish(const AdmState* st, int64_t* result) {
  if (threadIdx.x != 0) return;
  result[0] = (int64_t)st->pred[2];
  result[1] = (int64_t)st->evicted;
  result[2] = st->bad;
}

// ---- kv_sensitivity ----------------------------------------------------------

template <int DT>
__device__ __forceinline__ float round_dt(float x) {
  if constexpr (DT == SI_DT_F32) return x;
  else if constexpr (DT == SI_DT_F16) return f16_bits_to_f32(f32_to_f16_bits(x));
  else return bf16_bits_to_f32(f32_to_bf16_bits(x));
}

template <int DT>
__device__ __forceinline__ float elem(const void* p, int64_t i) {
  if constexpr (DT == SI_DT_F32) return reinterpret_cast<const float*>(p)[i];
  else if constexpr (DT == SI_DT_F16) return f16_bits_to_f32(reinterpret_cast<const uint16_t*>(p)[i]);
  else return bf16_bits_to_f32(reinterpret_cast<const uint16_t*>(p)[i]);
}

// amax with NaN propagation (torch's max reduction); m holds |x| so far.
__device__ __forceinline__ float amax_nan(float m, float x) {
  const float a = fabsf(x);
  return (a != a || m != m) ? __int_as_float(0x7fc00000) : fmaxf(m, a);
}

// 16 lanes per token-head (b rows of D values); a block covers 16 tokens of
// one head. VEC: 16-byte loads (D * elem_size a multiple of 16, aligned rows).
template <int DT, bool VEC>
__global__ __launch_bounds__(256) void kv_sens_kernel(const void* __restrict__ k,
                                                      const void* __restrict__ v, int64_t B,
                                                      int64_t H, int64_t S, int64_t D,
                                                      void* __restrict__ out) {
  constexpr int ES = DT == SI_DT_F32 ? 4 : 2;
  constexpr int VE = 16 / ES;  // elements per 16-byte load
  const int lane = threadIdx.x & 15;
  const int64_t t = (int64_t)blockIdx.x * 16 + (threadIdx.x >> 4);
  const int64_t h = blockIdx.y;
  float ka = 0.0f, va = 0.0f;
  if (t < S) {
    for (int64_t b = 0; b < B; ++b) {
      const int64_t row = ((b * H + h) * S + t) * D;
      if constexpr (VEC) {
        for (int64_t d = (int64_t)lane * VE; d < D; d += 16 * VE) {
          const uint4 xk = *reinterpret_cast<const uint4*>(reinterpret_cast<const char*>(k) + (row + d) * ES);
          const uint4 xv = *reinterpret_cast<const uint4*>(reinterpret_cast<const char*>(v) + (row + d) * ES);
          const uint32_t wk[4] = {xk.x, xk.y, xk.z, xk.w};
          const uint32_t wv[4] = {xv.x, xv.y, xv.z, xv.w};
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            if constexpr (DT == SI_DT_F32) {
              ka = amax_nan(ka, __uint_as_float(wk[e]));
              va = amax_nan(va, __uint_as_float(wv[e]));
            } else if constexpr (DT == SI_DT_F16) {
              ka = amax_nan(amax_nan(ka, f16_bits_to_f32(wk[e] & 0xffffu)), f16_bits_to_f32(wk[e] >> 16));
              va = amax_nan(amax_nan(va, f16_bits_to_f32(wv[e] & 0xffffu)), f16_bits_to_f32(wv[e] >> 16));
            } else {
              ka = amax_nan(amax_nan(ka, bf16_bits_to_f32(wk[e] & 0xffffu)), bf16_bits_to_f32(wk[e] >> 16));
              va = amax_nan(amax_nan(va, bf16_bits_to_f32(wv[e] & 0xffffu)), bf16_bits_to_f32(wv[e] >> 16));
            }
          }
        }
      } else {
        for (int64_t d = lane; d < D; d += 16) {
          ka = amax_nan(ka, elem<DT>(k, row + d));
          va = amax_nan(va, elem<DT>(v, row + d));
        }
      }
    }
  }
#pragma unroll
  for (int o = 8; o > 0; o >>= 1) {
    ka = amax_nan(ka, __shfl_xor(ka, o, 16));
    va = amax_nan(va, __shfl_xor(va, o, 16));
  }
  if (lane != 0 || t >= S) return;
  const float s = round_dt<DT>(round_dt<DT>(ka * ka) + round_dt<DT>(va * va)) / 2.0f;
  store_any(out, DT, t * H + h, s);
}

}  // namespace
}  // namespace si

using namespace si;

namespace {

size_t adm_align(size_t x) { return (x + 255) & ~(size_t)255; }

struct AdmLayout {
  size_t key, cand, hist, blk, state, total;
};

AdmLayout adm_layout(int64_t n) {
  AdmLayout l;
  const int64_t nblk = ceil_div(n, TIE_CHUNK);
  l.key = 0;
  l.cand = adm_align(l.key + (size_t)n * 4);
  l.hist = adm_align(l.cand + (size_t)n);
  l.blk = adm_align(l.hist + 256 * 8);
  l.state = adm_align(l.blk + (size_t)(nblk > 0 ? nblk : 1) * 8);
  l.total = adm_align(l.state + sizeof(AdmState));
  return l;
}

unsigned adm_grid(int64_t n) {
  return (unsigned)std::max<int64_t>(1, std::min<int64_t>(ceil_div(n, ADM_THREADS), 2048));
}

}  // namespace

extern "C" size_t si_admit_workspace_bytes(int64_t n_entries) {
  return n_entries < 0 ? 0 : adm_layout(n_entries).total;
}

extern "C" int si_admit_codes(const int8_t* codes, int8_t* out_codes, int64_t S, int64_t H,
                              const float* importance, const float* sensitivity,
                              const uint8_t* protected_mask, int64_t sink_tokens,
                              int64_t budget_bytes, int use_budget, int allow_eviction,
                              const int64_t* costs,
                              int64_t* result, void* workspace, size_t workspace_bytes,
                              si_stream_t stream) {
  clear_error();
  SI_CHECK_ARG(S >= 0 && H >= 0, "si_admit_codes: negative shape (%lld, %lld)", (long long)S,
               (long long)H);
  SI_CHECK_ARG(costs != nullptr && result != nullptr, "si_admit_codes: null costs or result");
  for (int c = 0; c < 5; ++c)
    SI_CHECK_ARG(costs[c] >= 0, "si_admit_codes: negative cost for code %d", c);
  const int64_t n = S * H;
  SI_CHECK_ARG(n == 0 || (codes && out_codes && importance),
               "si_admit_codes: null codes, out_codes or importance");
  const AdmLayout l = adm_layout(n);
  SI_CHECK_ARG(workspace != nullptr && workspace_bytes >= l.total &&
                   (reinterpret_cast<uintptr_t>(workspace) & 255) == 0,
               "si_admit_codes: workspace must be 256-byte aligned and hold %zu bytes", l.total);
  hipStream_t st = as_stream(stream);
  char* ws = static_cast<char*>(workspace);
  unsigned int* key = reinterpret_cast<unsigned int*>(ws + l.key);
  uint8_t* cand = reinterpret_cast<uint8_t*>(ws + l.cand);
  unsigned long long* hist = reinterpret_cast<unsigned long long*>(ws + l.hist);
  unsigned long long* blk = reinterpret_cast<unsigned long long*>(ws + l.blk);
  AdmState* state = reinterpret_cast<AdmState*>(ws + l.state);
  AdmCosts cs;
  for (int c = 0; c < 5; ++c) cs.cost[c] = costs[c];
  for (int c = 0; c < 3; ++c) cs.delta[c] = costs[c] - costs[c + 1];

  adm_init<<<1, 256, 0, st>>>(state, hist, budget_bytes, use_budget ? 1 : 0);
  if (int rc = check_launch("si_admit_codes")) return rc;
  if (n > 0) {
    const unsigned grid = adm_grid(n);
    const int64_t nblk = ceil_div(n, TIE_CHUNK);
    adm_prep<<<grid, ADM_THREADS, 0, st>>>(codes, out_codes, n, H, importance, sensitivity,
                                           protected_mask, sink_tokens, cs, key, cand, state);
    for (int mode = MODE_DOWN; mode <= MODE_EVICT; ++mode) {
      adm_sel_begin<<<1, 64, 0, st>>>(state, mode, allow_eviction);
      for (int d = 3; d >= 0; --d) {
        adm_hist<<<grid, ADM_THREADS, 0, st>>>(mode, d, key, cand, out_codes, n, cs, hist, state);
        adm_pick<<<1, 256, 0, st>>>(d, hist, state);
      }
      adm_tie_sum<<<(unsigned)nblk, ADM_THREADS, 0, st>>>(mode, key, cand, out_codes, n, cs, blk,
                                                           state);
      adm_tie_pick<<<1, 1024, 0, st>>>(mode, key, cand, out_codes, n, cs, blk, nblk, state);
      adm_apply<<<grid, ADM_THREADS, 0, st>>>(mode, key, cand, out_codes, n, cs, state,
                                              mode == MODE_DOWN ? 1 : 2);
    }
    if (int rc = check_launch("si_admit_codes")) return rc;
  }
  adm_finish<<<1, 64, 0, st>>>(state, result);
  return check_launch("si_admit_codes");
}

extern "C" int si_kv_sensitivity(const void* k, const void* v, int dtype, int64_t B, int64_t H,
                                 int64_t S, int64_t D, void* out, si_stream_t stream) {
  clear_error();
  SI_CHECK_ARG(dtype_ok(dtype), "si_kv_sensitivity: unsupported dtype %d", dtype);
  SI_CHECK_ARG(B >= 0 && H >= 0 && S >= 0 && D >= 0, "si_kv_sensitivity: negative shape");
  if (S == 0 || H == 0) return SI_OK;
  SI_CHECK_ARG(out != nullptr && (B * D == 0 || (k != nullptr && v != nullptr)),
               "si_kv_sensitivity: null pointer");
  SI_CHECK_ARG(H < 65536, "si_kv_sensitivity: too many heads (%lld)", (long long)H);
  const int es = dtype_size(dtype);
  const bool vec = (D * es) % 16 == 0 && ((reinterpret_cast<uintptr_t>(k) | reinterpret_cast<uintptr_t>(v)) & 15) == 0;
  const dim3 grid((unsigned)ceil_div(S, 16), (unsigned)H);
  hipStream_t st = as_stream(stream);
#define SI_SENS(DT_)                                                                  \
  do {                                                                                \
    if (vec) kv_sens_kernel<DT_, true><<<grid, 256, 0, st>>>(k, v, B, H, S, D, out);  \
    else kv_sens_kernel<DT_, false><<<grid, 256, 0, st>>>(k, v, B, H, S, D, out);     \
  } while (0)
  if (dtype == SI_DT_F32) SI_SENS(SI_DT_F32);
  else if (dtype == SI_DT_F16) SI_SENS(SI_DT_F16);
  else SI_SENS(SI_DT_BF16);
#undef SI_SENS
  return check_launch("si_kv_sensitivity");
}
