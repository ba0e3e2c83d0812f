// Precision-plan kernels: per-precision bucket positions by prefix sums.
//
// Bucket order is token-major (entry id e = t*H + h ascending within each
// precision), the order PrecisionPlan.from_codes produces with nonzero()
// (shadowinfer/shadowkv/precision_plan.py:136-151). Positions come from a
// three-step scan over tiles of 4096 entries:
//   1. plan_count   : per-tile counts of codes 0..3 (16-bit fields in a u64)
//   2. plan_offsets : exclusive scan of the tile counts -> per-tile bases,
//                     plus the bucket sizes
//   3. plan_slots   : per-thread exclusive scan inside each tile -> slot
// No atomics are involved, so the result is deterministic.
#include "si_common.h"

namespace si {
namespace {

constexpr int kThreads = 256;
constexpr int kPerThread = 16;
constexpr int kTile = kThreads * kPerThread;  // 4096 entries

using u64 = unsigned long long;

// Sanitized code of entry e: values outside 0..4 and entries hit by the
// optional eviction mask become 4 (absent).
__device__ __forceinline__ int sanitize(int c, const uint8_t* mask, int64_t e) {
  if (c < 0 || c > 4) c = 4;
  if (mask != nullptr && c < 4 && mask[e] != 0) c = 4;
  return c;
}

__device__ __forceinline__ void load_codes(const int8_t* codes, const uint8_t* mask, int64_t n,
                                           int64_t base, int out[kPerThread]) {
  if (base + kPerThread <= n && ((reinterpret_cast<uintptr_t>(codes + base) & 15) == 0)) {
    int4 raw = *reinterpret_cast<const int4*>(codes + base);
    const int8_t* b = reinterpret_cast<const int8_t*>(&raw);
#pragma unroll
    for (int i = 0; i < kPerThread; ++i) out[i] = sanitize(b[i], mask, base + i);
  } else {
#pragma unroll
    for (int i = 0; i < kPerThread; ++i)
      out[i] = (base + i < n) ? sanitize(codes[base + i], mask, base + i) : 4;
  }
}

__device__ __forceinline__ u64 count_packed(const int c[kPerThread]) {
  u64 v = 0;
#pragma unroll
  for (int i = 0; i < kPerThread; ++i) v += c[i] < 4 ? (1ull << (16 * c[i])) : 0ull;
  return v;
}

// Exclusive scan of one u64 per thread across a 256-thread block.
__device__ __forceinline__ u64 block_exclusive_scan(u64 v, u64* lds, u64* total) {
  const int lane = threadIdx.x & 63;
  const int wid = threadIdx.x >> 6;
  u64 x = v;
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) {
    u64 y = __shfl_up(x, off, 64);
    if (lane >= off) x += y;
  }
  if (lane == 63) lds[wid] = x;
  __syncthreads();
  u64 before = 0, tot = 0;
#pragma unroll
  for (int w = 0; w < kThreads / 64; ++w) {
    u64 s = lds[w];
    before += (w < wid) ? s : 0ull;
    tot += s;
  }
  __syncthreads();
  *total = tot;
  return before + x - v;
}

__global__ __launch_bounds__(kThreads) void plan_count(const int8_t* __restrict__ codes,
                                                       const uint8_t* __restrict__ mask,
                                                       int64_t n, u64* __restrict__ tile_counts) {
  __shared__ u64 lds[kThreads / 64];
  int c[kPerThread];
  const int64_t base = (int64_t)blockIdx.x * kTile + (int64_t)threadIdx.x * kPerThread;
  load_codes(codes, mask, n, base, c);
  u64 total;
  block_exclusive_scan(count_packed(c), lds, &total);
  if (threadIdx.x == 0) tile_counts[blockIdx.x] = total;
}

// One block. Tile counts are widened to 32-bit fields (two per u64) so a chunk
// of 256 tiles (<= 2^20 entries per code) cannot overflow; chunks carry int64.
__global__ __launch_bounds__(kThreads) void plan_offsets(const u64* __restrict__ tile_counts,
                                                         int64_t ntiles, int64_t n,
                                                         int32_t* __restrict__ tile_base,
                                                         int64_t* __restrict__ counts) {
  __shared__ u64 lds[kThreads / 64];
  int64_t carry[4] = {0, 0, 0, 0};
  for (int64_t chunk = 0; chunk < ntiles; chunk += kThreads) {
    const int64_t tile = chunk + threadIdx.x;
    const u64 packed = tile < ntiles ? tile_counts[tile] : 0ull;
    const u64 lo = (packed & 0xffffull) | (((packed >> 16) & 0xffffull) << 32);
    const u64 hi = ((packed >> 32) & 0xffffull) | (((packed >> 48) & 0xffffull) << 32);
    u64 tot_lo, tot_hi;
    const u64 ex_lo = block_exclusive_scan(lo, lds, &tot_lo);
    const u64 ex_hi = block_exclusive_scan(hi, lds, &tot_hi);
    if (tile < ntiles) {
      tile_base[tile * 4 + 0] = (int32_t)(carry[0] + (int64_t)(ex_lo & 0xffffffffull));
      tile_base[tile * 4 + 1] = (int32_t)(carry[1] + (int64_t)(ex_lo >> 32));
      tile_base[tile * 4 + 2] = (int32_t)(carry[2] + (int64_t)(ex_hi & 0xffffffffull));
      tile_base[tile * 4 + 3] = (int32_t)(carry[3] + (int64_t)(ex_hi >> 32));
    }
    carry[0] += (int64_t)(tot_lo & 0xffffffffull);
    carry[1] += (int64_t)(tot_lo >> 32);
    carry[2] += (int64_t)(tot_hi & 0xffffffffull);
    carry[3] += (int64_t)(tot_hi >> 32);
  }
  if (threadIdx.x == 0) {
    for (int p = 0; p < 4; ++p) counts[p] = carry[p];
    counts[4] = n - carry[0] - carry[1] - carry[2] - carry[3];
  }
}

__global__ __launch_bounds__(kThreads) void plan_slots(const int8_t* __restrict__ codes,
                                                       const uint8_t* __restrict__ mask, int64_t n,
                                                       const int32_t* __restrict__ tile_base,
                                                       int8_t* __restrict__ out_code,
                                                       int32_t* __restrict__ out_slot) {
  __shared__ u64 lds[kThreads / 64];
  int c[kPerThread];
  const int64_t base = (int64_t)blockIdx.x * kTile + (int64_t)threadIdx.x * kPerThread;
  load_codes(codes, mask, n, base, c);
  u64 total;
  const u64 before = block_exclusive_scan(count_packed(c), lds, &total);
  int run[4];
#pragma unroll
  for (int p = 0; p < 4; ++p)
    run[p] = tile_base[blockIdx.x * 4 + p] + (int)((before >> (16 * p)) & 0xffffull);
  int slots[kPerThread];
  int8_t cc[kPerThread];
#pragma unroll
  for (int i = 0; i < kPerThread; ++i) {
    const int ci = c[i];
    int s = -1;
#pragma unroll
    for (int p = 0; p < 4; ++p) {
      if (ci == p) s = run[p]++;
    }
    slots[i] = s;
    cc[i] = (int8_t)ci;
  }
  const bool vec = base + kPerThread <= n &&
                   ((reinterpret_cast<uintptr_t>(out_code + base) & 15) == 0) &&
                   ((reinterpret_cast<uintptr_t>(out_slot + base) & 15) == 0);
  if (vec) {
    uint32_t w[4];
#pragma unroll
    for (int j = 0; j < 4; ++j)
      w[j] = (uint32_t)(uint8_t)cc[4 * j] | ((uint32_t)(uint8_t)cc[4 * j + 1] << 8) |
             ((uint32_t)(uint8_t)cc[4 * j + 2] << 16) | ((uint32_t)(uint8_t)cc[4 * j + 3] << 24);
    *reinterpret_cast<int4*>(out_code + base) = make_int4((int)w[0], (int)w[1], (int)w[2], (int)w[3]);
#pragma unroll
    for (int i = 0; i < kPerThread; i += 4)
      *reinterpret_cast<int4*>(out_slot + base + i) = make_int4(slots[i], slots[i + 1],
                                                                slots[i + 2], slots[i + 3]);
  } else {
    for (int i = 0; i < kPerThread; ++i) {
      if (base + i < n) {
        out_code[base + i] = cc[i];
        out_slot[base + i] = slots[i];
      }
    }
  }
}

struct ScatterOut {
  int64_t* flat[4];
  int32_t* entry[4];
};

__global__ __launch_bounds__(256) void plan_scatter(const int8_t* __restrict__ code,
                                                   const int32_t* __restrict__ slot, int64_t S,
                                                   int64_t H, ScatterOut out) {
  const int64_t n = S * H;
  for (int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; e < n;
       e += (int64_t)gridDim.x * blockDim.x) {
    const int c = code[e];
    if (c < 0 || c > 3) continue;
    const int32_t s = slot[e];
    const int64_t t = e / H;
    const int64_t h = e - t * H;
    int64_t* f = nullptr;
    int32_t* en = nullptr;
#pragma unroll
    for (int p = 0; p < 4; ++p) {
      if (c == p) {
        f = out.flat[p];
        en = out.entry[p];
      }
    }
    if (f != nullptr) f[s] = h * S + t;
    if (en != nullptr) en[s] = (int32_t)e;
  }
}

size_t workspace_bytes(int64_t n) {
  const int64_t ntiles = ceil_div(n > 0 ? n : 1, kTile);
  return (size_t)(ntiles * sizeof(u64) + ntiles * 4 * sizeof(int32_t) + 256);
}

}  // namespace
}  // namespace si

extern "C" size_t si_plan_workspace_bytes(int64_t n_entries) {
  return si::workspace_bytes(n_entries);
}

extern "C" int si_plan_scan(const int8_t* codes, const uint8_t* evict_mask, int64_t n,
                            int8_t* out_code, int32_t* out_slot, int64_t* out_counts,
                            void* workspace, size_t workspace_bytes, si_stream_t stream) {
  using namespace si;
  clear_error();
  SI_CHECK_ARG(n >= 0, "si_plan_scan: n_entries must be >= 0 (got %lld)", (long long)n);
  SI_CHECK_ARG(n < (int64_t)1 << 31, "si_plan_scan: n_entries must be < 2^31");
  SI_CHECK_ARG(out_counts != nullptr, "si_plan_scan: out_counts is NULL");
  SI_CHECK_ARG(n == 0 || (codes && out_code && out_slot), "si_plan_scan: NULL buffer");
  SI_CHECK_ARG(workspace != nullptr && workspace_bytes >= si::workspace_bytes(n),
               "si_plan_scan: workspace too small (%zu < %zu)", workspace_bytes,
               si::workspace_bytes(n));
  hipStream_t st = as_stream(stream);
  const int64_t ntiles = ceil_div(n > 0 ? n : 1, kTile);
  u64* tile_counts = reinterpret_cast<u64*>(workspace);
  int32_t* tile_base = reinterpret_cast<int32_t*>(tile_counts + ntiles);
  if (n > 0) {
    plan_count<<<dim3((unsigned)ntiles), dim3(kThreads), 0, st>>>(codes, evict_mask, n,
                                                                  tile_counts);
    if (int rc = check_launch("si_plan_scan/count")) return rc;
  }
  plan_offsets<<<1, kThreads, 0, st>>>(tile_counts, n > 0 ? ntiles : 0, n, tile_base,
                                       out_counts);
  if (int rc = check_launch("si_plan_scan/offsets")) return rc;
  if (n > 0) {
    plan_slots<<<dim3((unsigned)ntiles), dim3(kThreads), 0, st>>>(codes, evict_mask, n,
                                                                  tile_base, out_code,
                                                                  out_slot);
    if (int rc = check_launch("si_plan_scan/slots")) return rc;
  }
  return SI_OK;
}

extern "C" int si_plan_scatter(const int8_t* code, const int32_t* slot, int64_t S, int64_t H,
                               int64_t* const* flat_out, int32_t* const* entry_out,
                               si_stream_t stream) {
  using namespace si;
  clear_error();
  SI_CHECK_ARG(S >= 0 && H >= 0, "si_plan_scatter: negative shape");
  const int64_t n = S * H;
  if (n == 0) return SI_OK;
  SI_CHECK_ARG(code && slot, "si_plan_scatter: NULL code/slot");
  ScatterOut out;
  for (int p = 0; p < 4; ++p) {
    out.flat[p] = flat_out ? flat_out[p] : nullptr;
    out.entry[p] = entry_out ? entry_out[p] : nullptr;
  }
  const int64_t blocks = std::min<int64_t>(ceil_div(n, 256), 65536);
  plan_scatter<<<dim3((unsigned)blocks), dim3(256), 0, as_stream(stream)>>>(code, slot, S, H,
                                                                           out);
  return check_launch("si_plan_scatter");
}
