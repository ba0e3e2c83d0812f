// Precision-plan kernels: per-precision bucket positions by prefix sums.
//
// Bucket order is token-major (entry id e = t*H + h ascending within each
// precision), the order PrecisionPlan.from_codes produces with nonzero()
// (shadowinfer/shadowkv/precision_plan.py:136-151). Positions come from a
// three-step scan over tiles of kTile entries (1024; four per thread, which
// puts 256 blocks on a 8192 x 32 plan: 12.0 -> 8.0 us for the evict rescan
// against sixteen per thread):
//   1. plan_count   : per-tile counts of codes 0..3 (16-bit fields in a u64)
//   2. plan_offsets : exclusive scan of the tile counts -> per-tile bases,
//                     plus the bucket sizes
//   3. plan_slots   : per-thread exclusive scan inside each tile -> slot
// No atomics are involved, so the result is deterministic.
#include "si_common.h"

namespace si {
namespace {

constexpr int kThreads = 256;
#ifndef SI_PLAN_PER_THREAD
#define SI_PLAN_PER_THREAD 4
#endif
constexpr int kPerThread = SI_PLAN_PER_THREAD;  // 4, 8 or 16
constexpr int kTile = kThreads * kPerThread;
static_assert(kPerThread == 4 || kPerThread == 8 || kPerThread == 16, "entries per thread");

using u64 = unsigned long long;

// Sanitized code of entry e: values outside 0..4 and entries hit by the
// optional eviction mask become 4 (absent).
__device__ __forceinline__ int sanitize(int c, const uint8_t* mask, int64_t e) {
  if (c < 0 || c > 4) c = 4;
  if (mask != nullptr && c < 4 && mask[e] != 0) c = 4;
  return c;
}

// kPerThread bytes (4, 8 or 16) from an aligned address, as 32-bit words.
__device__ __forceinline__ void load_bytes(const void* p, uint32_t w[kPerThread / 4]) {
  if constexpr (kPerThread == 16) {
    const uint4 v = *reinterpret_cast<const uint4*>(p);
    w[0] = v.x; w[1] = v.y; w[2] = v.z; w[3] = v.w;
  } else if constexpr (kPerThread == 8) {
    const uint2 v = *reinterpret_cast<const uint2*>(p);
    w[0] = v.x; w[1] = v.y;
  } else {
    w[0] = *reinterpret_cast<const uint32_t*>(p);
  }
}

__device__ __forceinline__ void load_codes(const int8_t* codes, const uint8_t* mask, int64_t n,
                                           int64_t base, int out[kPerThread]) {
  const uintptr_t mis = reinterpret_cast<uintptr_t>(codes + base) |
                        (mask != nullptr ? reinterpret_cast<uintptr_t>(mask + base) : 0);
  if (base + kPerThread <= n && (mis & (kPerThread - 1)) == 0) {
    uint32_t cw[kPerThread / 4], mw[kPerThread / 4];
    load_bytes(codes + base, cw);
    if (mask != nullptr) load_bytes(mask + base, mw);
#pragma unroll
    for (int i = 0; i < kPerThread; ++i) {
      int c = (int)(int8_t)(cw[i / 4] >> (8 * (i % 4)));
      if (c < 0 || c > 4) c = 4;
      if (mask != nullptr && c < 4 && ((mw[i / 4] >> (8 * (i % 4))) & 0xffu) != 0) c = 4;
      out[i] = c;
    }
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

// A thread's 16 codes and slots at entries base .. base+15 (16-byte stores
// where the run is whole and aligned).
__device__ __forceinline__ void store_code_slot(int8_t* out_code, int32_t* out_slot, int64_t n,
                                                int64_t base, const int c[kPerThread],
                                                const int slots[kPerThread]) {
  const bool vec = base + kPerThread <= n &&
                   ((reinterpret_cast<uintptr_t>(out_code + base) & (kPerThread - 1)) == 0) &&
                   ((reinterpret_cast<uintptr_t>(out_slot + base) & 15) == 0);
  if (vec) {
    uint32_t w[kPerThread / 4];
#pragma unroll
    for (int j = 0; j < kPerThread / 4; ++j)
      w[j] = (uint32_t)(uint8_t)c[4 * j] | ((uint32_t)(uint8_t)c[4 * j + 1] << 8) |
             ((uint32_t)(uint8_t)c[4 * j + 2] << 16) | ((uint32_t)(uint8_t)c[4 * j + 3] << 24);
    if constexpr (kPerThread == 16)
      *reinterpret_cast<uint4*>(out_code + base) = make_uint4(w[0], w[1], w[2], w[3]);
    else if constexpr (kPerThread == 8)
      *reinterpret_cast<uint2*>(out_code + base) = make_uint2(w[0], w[1]);
    else
      *reinterpret_cast<uint32_t*>(out_code + base) = w[0];
#pragma unroll
    for (int i = 0; i < kPerThread; i += 4)
      *reinterpret_cast<int4*>(out_slot + base + i) = make_int4(slots[i], slots[i + 1],
                                                                slots[i + 2], slots[i + 3]);
  } else {
    for (int i = 0; i < kPerThread; ++i) {
      if (base + i < n) {
        out_code[base + i] = (int8_t)c[i];
        out_slot[base + i] = slots[i];
      }
    }
  }
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
#pragma unroll
  for (int i = 0; i < kPerThread; ++i) {
    const int ci = c[i];
    int s = -1;
#pragma unroll
    for (int p = 0; p < 4; ++p) {
      if (ci == p) s = run[p]++;
    }
    slots[i] = s;
  }
  store_code_slot(out_code, out_slot, n, base, c, slots);
}

struct ScatterOut {
  int64_t* flat[4];
  int32_t* entry[4];
  int64_t cap[4];  // slots at or past cap[p] are not written
};

// Up to this many tiles (1M entries) each plan_slots_lists block adds up the
// counts of the tiles before it itself, so no separate offsets pass runs.
constexpr int64_t kFusedMaxTiles = 1024;

struct ListsOut {
  int64_t* flat[4];  // h*S + t per slot, or null
  int64_t cap[4];    // rows each list holds
};

// plan_slots with the tile offsets and the flat-list scatter folded in: the
// block sums the packed counts of tiles 0 .. blockIdx.x-1 (32-bit fields, so
// up to kFusedMaxTiles tiles cannot overflow), scans its own tile, writes
// code and slot, and stores h*S + t of every entry at its slot of the list of
// its precision (slots at or past cap[p] are not written; the caller sizes
// the lists). The last block writes the bucket sizes.
__global__ __launch_bounds__(kThreads) void plan_slots_lists(const int8_t* __restrict__ codes,
                                                             const uint8_t* __restrict__ mask,
                                                             int64_t S, int64_t H,
                                                             const u64* __restrict__ tile_counts,
                                                             int8_t* __restrict__ out_code,
                                                             int32_t* __restrict__ out_slot,
                                                             int64_t* __restrict__ counts,
                                                             ListsOut lists) {
  __shared__ u64 lds[kThreads / 64];
  __shared__ int64_t prior[4];
  const int64_t n = S * H;
  // counts of the tiles before this one (32-bit fields: lo = codes 0, 1; hi = 2, 3)
  u64 lo = 0, hi = 0;
  for (int64_t t = threadIdx.x; t < (int64_t)blockIdx.x; t += kThreads) {
    const u64 c = tile_counts[t];
    lo += (c & 0xffffull) | (((c >> 16) & 0xffffull) << 32);
    hi += ((c >> 32) & 0xffffull) | (((c >> 48) & 0xffffull) << 32);
  }
  u64 tot_lo, tot_hi;
  block_exclusive_scan(lo, lds, &tot_lo);
  block_exclusive_scan(hi, lds, &tot_hi);
  if (threadIdx.x == 0) {
    prior[0] = (int64_t)(tot_lo & 0xffffffffull);
    prior[1] = (int64_t)(tot_lo >> 32);
    prior[2] = (int64_t)(tot_hi & 0xffffffffull);
    prior[3] = (int64_t)(tot_hi >> 32);
  }
  __syncthreads();
  int c[kPerThread];
  const int64_t base = (int64_t)blockIdx.x * kTile + (int64_t)threadIdx.x * kPerThread;
  load_codes(codes, mask, n, base, c);
  u64 total;
  const u64 before = block_exclusive_scan(count_packed(c), lds, &total);
  if (blockIdx.x == gridDim.x - 1 && threadIdx.x == 0) {
    int64_t sum = 0;
    for (int p = 0; p < 4; ++p) {
      counts[p] = prior[p] + (int64_t)((total >> (16 * p)) & 0xffffull);
      sum += counts[p];
    }
    counts[4] = n - sum;
  }
  int run[4];
#pragma unroll
  for (int p = 0; p < 4; ++p) run[p] = (int)prior[p] + (int)((before >> (16 * p)) & 0xffffull);
  int slots[kPerThread];
#pragma unroll
  for (int i = 0; i < kPerThread; ++i) {
    const int ci = c[i];
    int sl = -1;
#pragma unroll
    for (int p = 0; p < 4; ++p) {
      if (ci == p) sl = run[p]++;
    }
    slots[i] = sl;
  }
  store_code_slot(out_code, out_slot, n, base, c, slots);
  int64_t t = base / H;
  int64_t h = base - t * H;
#pragma unroll
  for (int i = 0; i < kPerThread; ++i) {
    const int ci = c[i];
    if (slots[i] >= 0) {
      int64_t* f = nullptr;
      int64_t cap = 0;
#pragma unroll
      for (int p = 0; p < 4; ++p) {
        if (ci == p) {
          f = lists.flat[p];
          cap = lists.cap[p];
        }
      }
      if (f != nullptr && slots[i] < cap) f[slots[i]] = h * S + t;
    }
    if (++h == H) {
      h = 0;
      ++t;
    }
  }
}

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
    int64_t cap = 0;
#pragma unroll
    for (int p = 0; p < 4; ++p) cap = c == p ? out.cap[p] : cap;
    if (s >= cap) continue;
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

extern "C" int si_plan_scan_lists(const int8_t* codes, const uint8_t* evict_mask, int64_t S,
                                  int64_t H, int8_t* out_code, int32_t* out_slot,
                                  int64_t* out_counts, int64_t* const* flat_out,
                                  const int64_t* flat_capacity, void* workspace,
                                  size_t workspace_bytes, si_stream_t stream) {
  using namespace si;
  clear_error();
  SI_CHECK_ARG(S >= 0 && H >= 0, "si_plan_scan_lists: negative shape");
  const int64_t n = S * H;
  SI_CHECK_ARG(n < (int64_t)1 << 31, "si_plan_scan_lists: S * H must be < 2^31");
  SI_CHECK_ARG(out_counts != nullptr && flat_out != nullptr && flat_capacity != nullptr,
               "si_plan_scan_lists: NULL argument");
  const int64_t ntiles = ceil_div(n > 0 ? n : 1, kTile);
  if (n == 0 || ntiles > kFusedMaxTiles) {
    // large plans: the three-pass scan, then the scatter into lists of the
    // capacities given (they must hold the new buckets)
    if (int rc = si_plan_scan(codes, evict_mask, n, out_code, out_slot, out_counts, workspace,
                              workspace_bytes, stream))
      return rc;
    if (n == 0) return SI_OK;
    ScatterOut out;
    for (int p = 0; p < 4; ++p) {
      out.flat[p] = flat_capacity[p] > 0 ? flat_out[p] : nullptr;
      out.entry[p] = nullptr;
      out.cap[p] = flat_capacity[p];
    }
    const int64_t blocks = std::min<int64_t>(ceil_div(n, 256), 65536);
    plan_scatter<<<dim3((unsigned)blocks), dim3(256), 0, as_stream(stream)>>>(out_code, out_slot,
                                                                             S, H, out);
    return check_launch("si_plan_scan_lists/scatter");
  }
  SI_CHECK_ARG(codes && out_code && out_slot, "si_plan_scan_lists: NULL buffer");
  SI_CHECK_ARG(workspace != nullptr && workspace_bytes >= si::workspace_bytes(n),
               "si_plan_scan_lists: workspace too small (%zu < %zu)", workspace_bytes,
               si::workspace_bytes(n));
  ListsOut lists;
  for (int p = 0; p < 4; ++p) {
    SI_CHECK_ARG(flat_capacity[p] >= 0, "si_plan_scan_lists: negative capacity");
    lists.flat[p] = flat_capacity[p] > 0 ? flat_out[p] : nullptr;
    lists.cap[p] = flat_capacity[p];
    SI_CHECK_ARG(flat_capacity[p] == 0 || flat_out[p] != nullptr,
                 "si_plan_scan_lists: NULL list %d", p);
  }
  hipStream_t st = as_stream(stream);
  u64* tile_counts = reinterpret_cast<u64*>(workspace);
  plan_count<<<dim3((unsigned)ntiles), dim3(kThreads), 0, st>>>(codes, evict_mask, n, tile_counts);
  if (int rc = check_launch("si_plan_scan_lists/count")) return rc;
  plan_slots_lists<<<dim3((unsigned)ntiles), dim3(kThreads), 0, st>>>(
      codes, evict_mask, S, H, tile_counts, out_code, out_slot, out_counts, lists);
  return check_launch("si_plan_scan_lists/slots");
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
    out.cap[p] = INT64_MAX;  // the caller sizes the lists by the plan's counts
  }
  const int64_t blocks = std::min<int64_t>(ceil_div(n, 256), 65536);
  plan_scatter<<<dim3((unsigned)blocks), dim3(256), 0, as_stream(stream)>>>(code, slot, S, H,
                                                                           out);
  return check_launch("si_plan_scatter");
}
