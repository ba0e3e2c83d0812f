// ABI plumbing: version, thread-local error text and the self-check of the
// hardware bf16 conversion the kernels rely on.
#include <stdarg.h>
#include <string.h>

#include "si_common.h"

namespace si {

static thread_local char g_error[512];

void set_error(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_error, sizeof(g_error), fmt, ap);
  va_end(ap);
}

void clear_error() { g_error[0] = '\0'; }

int check_launch(const char* what) {
  hipError_t err = hipGetLastError();
  if (err != hipSuccess) {
    set_error("%s: kernel launch failed: %s", what, hipGetErrorString(err));
    return SI_ERR_HIP;
  }
  return SI_OK;
}

}  // namespace si

extern "C" int si_abi_version(void) { return SI_ABI_VERSION; }

extern "C" const char* si_last_error(void) { return si::g_error; }

namespace si {
namespace {

// Bit-arithmetic round to nearest even, the definition the hardware
// conversion (f32_to_bf16_bits) is held to.
__device__ __forceinline__ uint32_t bf16_bits_reference(uint32_t u) {
  if ((u & 0x7fffffffu) > 0x7f800000u) return 0x7fc0u;
  u += 0x7fffu + ((u >> 16) & 1u);
  return u >> 16;
}

// Fp32 patterns base + 2 * thread + {0, 1}: counts[0] += patterns where the
// pair conversion differs from the reference, counts[1] += patterns where the
// single-value conversion does.
__global__ __launch_bounds__(256) void bf16_convert_check(unsigned long long* counts,
                                                          uint32_t base) {
  const uint32_t i0 = base + 2u * (blockIdx.x * 256u + threadIdx.x);
  const float a = __uint_as_float(i0), b = __uint_as_float(i0 + 1u);
  const uint32_t pair = f32x2_to_bf16x2_bits(a, b);
  const uint32_t ra = bf16_bits_reference(i0), rb = bf16_bits_reference(i0 + 1u);
  const unsigned bad_pair = ((pair & 0xffffu) != ra) + ((pair >> 16) != rb);
  const unsigned bad_single = (f32_to_bf16_bits(a) != ra) + (f32_to_bf16_bits(b) != rb);
  if (bad_pair) atomicAdd(&counts[0], (unsigned long long)bad_pair);
  if (bad_single) atomicAdd(&counts[1], (unsigned long long)bad_single);
}

}  // namespace
}  // namespace si

extern "C" int si_check_bf16_convert(unsigned long long* counts, si_stream_t stream) {
  si::clear_error();
  SI_CHECK_ARG(counts != nullptr, "si_check_bf16_convert: NULL counts");
  hipStream_t st = si::as_stream(stream);
  // 2^32 patterns: 8 launches of 2^20 blocks x 256 threads x 2 patterns
  for (uint32_t part = 0; part < 8; ++part)
    si::bf16_convert_check<<<1u << 20, 256, 0, st>>>(counts, part << 29);
  return si::check_launch("si_check_bf16_convert");
}
