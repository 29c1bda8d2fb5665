// Exhaustive device check of the rounding helpers the Q/K norm + RoPE kernel
// relies on (pack_bf16_rne, sqrt_rn), over all 2^32 float bit patterns.
#include "tmhd_internal.h"

namespace tmhd {
namespace {

__global__ void __launch_bounds__(256) rounding_selfcheck_kernel(unsigned long long *counts) {
  const uint32_t tid = blockIdx.x * blockDim.x + threadIdx.x;  // 2^20 threads, 4096 patterns each
  unsigned long long bad_bf16 = 0, bad_sqrt = 0;
  for (uint32_t it = 0; it < 4096; ++it) {
    const uint32_t u = tid + (it << 20);
    const float x = __uint_as_float(u);
    const bool nan = (u & 0x7fffffffu) > 0x7f800000u;
    // bf16: every non-NaN value and every quiet NaN whose low 16 bits are
    // zero must round as + 0x7FFF + bit 16, low half cleared
    if (!nan || ((u & 0xffffu) == 0 && (u & 0x00400000u))) {
      const uint32_t want = ((u + 0x7fffu + ((u >> 16) & 1u)) >> 16) & 0xffffu;
      if ((pack_bf16_rne(x, x) & 0xffffu) != want || (pack_bf16_rne(0.0f, x) >> 16) != want) ++bad_bf16;
    }
    // sqrt: every non-negative pattern; finite positive x must satisfy
    // m-^2 < x < m+^2 for the midpoints m-, m+ to the root's neighbours
    // (exact in double: 25-bit midpoints, 50-bit squares)
    if (!(u >> 31)) {
      const float r = sqrt_rn(x);
      const uint32_t ru = __float_as_uint(r);
      bool ok;
      if (nan)
        ok = r != r;
      else if (u == 0x7f800000u || u == 0u)
        ok = ru == u;
      else {
        const double lo = ((double)__uint_as_float(ru - 1u) + (double)r) * 0.5;
        const double hi = ((double)__uint_as_float(ru + 1u) + (double)r) * 0.5;
        ok = r > 0.0f && ru < 0x7f800000u && lo * lo < (double)x && (double)x < hi * hi;
      }
      if (!ok) ++bad_sqrt;
    }
  }
  if (bad_bf16) atomicAdd(&counts[0], bad_bf16);
  if (bad_sqrt) atomicAdd(&counts[1], bad_sqrt);
}

}  // namespace
}  // namespace tmhd

extern "C" int tmhd_selfcheck_rounding(unsigned long long *counts, void *stream) {
  using namespace tmhd;
  if (!counts || ((uintptr_t)counts % 8)) return set_error(TMHD_ERR_INVALID, "tmhd_selfcheck_rounding: counts");
  hipLaunchKernelGGL(rounding_selfcheck_kernel, dim3(4096), dim3(256), 0, (hipStream_t)stream, counts);
  return check_launch("tmhd_selfcheck_rounding");
}
