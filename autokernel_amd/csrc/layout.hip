// layout.hip -- a plain device copy: the bandwidth reference the benchmark times beside the
// HBM-bound ops (the practical ceiling at a given size).
#include <limits.h>

#include "ak_common.h"

namespace ak {

// One 16-byte vector per thread, all blocks in one pass. Measured on MI355X (cold cache) as the
// fastest of 1, 4 and 8 vectors per thread, with or without nontemporal hints.
__global__ __launch_bounds__(256) void copy16(const u32x4* __restrict__ src, u32x4* __restrict__ dst, int64_t n) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i < n) dst[i] = src[i];
}

}  // namespace ak

using namespace ak;

extern "C" int ak_copy(const void* src, void* dst, int64_t bytes, hipStream_t stream) {
  if (bytes < 0) return AK_EINVAL;
  if (bytes == 0) return AK_OK;
  if (!src || !dst) return AK_EINVAL;
  if (bytes % 16 != 0 || !host_aligned16(src) || !host_aligned16(dst)) return AK_EUNSUPPORTED;
  const int64_t n = bytes / 16, nb = cdiv(n, 256);
  if (nb > INT_MAX) return AK_EINVAL;
  launch_timed(copy16, dim3((unsigned)nb), dim3(256), 0, stream, (const u32x4*)src, (u32x4*)dst, n);
  return record_launch();
}
