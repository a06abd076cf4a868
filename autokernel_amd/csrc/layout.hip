// layout.hip -- 2-D transpose (a layout helper) and a plain device copy (the bandwidth reference).
//
// dst[c][r] = src[r][c] for a rows x cols matrix. 64 x 64 tiles through LDS: 16-byte loads along
// src rows, 16-byte stores along dst rows; the LDS tile has a padded pitch (66 halves) so the
// column gathers of the store phase hit distinct banks. Partial or unaligned tiles take a scalar
// path. HBM-bound: reads and writes rows * cols elements once.
#include <limits.h>

#include "ak_common.h"

namespace ak {

constexpr int kTT = 64;        // tile edge
constexpr int kTPitch = 66;    // LDS pitch in 2-byte elements

__global__ __launch_bounds__(256) void transpose16(const uint16_t* __restrict__ src, uint16_t* __restrict__ dst,
                                                   int rows, int cols, int64_t ld_src, int64_t ld_dst, int vec) {
  __shared__ uint16_t t[kTT * kTPitch];
  const int tiles_c = (cols + kTT - 1) / kTT;
  const int r0 = (blockIdx.x / tiles_c) * kTT, c0 = (blockIdx.x % tiles_c) * kTT;
  const bool full = vec && r0 + kTT <= rows && c0 + kTT <= cols;
  const int tid = threadIdx.x;
  if (full) {
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const int q = tid + i * 256, r = q >> 3, ch = q & 7;
      const u32x4 v = ld16(src + (int64_t)(r0 + r) * ld_src + c0 + ch * 8);
#pragma unroll
      for (int w = 0; w < 4; ++w) {
        t[r * kTPitch + ch * 8 + 2 * w] = (uint16_t)(v[w] & 0xffffu);
        t[r * kTPitch + ch * 8 + 2 * w + 1] = (uint16_t)(v[w] >> 16);
      }
    }
  } else {
    for (int q = tid; q < kTT * kTT; q += 256) {
      const int r = q / kTT, c = q % kTT;
      if (r0 + r < rows && c0 + c < cols) t[r * kTPitch + c] = src[(int64_t)(r0 + r) * ld_src + c0 + c];
    }
  }
  __syncthreads();
  if (full) {
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const int q = tid + i * 256, dr = q >> 3, ch = q & 7;  // dst row = src col c0 + dr
      u32x4 v;
#pragma unroll
      for (int w = 0; w < 4; ++w)
        v[w] = (uint32_t)t[(ch * 8 + 2 * w) * kTPitch + dr] | ((uint32_t)t[(ch * 8 + 2 * w + 1) * kTPitch + dr] << 16);
      st16(dst + (int64_t)(c0 + dr) * ld_dst + r0 + ch * 8, v);
    }
  } else {
    for (int q = tid; q < kTT * kTT; q += 256) {
      const int dr = q / kTT, dc = q % kTT;  // dst (c0 + dr, r0 + dc)
      if (c0 + dr < cols && r0 + dc < rows) dst[(int64_t)(c0 + dr) * ld_dst + r0 + dc] = t[dc * kTPitch + dr];
    }
  }
}

__global__ __launch_bounds__(256) void transpose32(const float* __restrict__ src, float* __restrict__ dst, int rows,
                                                   int cols, int64_t ld_src, int64_t ld_dst) {
  __shared__ float t[32 * 33];
  const int tiles_c = (cols + 31) / 32;
  const int r0 = (blockIdx.x / tiles_c) * 32, c0 = (blockIdx.x % tiles_c) * 32;
  for (int q = threadIdx.x; q < 32 * 32; q += 256) {
    const int r = q / 32, c = q % 32;
    if (r0 + r < rows && c0 + c < cols) t[r * 33 + c] = src[(int64_t)(r0 + r) * ld_src + c0 + c];
  }
  __syncthreads();
  for (int q = threadIdx.x; q < 32 * 32; q += 256) {
    const int dr = q / 32, dc = q % 32;
    if (c0 + dr < cols && r0 + dc < rows) dst[(int64_t)(c0 + dr) * ld_dst + r0 + dc] = t[dc * 33 + dr];
  }
}

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
  copy16<<<(unsigned)nb, 256, 0, stream>>>((const u32x4*)src, (u32x4*)dst, n);
  return record_launch();
}

extern "C" int ak_transpose(int dtype, const void* src, void* dst, int64_t rows, int64_t cols, int64_t ld_src,
                            int64_t ld_dst, hipStream_t stream) {
  if (rows < 0 || cols < 0 || rows > INT_MAX || cols > INT_MAX) return AK_EINVAL;
  if (rows == 0 || cols == 0) return AK_OK;
  if (!src || !dst || ld_src < cols || ld_dst < rows) return AK_EINVAL;
  if (dtype == AK_F32) {
    const int64_t nb = cdiv(rows, 32) * cdiv(cols, 32);
    if (nb > INT_MAX) return AK_EINVAL;
    transpose32<<<(unsigned)nb, 256, 0, stream>>>((const float*)src, (float*)dst, (int)rows, (int)cols, ld_src, ld_dst);
    return record_launch();
  }
  if (dtype != AK_F16 && dtype != AK_BF16) return AK_EINVAL;
  const int64_t nb = cdiv(rows, kTT) * cdiv(cols, kTT);
  if (nb > INT_MAX) return AK_EINVAL;
  const int vec = ld_src % 8 == 0 && ld_dst % 8 == 0 && host_aligned16(src) && host_aligned16(dst);
  transpose16<<<(unsigned)nb, 256, 0, stream>>>((const uint16_t*)src, (uint16_t*)dst, (int)rows, (int)cols, ld_src,
                                                ld_dst, vec);
  return record_launch();
}
