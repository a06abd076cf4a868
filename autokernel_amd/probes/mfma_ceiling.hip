// mfma_ceiling.hip -- the sustained MFMA throughput of one MI355X with no memory traffic.
//
//     autokernel_amd/probes/mfma_ceiling            (built by autokernel_amd.build)
//
// Every wave runs a register-only loop of independent MFMA chains (16x16x32: 8 accumulators,
// 32x32x16: 4) on operands that never change, f16 or bf16, either uniform in [-1, 1) (random
// mantissa bits, as real data has) or all zeros. Grids of 512 or 1024 blocks of 4 waves put 2 or
// 4 waves on every SIMD of the 256 CUs. Each block's first wave reads the shader clock counter
// (s_memtime) and the 100 MHz constant clock (s_memrealtime) at its start and end, so the line
// also gives the clock the loop actually ran at. The part is power-limited: switching operand
// bits costs power, so the clock (and with it the TFLOP/s) depends on the data. Memory is touched
// only by the final store of one float per lane and two counters per block.
#include <hip/hip_runtime.h>

#include <cstdint>
#include <cstdio>
#include <cstdlib>

typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

__device__ uint32_t mix(uint32_t x) {
  x ^= x >> 16; x *= 0x7feb352du; x ^= x >> 15; x *= 0x846ca68bu; x ^= x >> 16;
  return x;
}

// SHAPE 0: v_mfma_f32_16x16x32, SHAPE 1: v_mfma_f32_32x32x16; BF: bf16 operands
template <int SHAPE, bool BF, bool ZERO>
__global__ __launch_bounds__(256) void mfma_loop(float* out, unsigned long long* clk, int iters) {
  const uint32_t t = blockIdx.x * 256u + threadIdx.x;
  const unsigned long long c0 = __builtin_amdgcn_s_memtime();
  const unsigned long long r0 = __builtin_amdgcn_s_memrealtime();
  using V = typename std::conditional<BF, bf16x8, f16x8>::type;
  using E = typename std::conditional<BF, __bf16, _Float16>::type;
  V a[4], b[4];
  for (int i = 0; i < 4; ++i)
    for (int e = 0; e < 8; ++e) {
      const float va = ((int)(mix(t * 64u + i * 8u + e) & 1023u) - 512) / 512.0f;
      const float vb = ((int)(mix(t * 64u + 32u + i * 8u + e) & 1023u) - 512) / 512.0f;
      a[i][e] = (E)(ZERO ? 0.0f : va);
      b[i][e] = (E)(ZERO ? 0.0f : vb);
    }
  float s = 0.f;
  if constexpr (SHAPE == 0) {
    f32x4 acc[8] = {};
    for (int it = 0; it < iters; ++it)
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          if constexpr (BF) acc[j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a[i], b[j & 3], acc[j], 0, 0, 0);
          else acc[j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a[i], b[j & 3], acc[j], 0, 0, 0);
        }
    for (int j = 0; j < 8; ++j)
      for (int e = 0; e < 4; ++e) s += acc[j][e];
  } else {
    f32x16 acc[4] = {};
    for (int it = 0; it < iters; ++it)
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          if constexpr (BF) acc[j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[i], b[j], acc[j], 0, 0, 0);
          else acc[j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a[i], b[j], acc[j], 0, 0, 0);
        }
    for (int j = 0; j < 4; ++j)
      for (int e = 0; e < 16; ++e) s += acc[j][e];
  }
  out[t] = s;
  if (threadIdx.x == 0) {
    clk[2 * blockIdx.x] = __builtin_amdgcn_s_memtime() - c0;
    clk[2 * blockIdx.x + 1] = __builtin_amdgcn_s_memrealtime() - r0;
  }
}

#define CHECK(x)                                                               \
  do {                                                                         \
    hipError_t e_ = (x);                                                       \
    if (e_ != hipSuccess) {                                                    \
      fprintf(stderr, "%s: %s\n", #x, hipGetErrorString(e_));                  \
      exit(1);                                                                 \
    }                                                                          \
  } while (0)

constexpr int kMaxBlocks = 1024;
static float* g_out;
static unsigned long long* g_clk;

template <int SHAPE, bool BF, bool ZERO>
static void run(int blocks, int iters) {
  hipEvent_t e0, e1;
  CHECK(hipEventCreate(&e0));
  CHECK(hipEventCreate(&e1));
  mfma_loop<SHAPE, BF, ZERO><<<blocks, 256>>>(g_out, g_clk, iters / 10);  // warm-up
  CHECK(hipGetLastError());
  CHECK(hipDeviceSynchronize());
  CHECK(hipEventRecord(e0));
  mfma_loop<SHAPE, BF, ZERO><<<blocks, 256>>>(g_out, g_clk, iters);
  CHECK(hipGetLastError());
  CHECK(hipEventRecord(e1));
  CHECK(hipEventSynchronize(e1));
  float ms = 0.f;
  CHECK(hipEventElapsedTime(&ms, e0, e1));
  static unsigned long long h[2 * kMaxBlocks];
  CHECK(hipMemcpy(h, g_clk, 2 * blocks * sizeof(unsigned long long), hipMemcpyDeviceToHost));
  double cyc = 0, ref = 0;
  for (int b = 0; b < blocks; ++b) {
    cyc += (double)h[2 * b];
    ref += (double)h[2 * b + 1];
  }
  // per loop iteration per wave: 32 x 16x16x32 (16384 FLOP each) or 16 x 32x32x16 (32768 each)
  const double flop = (double)blocks * 4 * iters * (SHAPE == 0 ? 32.0 * 16384 : 16.0 * 32768);
  printf("%-9s %-4s %-6s waves/SIMD %d  %8.3f ms  %7.1f TFLOP/s  %5.1f%% of 2516.6  clock %.3f GHz\n",
         SHAPE == 0 ? "16x16x32" : "32x32x16", BF ? "bf16" : "f16", ZERO ? "zeros" : "random", blocks / 256, ms,
         flop / ms / 1e9, flop / ms / 1e9 / 2516.6 * 100.0, cyc / ref * 0.1);
  fflush(stdout);
  CHECK(hipEventDestroy(e0));
  CHECK(hipEventDestroy(e1));
}

int main() {
  CHECK(hipMalloc(&g_out, (size_t)kMaxBlocks * 256 * sizeof(float)));
  CHECK(hipMalloc(&g_clk, 2 * kMaxBlocks * sizeof(unsigned long long)));
  const int iters = 40000;  // about 25-60 ms per launch
  for (int blocks : {512, 1024}) {
    run<0, false, false>(blocks, iters);
    run<1, false, false>(blocks, iters);
    run<0, true, false>(blocks, iters);
    run<1, true, false>(blocks, iters);
    run<0, false, true>(blocks, iters);
    run<1, false, true>(blocks, iters);
  }
  CHECK(hipFree(g_out));
  CHECK(hipFree(g_clk));
  return 0;
}
