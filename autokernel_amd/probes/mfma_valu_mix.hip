// mfma_valu_mix.hip -- how much VALU and transcendental work hides behind MFMAs on one SIMD.
//
//     autokernel_amd/probes/mfma_valu_mix            (built by autokernel_amd.build)
//
// Each wave loops over 4 independent v_mfma_f32_32x32x16_f16 (32 cycles each, 128 per iteration)
// followed by NV independent fp32 FMAs and NE v_exp_f32 on other registers; 512 blocks of 4 waves
// put 2 waves on every SIMD of the 256 CUs, so the MFMA pipe alone needs 256 SIMD cycles per loop
// iteration. The line gives the cycles the iteration actually took (shader-clock counter over the
// 100 MHz constant clock, averaged over blocks) and the MFMA throughput: where the VALU work stops
// hiding behind the MFMAs and starts adding to them. Attention's softmax issues about 16 VALU
// operations and 4 exponentials per 4 MFMAs per wave (D = 128); a GEMM's k-loop issues almost none.
#include <hip/hip_runtime.h>

#include <cstdint>
#include <cstdio>
#include <cstdlib>

typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

__device__ uint32_t mix(uint32_t x) {
  x ^= x >> 16; x *= 0x7feb352du; x ^= x >> 15; x *= 0x846ca68bu; x ^= x >> 16;
  return x;
}

template <int NV, int NE>
__global__ __launch_bounds__(256) void mix_loop(float* out, unsigned long long* clk, int iters) {
  const uint32_t t = blockIdx.x * 256u + threadIdx.x;
  const unsigned long long c0 = __builtin_amdgcn_s_memtime();
  const unsigned long long r0 = __builtin_amdgcn_s_memrealtime();
  f16x8 a[4], b[4];
  for (int i = 0; i < 4; ++i)
    for (int e = 0; e < 8; ++e) {
      a[i][e] = (_Float16)(((int)(mix(t * 64u + i * 8u + e) & 1023u) - 512) / 512.0f);
      b[i][e] = (_Float16)(((int)(mix(t * 64u + 32u + i * 8u + e) & 1023u) - 512) / 512.0f);
    }
  f32x16 acc[4] = {};
  float v[16], w[8];
  for (int i = 0; i < 16; ++i) v[i] = (float)(mix(t + i) & 255u) * 1e-3f;
  for (int i = 0; i < 8; ++i) w[i] = (float)(mix(t + 99u + i) & 255u) * -1e-3f;
  for (int it = 0; it < iters; ++it) {
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a[j], b[j], acc[j], 0, 0, 0);
#pragma unroll
    for (int i = 0; i < NV; ++i) v[i & 15] = __builtin_fmaf(v[i & 15], 0.999f, 1e-4f);
#pragma unroll
    for (int i = 0; i < NE; ++i) w[i & 7] = __builtin_amdgcn_exp2f(w[i & 7]) - 1.0001f;
  }
  float s = 0.f;
  for (int j = 0; j < 4; ++j)
    for (int e = 0; e < 16; ++e) s += acc[j][e];
  for (int i = 0; i < 16; ++i) s += v[i];
  for (int i = 0; i < 8; ++i) s += w[i];
  out[t] = s;
  if (threadIdx.x == 0) {
    clk[2 * blockIdx.x] = __builtin_amdgcn_s_memtime() - c0;
    clk[2 * blockIdx.x + 1] = __builtin_amdgcn_s_memrealtime() - r0;
  }
}

#define CHECK(x)                                                  \
  do {                                                            \
    hipError_t e_ = (x);                                          \
    if (e_ != hipSuccess) {                                       \
      fprintf(stderr, "%s: %s\n", #x, hipGetErrorString(e_));     \
      exit(1);                                                    \
    }                                                             \
  } while (0)

constexpr int kBlocks = 512;  // 2 waves per SIMD
static float* g_out;
static unsigned long long* g_clk;

template <int NV, int NE>
static void run(int iters) {
  hipEvent_t e0, e1;
  CHECK(hipEventCreate(&e0));
  CHECK(hipEventCreate(&e1));
  mix_loop<NV, NE><<<kBlocks, 256>>>(g_out, g_clk, iters / 10);  // warm-up
  CHECK(hipGetLastError());
  CHECK(hipDeviceSynchronize());
  CHECK(hipEventRecord(e0));
  mix_loop<NV, NE><<<kBlocks, 256>>>(g_out, g_clk, iters);
  CHECK(hipGetLastError());
  CHECK(hipEventRecord(e1));
  CHECK(hipEventSynchronize(e1));
  float ms = 0.f;
  CHECK(hipEventElapsedTime(&ms, e0, e1));
  static unsigned long long h[2 * kBlocks];
  CHECK(hipMemcpy(h, g_clk, sizeof(h), hipMemcpyDeviceToHost));
  double cyc = 0, ref = 0;
  for (int b = 0; b < kBlocks; ++b) {
    cyc += (double)h[2 * b];
    ref += (double)h[2 * b + 1];
  }
  const double ghz = cyc / ref * 0.1;
  const double flop = (double)kBlocks * 4 * iters * 4 * 32768.0;
  printf("VALU %2d  exp %2d  per 4 MFMA: %8.1f TFLOP/s  clock %.3f GHz  %6.1f SIMD cycles per iteration (MFMA alone: 256)\n",
         NV, NE, flop / ms / 1e9, ghz, ms * 1e-3 * ghz * 1e9 / iters);
  fflush(stdout);
  CHECK(hipEventDestroy(e0));
  CHECK(hipEventDestroy(e1));
}

int main() {
  CHECK(hipMalloc(&g_out, (size_t)kBlocks * 256 * sizeof(float)));
  CHECK(hipMalloc(&g_clk, 2 * kBlocks * sizeof(unsigned long long)));
  const int iters = 20000;
  run<0, 0>(iters);
  run<8, 0>(iters);
  run<16, 0>(iters);
  run<32, 0>(iters);
  run<64, 0>(iters);
  run<0, 4>(iters);
  run<0, 8>(iters);
  run<0, 16>(iters);
  run<16, 4>(iters);
  run<16, 8>(iters);
  run<32, 8>(iters);
  CHECK(hipFree(g_out));
  CHECK(hipFree(g_clk));
  return 0;
}
