// ak_common.h -- shared device helpers for the gfx950 kernels of libak355.
//
// Element types are carried as traits (TF32 / TF16 / TBF16): storage type, elements per
// 16-byte vector, and conversions to / from fp32. Rounding to f16 / bf16 is round-to-nearest-even
// and overflows to +-inf (never clamps), which is what a torch tensor op does when it stores an
// fp32 result into a half / bfloat16 tensor.
#pragma once

#include <hip/hip_ext.h>
#include <hip/hip_runtime.h>
#include <stdint.h>
#include <string.h>

#include "../../include/ak355.h"

namespace ak {

constexpr int kWave = 64;  // CDNA wavefront width

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));

// ---------------------------------------------------------------------------------------------
// Element-type traits
// ---------------------------------------------------------------------------------------------
struct TF32 {
  using S = float;
  static constexpr int kVec = 4;  // elements per 16-byte vector
  static constexpr int kCode = AK_F32;
  __device__ __forceinline__ static float to_f(S v) { return v; }
  __device__ __forceinline__ static S from_f(float f) { return f; }
  __device__ __forceinline__ static float rnd(float f) { return f; }
  // i-th element of a 16-byte vector
  __device__ __forceinline__ static float lane_elem(const u32x4& v, int i) {
    return __uint_as_float(v[i]);
  }
  __device__ __forceinline__ static void set_elem(u32x4& v, int i, float f) { v[i] = __float_as_uint(f); }
};

// The fp32 value is made opaque before a conversion to f16: hipcc otherwise folds a multiply, fma
// or add that feeds the conversion into v_fma_mixlo_f16, which rounds the exact result to f16
// once. A torch op rounds to fp32 first and then to f16; the two differ where the fp32 value
// lies exactly halfway between two f16 values (gelu(-1.4853515625) is one). The empty asm emits
// no instruction and, not being volatile, does not constrain scheduling.
__device__ __forceinline__ float f32_opaque(float f) {
  asm("" : "+v"(f));
  return f;
}

struct TF16 {
  using S = uint16_t;
  static constexpr int kVec = 8;
  static constexpr int kCode = AK_F16;
  __device__ __forceinline__ static float to_f(S v) { return (float)__builtin_bit_cast(_Float16, v); }
  __device__ __forceinline__ static S from_f(float f) { return __builtin_bit_cast(uint16_t, (_Float16)f32_opaque(f)); }
  __device__ __forceinline__ static float rnd(float f) { return (float)(_Float16)f32_opaque(f); }
  __device__ __forceinline__ static float lane_elem(const u32x4& v, int i) {
    uint32_t w = v[i >> 1];
    return to_f((S)((i & 1) ? (w >> 16) : (w & 0xffffu)));
  }
  __device__ __forceinline__ static void set_elem(u32x4& v, int i, float f) {
    uint32_t h = from_f(f);
    uint32_t w = v[i >> 1];
    v[i >> 1] = (i & 1) ? ((w & 0xffffu) | (h << 16)) : ((w & 0xffff0000u) | h);
  }
};

struct TBF16 {
  using S = uint16_t;
  static constexpr int kVec = 8;
  static constexpr int kCode = AK_BF16;
  __device__ __forceinline__ static float to_f(S v) { return __uint_as_float(((uint32_t)v) << 16); }
  __device__ __forceinline__ static S from_f(float f) { return __builtin_bit_cast(uint16_t, (__bf16)f); }
  __device__ __forceinline__ static float rnd(float f) { return to_f(from_f(f)); }
  __device__ __forceinline__ static float lane_elem(const u32x4& v, int i) {
    uint32_t w = v[i >> 1];
    return (i & 1) ? __uint_as_float(w & 0xffff0000u) : __uint_as_float(w << 16);
  }
  __device__ __forceinline__ static void set_elem(u32x4& v, int i, float f) {
    uint32_t h = from_f(f);
    uint32_t w = v[i >> 1];
    v[i >> 1] = (i & 1) ? ((w & 0xffffu) | (h << 16)) : ((w & 0xffff0000u) | h);
  }
};

// ---------------------------------------------------------------------------------------------
// Memory helpers
// ---------------------------------------------------------------------------------------------
__device__ __forceinline__ u32x4 ld16(const void* p) { return *reinterpret_cast<const u32x4*>(p); }
__device__ __forceinline__ void st16(void* p, const u32x4& v) { *reinterpret_cast<u32x4*>(p) = v; }
// Nontemporal store: data written once and not read back soon. Written as the instruction itself:
// a branch between this and a plain store (a run-time choice) would otherwise be merged into one
// plain store by the compiler, which drops the nontemporal hint.
__device__ __forceinline__ void st16_stream(void* p, const u32x4& v) {
  asm volatile("global_store_dwordx4 %0, %1, off nt" ::"v"(p), "v"(v) : "memory");
}

// ---------------------------------------------------------------------------------------------
// Wave64 reductions on the VALU. Steps 0-3 exchange inside rows of 16 lanes through DPP (lane ^ 1,
// lane ^ 2, the mirrored lane of an 8-lane half row, the mirrored lane of a 16-lane row); steps 4
// and 5 pair 16-lane rows through v_permlane16_swap and 32-lane halves through v_permlane32_swap.
// After steps 0..k every lane of an aligned 2^(k+1)-lane segment holds the segment's result. Each
// step combines two values with a commutative operation, so all lanes hold the same bits and the
// order is the same run to run (bitwise reproducible).
// ---------------------------------------------------------------------------------------------
template <int STEP, typename Op>
__device__ __forceinline__ float wave_step(float v, Op op) {
  if constexpr (STEP < 4) {
    // quad_perm [1,0,3,2], quad_perm [2,3,0,1], row_half_mirror, row_mirror
    constexpr int ctrl = STEP == 0 ? 0xB1 : STEP == 1 ? 0x4E : STEP == 2 ? 0x141 : 0x140;
    const float p = __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), ctrl, 0xF, 0xF, false));
    return op(v, p);
  } else if constexpr (STEP == 4) {
    const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return op(__uint_as_float(r[0]), __uint_as_float(r[1]));
  } else {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return op(__uint_as_float(r[0]), __uint_as_float(r[1]));
  }
}
// Reduce over aligned segments of L lanes (L a power of two, 1..64); every lane gets its result.
template <int L, typename Op>
__device__ __forceinline__ float seg_reduce(float v, Op op) {
  static_assert(L >= 1 && L <= 64 && (L & (L - 1)) == 0, "segment of 1..64 lanes");
  if constexpr (L >= 2) v = wave_step<0>(v, op);
  if constexpr (L >= 4) v = wave_step<1>(v, op);
  if constexpr (L >= 8) v = wave_step<2>(v, op);
  if constexpr (L >= 16) v = wave_step<3>(v, op);
  if constexpr (L >= 32) v = wave_step<4>(v, op);
  if constexpr (L >= 64) v = wave_step<5>(v, op);
  return v;
}

// NaN-propagating max (torch.max semantics): any NaN operand gives NaN.
__device__ __forceinline__ float nan_max(float a, float b) {
  return (a != a || a > b) ? a : b;
}

struct OpAdd {
  __device__ __forceinline__ float operator()(float a, float b) const { return a + b; }
};
struct OpMax {
  __device__ __forceinline__ float operator()(float a, float b) const { return fmaxf(a, b); }
};
struct OpNanMax {
  __device__ __forceinline__ float operator()(float a, float b) const { return nan_max(a, b); }
};
__device__ __forceinline__ float wave_sum(float v) { return seg_reduce<kWave>(v, OpAdd()); }
__device__ __forceinline__ float wave_max(float v) { return seg_reduce<kWave>(v, OpMax()); }
__device__ __forceinline__ float wave_nan_max(float v) { return seg_reduce<kWave>(v, OpNanMax()); }

// ---------------------------------------------------------------------------------------------
// LDS DMA (global / buffer loads that write LDS directly) and the waits around it
// ---------------------------------------------------------------------------------------------
typedef __attribute__((address_space(3))) void lds_void;

// This wave's vector-memory operations older than the newest N have completed (LDS-DMA
// transfers included). expcnt / lgkmcnt are left at their maxima (no wait).
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt field");
  // vmcnt(N) (bits 3:0 and 15:14)
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (0x7 << 4) | (0xf << 8));
}

// Barrier for the DMA pipelines: this wave's DMA transfers older than the newest N have landed
// and its own LDS reads have returned, then s_barrier. No memory-model fence: a workgroup release
// fence would also wait for the newest DMA transfers (they write LDS), collapsing the pipeline to
// one tile in flight. The signal fences keep the compiler from moving memory accesses across.
template <int N>
__device__ __forceinline__ void dma_barrier() {
  static_assert(N >= 0 && N < 64, "vmcnt field");
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
  // vmcnt(N), lgkmcnt(0), expcnt untouched
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (0x7 << 4));
  __builtin_amdgcn_s_barrier();
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
}

__device__ __forceinline__ int lane_id() { return threadIdx.x & (kWave - 1); }
__device__ __forceinline__ int wave_id() { return threadIdx.x >> 6; }

__device__ __forceinline__ bool aligned16(const void* p) { return (((uintptr_t)p) & 15u) == 0; }

// ---------------------------------------------------------------------------------------------
// Host-side helpers
// ---------------------------------------------------------------------------------------------
int record_launch(void);  // checks hipGetLastError(), stores its text, returns AK_OK / AK_EHIP
int record_hip_error(hipError_t e);  // AK_OK for hipSuccess, else stores e's text and returns AK_EHIP

// Start / stop events set by ak_set_launch_events for the calling thread's next timed launch
// (null when none); taking them clears the slot.
struct LaunchEvents {
  hipEvent_t start, stop;
};
LaunchEvents take_launch_events(void);

// Launch through hipExtLaunchKernelGGL when events are pending on this thread, so the dispatch
// itself records them at the kernel's start and end; a plain launch otherwise.
template <typename... Args, typename F = void (*)(Args...)>
inline void launch_timed(F kernel, dim3 grid, dim3 block, uint32_t shmem, hipStream_t s, Args... args) {
  const LaunchEvents e = take_launch_events();
  if (e.start || e.stop) hipExtLaunchKernelGGL(kernel, grid, block, shmem, s, e.start, e.stop, 0, args...);
  else kernel<<<grid, block, shmem, s>>>(args...);
}

inline bool host_aligned16(const void* p) { return (((uintptr_t)p) & 15u) == 0; }
inline int64_t cdiv(int64_t a, int64_t b) { return (a + b - 1) / b; }

// floor(n / d) for n, d < 2^31 as one multiply and one shift (Granlund and Montgomery, "Division
// by invariant integers using multiplication", 1994): with s = ceil(log2 d) and
// m = ceil(2^(31+s) / d) < 2^32, (n m) >> (31 + s) = floor(n / d), because the excess
// n (m d - 2^(31+s)) < 2^31 d <= 2^(31+s). The host computes (m, s) once per launch; a kernel's
// 64-bit index divisions otherwise compile to long VALU sequences per thread.
struct FastDiv {
  uint32_t m, s;
};
inline FastDiv make_fastdiv(uint32_t d) {
  uint32_t s = 0;
  while ((1ull << s) < d) ++s;
  return FastDiv{(uint32_t)(((1ull << (31 + s)) + d - 1) / d), s};
}
__device__ __forceinline__ uint32_t fdiv(uint32_t n, FastDiv f) {
  return (uint32_t)(((uint64_t)n * f.m) >> (31 + f.s));
}

}  // namespace ak

// Dispatch an element-type code to a traits type: AK_DISPATCH(dtype, T, { body using T; })
#define AK_DISPATCH(code, T, ...)                         \
  switch (code) {                                         \
    case AK_F32: { using T = ::ak::TF32; __VA_ARGS__; break; }   \
    case AK_F16: { using T = ::ak::TF16; __VA_ARGS__; break; }   \
    case AK_BF16: { using T = ::ak::TBF16; __VA_ARGS__; break; } \
    default: return AK_EINVAL;                            \
  }
