// row_common.h -- the row-parallel scheme shared by rmsnorm, layernorm, softmax, cross_entropy
// and the last-dim reductions.
//
// A row of `cols` elements is owned by a group of L lanes (L = 8 .. 1024). When the row start is
// 16-byte aligned and cols is a multiple of the 16-byte vector width, each lane loads up to VPT
// 16-byte vectors (vector v = lane_in_group + j * L) into fp32 registers, so the row is read from
// HBM exactly once and written once. Groups narrower than a wave share the wave (several rows per
// wave, segmented butterflies); groups wider than a wave combine their per-wave partials through
// LDS in a fixed order. Rows that are misaligned or too wide for registers use the looped kernels
// (one 256-thread block per row, scalar loads, two passes).
#pragma once
#include "ak_common.h"

namespace ak {


// Reduction over the L lanes of a segment (L <= 64: every lane ends with the segment result; a
// wider group reduces each of its waves here and combines them in group_combine).
template <int L>
__device__ __forceinline__ float seg_sum(float v) { return seg_reduce<(L < kWave ? L : kWave)>(v, OpAdd()); }
template <int L>
__device__ __forceinline__ float seg_max(float v) { return seg_reduce<(L < kWave ? L : kWave)>(v, OpMax()); }
template <int L>
__device__ __forceinline__ float seg_nan_max(float v) { return seg_reduce<(L < kWave ? L : kWave)>(v, OpNanMax()); }

// Combine per-wave partials of a group of L > 64 lanes (L / 64 waves) through LDS.
// Every wave of the block must call it (it contains barriers). kind: 0 sum, 1 max, 2 nan-max.
template <int L, int KIND>
__device__ __forceinline__ float group_combine(float v, float* red) {
  if constexpr (L <= kWave) {
    return v;
  } else {
    constexpr int G = L / kWave;
    __syncthreads();  // previous readers of red are done
    if (lane_id() == 0) red[wave_id()] = v;
    __syncthreads();
    const int g0 = (wave_id() / G) * G;
    float r = red[g0];
#pragma unroll
    for (int i = 1; i < G; ++i) {
      float o = red[g0 + i];
      if constexpr (KIND == 0) r += o;
      else if constexpr (KIND == 1) r = fmaxf(r, o);
      else r = nan_max(r, o);
    }
    return r;
  }
}

template <int L, int KIND>
__device__ __forceinline__ float group_reduce(float v, float* red) {
  if constexpr (KIND == 0) v = seg_sum<L>(v);
  else if constexpr (KIND == 1) v = seg_max<L>(v);
  else v = seg_nan_max<L>(v);
  return group_combine<L, KIND>(v, red);
}

// Launch geometry of a row-cached kernel with L lanes per row.
template <int L>
struct RowGeom {
  static constexpr int kWPB = (L / kWave) > 4 ? (L / kWave) : 4;  // waves per block
  static constexpr int kThreads = kWPB * kWave;
  static constexpr int kRowsPerBlock = kThreads / L;
  // lane index inside the row group and the block-local group index
  __device__ __forceinline__ static int lane_in_row() { return threadIdx.x % L; }
  __device__ __forceinline__ static int group() { return threadIdx.x / L; }
};

// A row cached in fp32 registers: f[j * kVec + e] is element (lane + j * L) * kVec + e.
template <typename T, int L, int VPT>
struct RowRegs {
  static constexpr int kE = VPT * T::kVec;
  float f[kE];

  __device__ __forceinline__ static bool valid(int j, int gl, int nvec) { return gl + j * L < nvec; }

  __device__ __forceinline__ void load(const typename T::S* row, int nvec, int gl) {
#pragma unroll
    for (int j = 0; j < VPT; ++j) {
      const int idx = gl + j * L;
      u32x4 v = {0u, 0u, 0u, 0u};
      if (idx < nvec) v = ld16(row + (int64_t)idx * T::kVec);
#pragma unroll
      for (int e = 0; e < T::kVec; ++e) f[j * T::kVec + e] = T::lane_elem(v, e);
    }
  }
  // Load a per-column vector (weights) with the same lane mapping.
  __device__ __forceinline__ void load_cols(const typename T::S* w, int nvec, int gl) { load(w, nvec, gl); }

  // nt: nontemporal stores (outputs far larger than what a consumer could find in cache)
  __device__ __forceinline__ void store(typename T::S* row, int nvec, int gl, bool nt = false) const {
#pragma unroll
    for (int j = 0; j < VPT; ++j) {
      const int idx = gl + j * L;
      if (idx < nvec) {
        u32x4 v;
#pragma unroll
        for (int e = 0; e < T::kVec; ++e) T::set_elem(v, e, f[j * T::kVec + e]);
        if (nt) st16_stream(row + (int64_t)idx * T::kVec, v);
        else st16(row + (int64_t)idx * T::kVec, v);
      }
    }
  }
};

// Host-side choice of (L, VPT) for a row of `nvec` 16-byte vectors: about `want` vectors per lane
// (measured on MI355X, cold cache: rmsnorm f16 4096x4096 15.1 us with 4 per lane against 16.6 us
// with 8; softmax f16 8192x8192 43.8 us against 45.5 us; the last-dim sum prefers 2), at most
// 64 fp32 values per lane and 1024 lanes per row. Returns false when the row does not fit.
struct RowPlan {
  int L;
  int vpt;
};
inline int64_t next_pow2(int64_t v) {
  int64_t p = 1;
  while (p < v) p *= 2;
  return p;
}
inline bool plan_row(int64_t nvec, int kvec, RowPlan* p, int want = 4) {
  const int vmax = 64 / kvec;  // 8 for 2-byte types, 16 for fp32
  if (nvec <= kWave) {         // narrow row: a sub-wave segment, one vector per lane
    p->L = (int)(nvec <= 8 ? 8 : next_pow2(nvec));
    p->vpt = 1;
    return true;
  }
  const int tgt = want < vmax ? want : vmax;
  int64_t L = next_pow2(cdiv(nvec, tgt));
  if (L < kWave) L = kWave;
  if (L > 1024) L = 1024;
  const int64_t vpt = next_pow2(cdiv(nvec, L));
  if (vpt > vmax) return false;
  p->L = (int)L;
  p->vpt = (int)vpt;
  return true;
}

}  // namespace ak

// Expand a row-cached kernel launch over the supported (L, VPT) pairs.
//   AK_ROW_SWITCH(plan, L, VPT, { launch<T, L, VPT>(...); })
#define AK_ROW_CASE(Lv, Vv, ...)                              \
  if (plan.L == Lv && plan.vpt == Vv) {                       \
    constexpr int L = Lv;                                     \
    constexpr int VPT = Vv;                                   \
    if constexpr (VPT * T::kVec <= 64) {                      \
      __VA_ARGS__;                                            \
      handled = true;                                         \
    }                                                         \
  }
#define AK_ROW_SWITCH(...)                                                          \
  do {                                                                           \
    AK_ROW_CASE(8, 1, __VA_ARGS__)                                              \
    else AK_ROW_CASE(16, 1, __VA_ARGS__)                                        \
    else AK_ROW_CASE(32, 1, __VA_ARGS__)                                        \
    else AK_ROW_CASE(64, 1, __VA_ARGS__)                                        \
    else AK_ROW_CASE(64, 2, __VA_ARGS__)                                        \
    else AK_ROW_CASE(64, 4, __VA_ARGS__)                                        \
    else AK_ROW_CASE(64, 8, __VA_ARGS__)                                        \
    else AK_ROW_CASE(64, 16, __VA_ARGS__)                                       \
    else AK_ROW_CASE(128, 2, __VA_ARGS__)                                       \
    else AK_ROW_CASE(128, 4, __VA_ARGS__)                                       \
    else AK_ROW_CASE(128, 8, __VA_ARGS__)                                       \
    else AK_ROW_CASE(128, 16, __VA_ARGS__)                                      \
    else AK_ROW_CASE(256, 2, __VA_ARGS__)                                       \
    else AK_ROW_CASE(256, 4, __VA_ARGS__)                                       \
    else AK_ROW_CASE(256, 8, __VA_ARGS__)                                       \
    else AK_ROW_CASE(256, 16, __VA_ARGS__)                                      \
    else AK_ROW_CASE(512, 2, __VA_ARGS__)                                       \
    else AK_ROW_CASE(512, 4, __VA_ARGS__)                                       \
    else AK_ROW_CASE(512, 8, __VA_ARGS__)                                       \
    else AK_ROW_CASE(512, 16, __VA_ARGS__)                                      \
    else AK_ROW_CASE(1024, 2, __VA_ARGS__)                                      \
    else AK_ROW_CASE(1024, 4, __VA_ARGS__)                                      \
    else AK_ROW_CASE(1024, 8, __VA_ARGS__)                                      \
    else AK_ROW_CASE(1024, 16, __VA_ARGS__)                                     \
  } while (0)
