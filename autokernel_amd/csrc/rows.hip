// rows.hip -- row-parallel ops on gfx950: rmsnorm, layernorm, softmax, cross_entropy and the
// last-dim reductions. All are HBM-bound: each row is read once into registers (row_common.h)
// and written once; reductions are wave64 butterflies plus a fixed-order LDS combine.
#include <limits.h>

#include <atomic>
#include <mutex>

#include "row_common.h"

namespace ak {

constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;
constexpr int kLoopThreads = 256;

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// Every wave of a 256-thread block calls this; kind as in group_combine.
template <int KIND>
__device__ __forceinline__ float block_reduce(float v, float* red) {
  return group_reduce<kLoopThreads, KIND>(v, red);
}

// =============================================================================================
// RMSNorm. Op sequence of reference.py:28-29, each a tensor op in x's dtype:
//   sq = x**2; ms = mean(sq); t = ms + eps; rms = sqrt(t); q = x / rms; y = q * weight
// so x*x rounds (and may overflow to inf) in f16 before the fp32-accumulated mean.
// =============================================================================================
// FORM 0: reference.py:28-29, y = (x / sqrt(mean(x^2) + eps)) * w.
// FORM 1: a LLaMA block's module (models/llama_7b.py:28-30), y = x * rsqrt(mean(x^2) + eps) * w,
// where rsqrt's result is itself a tensor rounded to the element type.
template <typename T, int FORM>
struct RmsStats {
  // the factor each x is multiplied by before its rounding
  __device__ __forceinline__ static float scale(float ss, int cols, float eps) {
    const float ms = T::rnd(ss / (float)cols);
    const float t = T::rnd(ms + eps);
    if constexpr (FORM == 0) return 1.0f / T::rnd(sqrtf(t));  // x / rms to within one fp32 ulp
    else return T::rnd(1.0f / sqrtf(t));
  }
};

template <typename T, int L, int VPT, int FORM>
__global__ __launch_bounds__(RowGeom<L>::kThreads) void rmsnorm_rows(
    const typename T::S* __restrict__ x, const typename T::S* __restrict__ w,
    typename T::S* __restrict__ y, int64_t rows, int cols, float eps) {
  using G = RowGeom<L>;
  __shared__ float red[G::kWPB];
  const int gl = G::lane_in_row();
  const int64_t row = (int64_t)blockIdx.x * G::kRowsPerBlock + G::group();
  const bool active = row < rows;
  const int nvec = active ? cols / T::kVec : 0;
  RowRegs<T, L, VPT> r;
  r.load(x + row * cols, nvec, gl);
  float ss = 0.f;
#pragma unroll
  for (int e = 0; e < RowRegs<T, L, VPT>::kE; ++e) ss += T::rnd(r.f[e] * r.f[e]);
  ss = group_reduce<L, 0>(ss, red);
  const float inv = RmsStats<T, FORM>::scale(ss, cols, eps);
#pragma unroll
  for (int j = 0; j < VPT; ++j) {
    const int idx = gl + j * L;
    if (idx < nvec) {
      // weights load here, after the reduction (measured faster than issuing them with the row:
      // 14.8 against 15.8 us for f16 4096x4096)
      const u32x4 wv = ld16(w + (int64_t)idx * T::kVec);
      u32x4 o;
#pragma unroll
      for (int e = 0; e < T::kVec; ++e)
        T::set_elem(o, e, T::rnd(r.f[j * T::kVec + e] * inv) * T::lane_elem(wv, e));
      st16(y + row * cols + (int64_t)idx * T::kVec, o);
    }
  }
}

template <typename T, int FORM>
__global__ __launch_bounds__(kLoopThreads) void rmsnorm_loop(
    const typename T::S* __restrict__ x, const typename T::S* __restrict__ w,
    typename T::S* __restrict__ y, int cols, float eps) {
  __shared__ float red[kLoopThreads / kWave];
  const typename T::S* xr = x + (int64_t)blockIdx.x * cols;
  typename T::S* yr = y + (int64_t)blockIdx.x * cols;
  float ss = 0.f;
  for (int c = threadIdx.x; c < cols; c += kLoopThreads) {
    const float v = T::to_f(xr[c]);
    ss += T::rnd(v * v);
  }
  ss = block_reduce<0>(ss, red);
  const float inv = RmsStats<T, FORM>::scale(ss, cols, eps);
  for (int c = threadIdx.x; c < cols; c += kLoopThreads)
    yr[c] = T::from_f(T::rnd(T::to_f(xr[c]) * inv) * T::to_f(w[c]));
}

template <typename T, int FORM>
static int launch_rmsnorm(const void* x, const void* w, void* y, int64_t rows, int64_t cols,
                          float eps, hipStream_t s) {
  using S = typename T::S;
  const S* xp = (const S*)x;
  const S* wp = (const S*)w;
  S* yp = (S*)y;
  RowPlan plan;
  const bool vec = cols % T::kVec == 0 && host_aligned16(x) && host_aligned16(y) && host_aligned16(w);
  bool handled = false;
  if (vec && plan_row(cols / T::kVec, T::kVec, &plan)) {
    AK_ROW_SWITCH({
      const dim3 grid((unsigned)cdiv(rows, RowGeom<L>::kRowsPerBlock));
      rmsnorm_rows<T, L, VPT, FORM><<<grid, RowGeom<L>::kThreads, 0, s>>>(xp, wp, yp, rows, (int)cols, eps);
    });
  }
  if (!handled) rmsnorm_loop<T, FORM><<<(unsigned)rows, kLoopThreads, 0, s>>>(xp, wp, yp, (int)cols, eps);
  return record_launch();
}

// =============================================================================================
// LayerNorm: F.layer_norm over the last dim (reference.py:20-23): fp32 mean and biased variance,
// rstd = rsqrt(var + eps), y = (x - mean) * rstd * w + b rounded once.
// =============================================================================================
template <typename T>
__device__ __forceinline__ float ln_out(float v, float mean, float rstd, const typename T::S* w,
                                        const typename T::S* b, int64_t c) {
  float o = (v - mean) * rstd;
  if (w) o *= T::to_f(w[c]);
  if (b) o += T::to_f(b[c]);
  return o;
}

template <typename T, int L, int VPT>
__global__ __launch_bounds__(RowGeom<L>::kThreads) void layernorm_rows(
    const typename T::S* __restrict__ x, const typename T::S* __restrict__ w,
    const typename T::S* __restrict__ b, typename T::S* __restrict__ y, int64_t rows, int cols,
    float eps) {
  using G = RowGeom<L>;
  using R = RowRegs<T, L, VPT>;
  __shared__ float red[G::kWPB];
  const int gl = G::lane_in_row();
  const int64_t row = (int64_t)blockIdx.x * G::kRowsPerBlock + G::group();
  const bool active = row < rows;
  const int nvec = active ? cols / T::kVec : 0;
  R r;
  r.load(x + row * cols, nvec, gl);
  u32x4 wv[VPT], bv[VPT];  // affine parameters issued with the row, not after the reductions
#pragma unroll
  for (int j = 0; j < VPT; ++j) {
    const int idx = gl + j * L;
    wv[j] = (w && idx < nvec) ? ld16(w + (int64_t)idx * T::kVec) : u32x4{0u, 0u, 0u, 0u};
    bv[j] = (b && idx < nvec) ? ld16(b + (int64_t)idx * T::kVec) : u32x4{0u, 0u, 0u, 0u};
  }
  float s = 0.f;
#pragma unroll
  for (int e = 0; e < R::kE; ++e) s += r.f[e];  // invalid vectors hold 0
  const float mean = group_reduce<L, 0>(s, red) / (float)cols;
  float d = 0.f;
#pragma unroll
  for (int j = 0; j < VPT; ++j) {
    if (R::valid(j, gl, nvec)) {
#pragma unroll
      for (int e = 0; e < T::kVec; ++e) {
        const float t = r.f[j * T::kVec + e] - mean;
        d += t * t;
      }
    }
  }
  const float var = group_reduce<L, 0>(d, red) / (float)cols;
  const float rstd = rsqrtf(var + eps);
#pragma unroll
  for (int j = 0; j < VPT; ++j) {
    const int idx = gl + j * L;
    if (idx < nvec) {
      u32x4 o;
#pragma unroll
      for (int e = 0; e < T::kVec; ++e) {
        float v = (r.f[j * T::kVec + e] - mean) * rstd;
        if (w) v *= T::lane_elem(wv[j], e);
        if (b) v += T::lane_elem(bv[j], e);
        T::set_elem(o, e, v);
      }
      st16(y + row * cols + (int64_t)idx * T::kVec, o);
    }
  }
}

template <typename T>
__global__ __launch_bounds__(kLoopThreads) void layernorm_loop(
    const typename T::S* __restrict__ x, const typename T::S* __restrict__ w,
    const typename T::S* __restrict__ b, typename T::S* __restrict__ y, int cols, float eps) {
  __shared__ float red[kLoopThreads / kWave];
  const typename T::S* xr = x + (int64_t)blockIdx.x * cols;
  typename T::S* yr = y + (int64_t)blockIdx.x * cols;
  float s = 0.f;
  for (int c = threadIdx.x; c < cols; c += kLoopThreads) s += T::to_f(xr[c]);
  const float mean = block_reduce<0>(s, red) / (float)cols;
  float d = 0.f;
  for (int c = threadIdx.x; c < cols; c += kLoopThreads) {
    const float t = T::to_f(xr[c]) - mean;
    d += t * t;
  }
  const float rstd = rsqrtf(block_reduce<0>(d, red) / (float)cols + eps);
  for (int c = threadIdx.x; c < cols; c += kLoopThreads)
    yr[c] = T::from_f(ln_out<T>(T::to_f(xr[c]), mean, rstd, w, b, c));
}

template <typename T>
static int launch_layernorm(const void* x, const void* w, const void* b, void* y, int64_t rows,
                            int64_t cols, float eps, hipStream_t s) {
  using S = typename T::S;
  const S* xp = (const S*)x;
  const S* wp = (const S*)w;
  const S* bp = (const S*)b;
  S* yp = (S*)y;
  RowPlan plan;
  const bool vec = cols % T::kVec == 0 && host_aligned16(x) && host_aligned16(y) &&
                   (!w || host_aligned16(w)) && (!b || host_aligned16(b));
  bool handled = false;
  if (vec && plan_row(cols / T::kVec, T::kVec, &plan)) {
    AK_ROW_SWITCH({
      const dim3 grid((unsigned)cdiv(rows, RowGeom<L>::kRowsPerBlock));
      layernorm_rows<T, L, VPT><<<grid, RowGeom<L>::kThreads, 0, s>>>(xp, wp, bp, yp, rows, (int)cols, eps);
    });
  }
  if (!handled) layernorm_loop<T><<<(unsigned)rows, kLoopThreads, 0, s>>>(xp, wp, bp, yp, (int)cols, eps);
  return record_launch();
}

// =============================================================================================
// Softmax over the last dim (reference.py:15-17): fp32 max, exp and sum, one rounding.
// =============================================================================================
template <typename T, int L, int VPT>
__global__ __launch_bounds__(RowGeom<L>::kThreads) void softmax_rows(
    const typename T::S* __restrict__ x, typename T::S* __restrict__ y, int64_t rows, int cols, int nt_out) {
  using G = RowGeom<L>;
  using R = RowRegs<T, L, VPT>;
  __shared__ float red[G::kWPB];
  const int gl = G::lane_in_row();
  const int64_t row = (int64_t)blockIdx.x * G::kRowsPerBlock + G::group();
  const bool active = row < rows;
  const int nvec = active ? cols / T::kVec : 0;
  R r;
  r.load(x + row * cols, nvec, gl);
  float m = -INFINITY;
#pragma unroll
  for (int j = 0; j < VPT; ++j)
    if (R::valid(j, gl, nvec))
#pragma unroll
      for (int e = 0; e < T::kVec; ++e) m = fmaxf(m, r.f[j * T::kVec + e]);
  m = group_reduce<L, 1>(m, red);
  const float mb = m * kLog2e;
  float s = 0.f;
#pragma unroll
  for (int j = 0; j < VPT; ++j) {
    if (R::valid(j, gl, nvec)) {
#pragma unroll
      for (int e = 0; e < T::kVec; ++e) {
        const float p = fast_exp2(__builtin_fmaf(r.f[j * T::kVec + e], kLog2e, -mb));
        r.f[j * T::kVec + e] = p;
        s += p;
      }
    }
  }
  s = group_reduce<L, 0>(s, red);
  const float inv = 1.0f / s;
#pragma unroll
  for (int e = 0; e < R::kE; ++e) r.f[e] *= inv;
  r.store(y + row * cols, nvec, gl, nt_out != 0);
}

// Online (max, sum-of-exp) accumulator used by the looped softmax and cross-entropy kernels.
// -inf entries contribute nothing, +inf or NaN entries make the sum NaN (torch's softmax result).
struct OnlineMS {
  float m = -INFINITY;
  float s = 0.f;
  bool nan = false;
  __device__ __forceinline__ void add(float v) {
    if (v != v) { nan = true; return; }
    const float mn = fmaxf(m, v);
    if (mn == -INFINITY) return;
    s = s * fast_exp2((m - mn) * kLog2e) + fast_exp2((v - mn) * kLog2e);
    m = mn;
  }
};

// Combine per-thread (m, s) over a 256-thread block in fixed order; returns the row's (M, S).
__device__ __forceinline__ void block_combine_ms(OnlineMS a, float* red, float* M, float* S) {
  float mx = block_reduce<1>(a.m, red);
  float sc = (a.m == -INFINITY) ? 0.f : a.s * fast_exp2((a.m - mx) * kLog2e);
  if (a.nan) sc = NAN;
  float tot = block_reduce<0>(sc, red);
  *M = mx;
  *S = tot;
}

// Wide rows that do not vectorise (a width that is not a multiple of the 16-byte vector, e.g. a
// 50257-entry vocabulary): one row per block of 1024 threads, element c = tid + 1024 k cached in
// registers (EPT per thread, so x is read once), with the vector path's arithmetic.
// Rows are addressed through a buffer resource spanning the row (gfx9 descriptor word 3 =
// 0x00020000, raw 32-bit data format, stride 0, num_records = the row's bytes): element c is one
// per-thread VGPR offset plus a uniform scalar offset, where 64-bit pointers would take two VGPRs
// per element and spill at this many elements per thread.
constexpr int kWideThreads = 1024;

__device__ __forceinline__ __amdgpu_buffer_rsrc_t row_rsrc(const void* row, int bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(row), (short)0, bytes, 0x00020000);
}
__device__ __forceinline__ void buf_ld(__amdgpu_buffer_rsrc_t r, int voff, int soff, uint16_t& v) {
  v = __builtin_amdgcn_raw_buffer_load_b16(r, voff, soff, 0);
}
__device__ __forceinline__ void buf_ld(__amdgpu_buffer_rsrc_t r, int voff, int soff, float& v) {
  v = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(r, voff, soff, 0));
}
__device__ __forceinline__ void buf_st(__amdgpu_buffer_rsrc_t r, int voff, int soff, uint16_t v) {
  __builtin_amdgcn_raw_buffer_store_b16(v, r, voff, soff, 0);
}
__device__ __forceinline__ void buf_st(__amdgpu_buffer_rsrc_t r, int voff, int soff, float v) {
  __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(uint32_t, v), r, voff, soff, 0);
}

// Loads this thread's EPT elements of the row (c = tid + 1024 k, c < cols) into v and returns
// their maximum (-inf for a thread with none). Every load is issued before the first use so all
// of them are in flight together, with no branch: a thread past the row's end re-reads element
// cols - 1 (so every access stays in the row; a wave's such loads share one cache line) and takes
// -inf by a select.
template <typename T, int EPT>
__device__ __forceinline__ float wide_load_max(const typename T::S* xr, int cols, float (&v)[EPT]) {
  using S = typename T::S;
  const __amdgpu_buffer_rsrc_t r = row_rsrc(xr, cols * (int)sizeof(S));
  S e[EPT];
#pragma unroll
  for (int k = 0; k < EPT; ++k)
    buf_ld(r, min((int)threadIdx.x + k * kWideThreads, cols - 1) * (int)sizeof(S), 0, e[k]);
  float m = -INFINITY;
#pragma unroll
  for (int k = 0; k < EPT; ++k) {
    v[k] = (int)threadIdx.x + k * kWideThreads < cols ? T::to_f(e[k]) : -INFINITY;
    m = fmaxf(m, v[k]);
  }
  return m;
}

template <typename T, int EPT>
__global__ __launch_bounds__(kWideThreads) void softmax_wide(const typename T::S* __restrict__ x,
                                                             typename T::S* __restrict__ y, int cols) {
  __shared__ float red[kWideThreads / kWave];
  const int64_t base = (int64_t)blockIdx.x * cols;
  float v[EPT];
  float m = group_reduce<kWideThreads, 1>(wide_load_max<T, EPT>(x + base, cols, v), red);
  const float mb = m * kLog2e;
  // p is recomputed in the write pass rather than kept (the same expression, so the same value):
  // holding both x and p would spill at 64 elements per thread.
  float s = 0.f;
#pragma unroll
  for (int k = 0; k < EPT; ++k)
    if (threadIdx.x + k * kWideThreads < cols) s += fast_exp2(__builtin_fmaf(v[k], kLog2e, -mb));
  s = group_reduce<kWideThreads, 0>(s, red);
  const float inv = 1.0f / s;
  using S = typename T::S;
  const __amdgpu_buffer_rsrc_t r = row_rsrc(y + base, cols * (int)sizeof(S));
  const int voff = threadIdx.x * (int)sizeof(S);
#pragma unroll
  for (int k = 0; k < EPT; ++k)
    if (threadIdx.x + k * kWideThreads < cols)
      buf_st(r, voff, k * kWideThreads * (int)sizeof(S), T::from_f(fast_exp2(__builtin_fmaf(v[k], kLog2e, -mb)) * inv));
}

// Wide 16-bit rows of any width and alignment, held packed: one row per 1024-thread block with the
// row's elements kept two per VGPR, as the 4-byte pairs memory already stores them. A block needs
// about half the registers of softmax_wide, so two rows are in flight per CU (one block's
// reductions and stores overlap the other's loads). Pair k of thread t is the aligned dword at
// element par + 2 (t + 1024 k) of the row, par = 1 when the row's first element is the high half
// of a dword (odd widths put every other row there). The element left at either end (the first
// when par = 1, the last when cols - par is odd) is one extra value held by thread 0 (first) or 1
// (last). Pairs past the row's end come back as zeros from the buffer's range check and are
// masked by index. The whole byte offset of a load is its VGPR offset: on gfx9 the range check
// covers the VGPR and instruction offsets, not the scalar offset, so a per-k scalar offset would let
// reads run past the row (and, on a tensor's last row, past its allocation). Requires the output
// rows to share the input rows' dword alignment.
template <typename T, int NP>
struct WidePairs {
  uint32_t p[NP];
  float xt;  // thread 0: the first element when par = 1; thread 1: the last when cols - par is odd
  bool has_xt;
  int npairs, par;

  __device__ __forceinline__ static float lo(uint32_t w) { return T::to_f((uint16_t)(w & 0xffffu)); }
  __device__ __forceinline__ static float hi(uint32_t w) { return T::to_f((uint16_t)(w >> 16)); }
  __device__ __forceinline__ bool valid(int k) const { return (int)threadIdx.x + k * kWideThreads < npairs; }

  // loads the row; returns this thread's maximum (-inf when it holds nothing)
  __device__ __forceinline__ float load_max(const uint16_t* row, int cols) {
    par = (int)(((uintptr_t)row >> 1) & 1u);
    npairs = (cols - par) >> 1;
    const __amdgpu_buffer_rsrc_t r = row_rsrc(row + par, npairs * 4);
#pragma unroll
    for (int k = 0; k < NP; ++k)
      p[k] = __builtin_amdgcn_raw_buffer_load_b32(r, ((int)threadIdx.x + k * kWideThreads) * 4, 0, 0);
    has_xt = (threadIdx.x == 0 && par) || (threadIdx.x == 1 && ((cols - par) & 1));
    xt = has_xt ? T::to_f(row[threadIdx.x == 0 ? 0 : cols - 1]) : -INFINITY;
    float m = xt;
#pragma unroll
    for (int k = 0; k < NP; ++k)
      if (valid(k)) m = fmaxf(m, fmaxf(lo(p[k]), hi(p[k])));
    return m;
  }
  // sum of f(x) over the thread's elements
  template <typename F>
  __device__ __forceinline__ float sum(F f) const {
    float s = has_xt ? f(xt) : 0.f;
#pragma unroll
    for (int k = 0; k < NP; ++k)
      if (valid(k)) s += f(lo(p[k])) + f(hi(p[k]));
    return s;
  }
};

template <typename T, int NP>
__global__ __launch_bounds__(kWideThreads, 2) void softmax_wide_pairs(const uint16_t* __restrict__ x,
                                                                     uint16_t* __restrict__ y, int cols) {
  __shared__ float red[kWideThreads / kWave];
  const int64_t base = (int64_t)blockIdx.x * cols;
  WidePairs<T, NP> w;
  const float m = group_reduce<kWideThreads, 1>(w.load_max(x + base, cols), red);
  const float mb = m * kLog2e;
  auto e = [&](float v) { return fast_exp2(__builtin_fmaf(v, kLog2e, -mb)); };
  const float s = group_reduce<kWideThreads, 0>(w.sum(e), red);
  const float inv = 1.0f / s;
  uint16_t* yr = y + base;
  const __amdgpu_buffer_rsrc_t r = row_rsrc(yr + w.par, w.npairs * 4);
#pragma unroll
  for (int k = 0; k < NP; ++k)
    if (w.valid(k)) {
      const uint32_t o = (uint32_t)T::from_f(e(w.lo(w.p[k])) * inv) | ((uint32_t)T::from_f(e(w.hi(w.p[k])) * inv) << 16);
      __builtin_amdgcn_raw_buffer_store_b32(o, r, (int)threadIdx.x * 4, k * kWideThreads * 4, 0);
    }
  if (w.has_xt) yr[threadIdx.x == 0 ? 0 : cols - 1] = T::from_f(e(w.xt) * inv);
}

// Streaming row statistics for 16-bit rows that do not vectorise (softmax_stream, ce_stream): one
// row per 256-thread block, read once as aligned dword pairs (the WidePairs layout) with an online
// (max, sum) per thread and 8 pairs in flight per thread. Nothing is cached in registers, so up to
// eight rows are in flight per CU. Per chunk of 16 elements: the chunk max (NaN-propagating), one
// rescale of the running sum, then exp2((x - max) log2 e) per element; the per-thread (max, sum)
// pairs combine in a fixed order (block_combine_ms), as in the looped kernels.
constexpr int kStreamUnroll = 8;
template <typename T>
__device__ __forceinline__ void stream_ms(const uint16_t* xr, int cols, float* red, float* M, float* S) {
  const int par = (int)(((uintptr_t)xr >> 1) & 1u);
  const int npairs = (cols - par) >> 1;
  const __amdgpu_buffer_rsrc_t r = row_rsrc(xr + par, npairs * 4);
  float m = -INFINITY, s = 0.f;
  // fold a chunk with maximum cm and values v[0..n) into (m, s)
  auto fold = [&](float cm, auto&& each) {
    const float mn = __builtin_elementwise_maximum(m, cm);
    if (mn == -INFINITY) return;  // nothing but -inf so far
    s = (m == -INFINITY) ? 0.f : s * fast_exp2((m - mn) * kLog2e);
    each([&](float v) { s += fast_exp2((v - mn) * kLog2e); });
    m = mn;
  };
  if ((threadIdx.x == 0 && par) || (threadIdx.x == 1 && ((cols - par) & 1))) {
    const float v = T::to_f(xr[threadIdx.x == 0 ? 0 : cols - 1]);
    fold(v, [&](auto&& f) { f(v); });
  }
  for (int b = 0; b < npairs; b += kLoopThreads * kStreamUnroll) {
    uint32_t p[kStreamUnroll];
#pragma unroll
    for (int u = 0; u < kStreamUnroll; ++u)
      p[u] = __builtin_amdgcn_raw_buffer_load_b32(r, ((int)threadIdx.x + b + u * kLoopThreads) * 4, 0, 0);
    float cm = -INFINITY;
#pragma unroll
    for (int u = 0; u < kStreamUnroll; ++u)
      if (b + u * kLoopThreads + (int)threadIdx.x < npairs)
        cm = __builtin_elementwise_maximum(cm, __builtin_elementwise_maximum(WidePairs<T, 1>::lo(p[u]), WidePairs<T, 1>::hi(p[u])));
    fold(cm, [&](auto&& f) {
#pragma unroll
      for (int u = 0; u < kStreamUnroll; ++u)
        if (b + u * kLoopThreads + (int)threadIdx.x < npairs) {
          f(WidePairs<T, 1>::lo(p[u]));
          f(WidePairs<T, 1>::hi(p[u]));
        }
    });
  }
  OnlineMS a;
  a.m = m;
  a.s = s;
  a.nan = (m != m);
  block_combine_ms(a, red, M, S);
}

// Streaming softmax for 16-bit rows: the online pass above, then a second read of the row (from
// the caches when they still hold it) that writes exp2((x - M) log2 e) / S as dword pairs.
template <typename T>
__global__ __launch_bounds__(kLoopThreads) void softmax_stream(const uint16_t* __restrict__ x,
                                                               uint16_t* __restrict__ y, int cols) {
  __shared__ float red[kLoopThreads / kWave];
  const int64_t base = (int64_t)blockIdx.x * cols;
  const uint16_t* xr = x + base;
  uint16_t* yr = y + base;
  float M, S;
  stream_ms<T>(xr, cols, red, &M, &S);
  const float inv = 1.0f / S;
  auto e = [&](float v) { return T::from_f(fast_exp2((v - M) * kLog2e) * inv); };
  const int par = (int)(((uintptr_t)xr >> 1) & 1u);
  const int npairs = (cols - par) >> 1;
  const __amdgpu_buffer_rsrc_t r = row_rsrc(xr + par, npairs * 4);
  const __amdgpu_buffer_rsrc_t w = row_rsrc(yr + par, npairs * 4);
  if ((threadIdx.x == 0 && par) || (threadIdx.x == 1 && ((cols - par) & 1))) {
    const int c = threadIdx.x == 0 ? 0 : cols - 1;
    yr[c] = e(T::to_f(xr[c]));
  }
  for (int b = 0; b < npairs; b += kLoopThreads * kStreamUnroll) {
    uint32_t p[kStreamUnroll];
#pragma unroll
    for (int u = 0; u < kStreamUnroll; ++u)
      p[u] = __builtin_amdgcn_raw_buffer_load_b32(r, ((int)threadIdx.x + b + u * kLoopThreads) * 4, 0, 0);
#pragma unroll
    for (int u = 0; u < kStreamUnroll; ++u)
      if (b + u * kLoopThreads + (int)threadIdx.x < npairs) {
        const uint32_t o = (uint32_t)e(WidePairs<T, 1>::lo(p[u])) | ((uint32_t)e(WidePairs<T, 1>::hi(p[u])) << 16);
        __builtin_amdgcn_raw_buffer_store_b32(o, w, (int)threadIdx.x * 4, (b + u * kLoopThreads) * 4, 0);
      }
  }
}

template <typename T>
__global__ __launch_bounds__(kLoopThreads) void softmax_loop(
    const typename T::S* __restrict__ x, typename T::S* __restrict__ y, int cols) {
  __shared__ float red[kLoopThreads / kWave];
  const typename T::S* xr = x + (int64_t)blockIdx.x * cols;
  typename T::S* yr = y + (int64_t)blockIdx.x * cols;
  OnlineMS a;
  for (int c = threadIdx.x; c < cols; c += kLoopThreads) a.add(T::to_f(xr[c]));
  float M, S;
  block_combine_ms(a, red, &M, &S);
  // The write pass uses the online pass's exponent form, (x - M) log2 e. The fused form
  // x log2 e - round(M log2 e) of the cached kernels would shift every exponent by the rounding of
  // M log2 e (0.008 at |M| ~ 1e5), a scale that S, summed in the other form, does not share.
  const float inv = 1.0f / S;
  for (int c = threadIdx.x; c < cols; c += kLoopThreads)
    yr[c] = T::from_f(fast_exp2((T::to_f(xr[c]) - M) * kLog2e) * inv);
}

template <typename T>
static int launch_softmax(const void* x, void* y, int64_t rows, int64_t cols, hipStream_t s) {
  using S = typename T::S;
  const S* xp = (const S*)x;
  S* yp = (S*)y;
  RowPlan plan;
  const bool vec = cols % T::kVec == 0 && host_aligned16(x) && host_aligned16(y);
  bool handled = false;
  // An output larger than the 256 MB Infinity Cache is stored nontemporally; smaller outputs keep
  // plain stores, so the consumer that usually reads them next finds them in cache. Measured, f16
  // [8192, 8192] (128 MiB), cold, softmax then a consumer of its output: with a reduce sum 62.9 us
  // plain against 69.7 us nontemporal, with a [8192, 8192] x [8192, 128] product 88.2 against
  // 89.5 us. Nontemporal stores win only for back-to-back softmax calls whose outputs nobody reads
  // (the dirty lines' write-back then lands in the next kernel): 56.3 against 67.3 us per
  // RoPE(q), RoPE(k), softmax step.
  const int nt_out = rows * cols * (int64_t)sizeof(S) > ((int64_t)256 << 20);
  if (vec && plan_row(cols / T::kVec, T::kVec, &plan)) {
    AK_ROW_SWITCH({
      const dim3 grid((unsigned)cdiv(rows, RowGeom<L>::kRowsPerBlock));
      launch_timed(softmax_rows<T, L, VPT>, grid, dim3(RowGeom<L>::kThreads), 0, s, xp, yp, rows, (int)cols, nt_out);
    });
  }
  // 16-bit rows that do not vectorise, when x and y rows share their dword alignment: the streaming
  // kernel up to 32768 columns and past 65536, the packed register-cached one in between (measured,
  // f16, 4096 rows: 16385 columns 67.0 us streaming / 99.3 us packed; 24577: 101 / 115; 32769: 138 /
  // 136; 40961: 182 / 152; 50257: 230 / 180 (the fp32-cached kernel: 234.9)).
  if constexpr (sizeof(S) == 2) {
    if (!handled && cols > 4096 && ((((uintptr_t)x ^ (uintptr_t)y) & 3u) == 0)) {
      const uint16_t* xs = (const uint16_t*)x;
      uint16_t* ys = (uint16_t*)y;
      if (cols > 32768 && cols <= 64 * kWideThreads)
        launch_timed(softmax_wide_pairs<T, 32>, dim3((unsigned)rows), dim3(kWideThreads), 0, s, xs, ys, (int)cols);
      else
        launch_timed(softmax_stream<T>, dim3((unsigned)rows), dim3(kLoopThreads), 0, s, xs, ys, (int)cols);
      handled = true;
    }
  }
  if (!handled && cols > 4096 && cols <= 16 * kWideThreads) {
    launch_timed(softmax_wide<T, 16>, dim3((unsigned)rows), dim3(kWideThreads), 0, s, xp, yp, (int)cols);
    handled = true;
  } else if (!handled && cols > 16 * kWideThreads && cols <= 64 * kWideThreads) {
    launch_timed(softmax_wide<T, 64>, dim3((unsigned)rows), dim3(kWideThreads), 0, s, xp, yp, (int)cols);
    handled = true;
  }
  if (!handled) launch_timed(softmax_loop<T>, dim3((unsigned)rows), dim3(kLoopThreads), 0, s, xp, yp, (int)cols);
  return record_launch();
}

// =============================================================================================
// Cross entropy (reference.py:58-60 = F.cross_entropy, mean reduction, ignore_index):
//   log_softmax in fp32 rounded to the logits' dtype, nll = -logp[target], then the mean of the
//   rounded values accumulated in fp32 and rounded once. Per-row losses go to a caller-owned
//   fp32 workspace; a single-block kernel then reduces them in a fixed order.
// =============================================================================================
template <typename T>
__device__ __forceinline__ float ce_row_loss(const typename T::S* xr, int64_t t, int64_t vocab,
                                             int64_t ignore_index, float M, float S) {
  if (t == ignore_index) return 0.f;
  if (t < 0 || t >= vocab) return NAN;
  const float lp = T::rnd(T::to_f(xr[t]) - M - logf(S));
  return -lp;
}

// The same loss for a sum taken as s = sum 2^(x log2 e - mb), mb = round(M log2 e): the target's
// exponent is formed the same way, so the rounding of mb (a factor 2^-eps in s) cancels in
// lp = (x_t log2 e - mb) ln 2 - log s. Subtracting M directly would leave eps ln 2 in the loss
// (5e-3 at |M| ~ 1e5).
template <typename T>
__device__ __forceinline__ float ce_row_loss_b2(const typename T::S* xr, int64_t t, int64_t vocab,
                                                int64_t ignore_index, float mb, float s) {
  if (t == ignore_index) return 0.f;
  if (t < 0 || t >= vocab) return NAN;
  const float lp = T::rnd(__builtin_fmaf(T::to_f(xr[t]), kLog2e, -mb) * kLn2 - logf(s));
  return -lp;
}

template <typename T, int L, int VPT>
__global__ __launch_bounds__(RowGeom<L>::kThreads) void ce_rows(
    const typename T::S* __restrict__ x, const int64_t* __restrict__ tgt, float* __restrict__ loss,
    int64_t rows, int cols, int64_t ignore_index) {
  using G = RowGeom<L>;
  using R = RowRegs<T, L, VPT>;
  __shared__ float red[G::kWPB];
  const int gl = G::lane_in_row();
  const int64_t row = (int64_t)blockIdx.x * G::kRowsPerBlock + G::group();
  const bool active = row < rows;
  const int nvec = active ? cols / T::kVec : 0;
  R r;
  r.load(x + row * cols, nvec, gl);
  float m = -INFINITY;
#pragma unroll
  for (int j = 0; j < VPT; ++j)
    if (R::valid(j, gl, nvec))
#pragma unroll
      for (int e = 0; e < T::kVec; ++e) m = fmaxf(m, r.f[j * T::kVec + e]);
  m = group_reduce<L, 1>(m, red);
  const float mb = m * kLog2e;
  float s = 0.f;
#pragma unroll
  for (int j = 0; j < VPT; ++j)
    if (R::valid(j, gl, nvec))
#pragma unroll
      for (int e = 0; e < T::kVec; ++e) s += fast_exp2(__builtin_fmaf(r.f[j * T::kVec + e], kLog2e, -mb));
  s = group_reduce<L, 0>(s, red);
  if (active && gl == 0) loss[row] = ce_row_loss_b2<T>(x + row * cols, tgt[row], cols, ignore_index, mb, s);
}

template <typename T, int EPT>
__global__ __launch_bounds__(kWideThreads) void ce_wide(const typename T::S* __restrict__ x,
                                                        const int64_t* __restrict__ tgt, float* __restrict__ loss,
                                                        int cols, int64_t ignore_index) {
  __shared__ float red[kWideThreads / kWave];
  const typename T::S* xr = x + (int64_t)blockIdx.x * cols;
  float v[EPT];
  const float m = group_reduce<kWideThreads, 1>(wide_load_max<T, EPT>(xr, cols, v), red);
  const float mb = m * kLog2e;
  float s = 0.f;
#pragma unroll
  for (int k = 0; k < EPT; ++k)
    if (threadIdx.x + k * kWideThreads < cols) s += fast_exp2(__builtin_fmaf(v[k], kLog2e, -mb));
  s = group_reduce<kWideThreads, 0>(s, red);
  if (threadIdx.x == 0) loss[blockIdx.x] = ce_row_loss_b2<T>(xr, tgt[blockIdx.x], cols, ignore_index, mb, s);
}

// Cross-entropy of a 16-bit row from the streaming statistics: loss = x_t - M - log S, as in ce_loop.
template <typename T>
__global__ __launch_bounds__(kLoopThreads) void ce_stream(const uint16_t* __restrict__ x,
                                                          const int64_t* __restrict__ tgt,
                                                          float* __restrict__ loss, int cols,
                                                          int64_t ignore_index) {
  __shared__ float red[kLoopThreads / kWave];
  const uint16_t* xr = x + (int64_t)blockIdx.x * cols;
  float M, S;
  stream_ms<T>(xr, cols, red, &M, &S);
  if (threadIdx.x == 0) loss[blockIdx.x] = ce_row_loss<T>(xr, tgt[blockIdx.x], cols, ignore_index, M, S);
}

template <typename T>
__global__ __launch_bounds__(kLoopThreads) void ce_loop(
    const typename T::S* __restrict__ x, const int64_t* __restrict__ tgt, float* __restrict__ loss,
    int cols, int64_t ignore_index) {
  __shared__ float red[kLoopThreads / kWave];
  const typename T::S* xr = x + (int64_t)blockIdx.x * cols;
  OnlineMS a;
  for (int c = threadIdx.x; c < cols; c += kLoopThreads) a.add(T::to_f(xr[c]));
  float M, S;
  block_combine_ms(a, red, &M, &S);
  if (threadIdx.x == 0) loss[blockIdx.x] = ce_row_loss<T>(xr, tgt[blockIdx.x], cols, ignore_index, M, S);
}

constexpr int kMeanThreads = 1024;

template <typename T>
__global__ __launch_bounds__(kMeanThreads) void ce_mean(const float* __restrict__ loss,
                                                        const int64_t* __restrict__ tgt,
                                                        typename T::S* __restrict__ out,
                                                        int64_t rows, int64_t ignore_index) {
  __shared__ float red[kMeanThreads / kWave];
  // Thread t adds rows t, t + 1024, t + 2048, ... in that order. Each pass loads eight rows' target
  // and loss before adding any of them, so the loads overlap (a dependent load per row took 4.2 us
  // for 4096 rows); the order of the additions is the same either way.
  constexpr int U = 8;
  float s = 0.f, n = 0.f;
  for (int64_t r0 = threadIdx.x; r0 < rows; r0 += (int64_t)U * kMeanThreads) {
    int64_t t[U];
    float l[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int64_t r = r0 + (int64_t)u * kMeanThreads;
      t[u] = r < rows ? tgt[r] : ignore_index;
      l[u] = r < rows ? loss[r] : 0.f;
    }
#pragma unroll
    for (int u = 0; u < U; ++u)
      if (t[u] != ignore_index) {
        s += l[u];
        n += 1.f;
      }
  }
  s = group_reduce<kMeanThreads, 0>(s, red);
  n = group_reduce<kMeanThreads, 0>(n, red);
  if (threadIdx.x == 0) out[0] = T::from_f(s / n);
}

template <typename T>
static int launch_ce(const void* logits, const int64_t* tgt, float* loss, void* out, int64_t rows,
                     int64_t vocab, int64_t ignore_index, hipStream_t s) {
  using S = typename T::S;
  const S* xp = (const S*)logits;
  RowPlan plan;
  const bool vec = vocab % T::kVec == 0 && host_aligned16(logits);
  bool handled = rows == 0;  // no rows: only the mean kernel runs (0 / 0 = NaN, as torch gives)
  if (!handled && vec && plan_row(vocab / T::kVec, T::kVec, &plan)) {
    AK_ROW_SWITCH({
      const dim3 grid((unsigned)cdiv(rows, RowGeom<L>::kRowsPerBlock));
      ce_rows<T, L, VPT><<<grid, RowGeom<L>::kThreads, 0, s>>>(xp, tgt, loss, rows, (int)vocab, ignore_index);
    });
  }
  // 16-bit rows that do not vectorise: the streaming kernel at any width past 4096 (measured, f16:
  // 8192 x 50257 152.5 us against 216.1 register-cached packed and 274.1 fp32-cached; 4096 x 16385
  // 33.0 against 80.1). For rows that vectorise the register-cached ce_rows stays faster (4096 x
  // 32000: 51.6 against 57.1 streaming).
  if constexpr (sizeof(S) == 2) {
    if (!handled && vocab > 4096) {
      ce_stream<T><<<(unsigned)rows, kLoopThreads, 0, s>>>((const uint16_t*)logits, tgt, loss, (int)vocab, ignore_index);
      handled = true;
    }
  }
  if (!handled && vocab > 4096 && vocab <= 16 * kWideThreads) {
    ce_wide<T, 16><<<(unsigned)rows, kWideThreads, 0, s>>>(xp, tgt, loss, (int)vocab, ignore_index);
    handled = true;
  } else if (!handled && vocab > 16 * kWideThreads && vocab <= 64 * kWideThreads) {
    ce_wide<T, 64><<<(unsigned)rows, kWideThreads, 0, s>>>(xp, tgt, loss, (int)vocab, ignore_index);
    handled = true;
  }
  if (!handled) ce_loop<T><<<(unsigned)rows, kLoopThreads, 0, s>>>(xp, tgt, loss, (int)vocab, ignore_index);
  ce_mean<T><<<1, kMeanThreads, 0, s>>>(loss, tgt, (S*)out, rows, ignore_index);
  return record_launch();
}

// =============================================================================================
// Last-dim reductions (reduce over a contiguous row): sum with fp32 accumulation rounded once
// (x.sum(-1), reference.py:72-74), max exact with NaN propagation (x.max(-1).values, :76-78).
// =============================================================================================
template <typename T, int L, int VPT, bool MAX>
__global__ __launch_bounds__(RowGeom<L>::kThreads) void reduce_rows(
    const typename T::S* __restrict__ x, typename T::S* __restrict__ y, int64_t rows, int cols) {
  using G = RowGeom<L>;
  using R = RowRegs<T, L, VPT>;
  __shared__ float red[G::kWPB];
  const int gl = G::lane_in_row();
  const int64_t row = (int64_t)blockIdx.x * G::kRowsPerBlock + G::group();
  const bool active = row < rows;
  const int nvec = active ? cols / T::kVec : 0;
  R r;
  r.load(x + row * cols, nvec, gl);
  float a = MAX ? -INFINITY : 0.f;
#pragma unroll
  for (int j = 0; j < VPT; ++j)
    if (R::valid(j, gl, nvec))
#pragma unroll
      for (int e = 0; e < T::kVec; ++e) a = MAX ? nan_max(a, r.f[j * T::kVec + e]) : a + r.f[j * T::kVec + e];
  a = group_reduce<L, MAX ? 2 : 0>(a, red);
  if (active && gl == 0) y[row] = T::from_f(a);
}

template <typename T, bool MAX>
__global__ __launch_bounds__(kLoopThreads) void reduce_loop(const typename T::S* __restrict__ x,
                                                            typename T::S* __restrict__ y, int cols) {
  __shared__ float red[kLoopThreads / kWave];
  const typename T::S* xr = x + (int64_t)blockIdx.x * cols;
  float a = MAX ? -INFINITY : 0.f;
  for (int c = threadIdx.x; c < cols; c += kLoopThreads) {
    const float v = T::to_f(xr[c]);
    a = MAX ? nan_max(a, v) : a + v;
  }
  a = block_reduce<MAX ? 2 : 0>(a, red);
  if (threadIdx.x == 0) y[blockIdx.x] = T::from_f(a);
}

// Reduction over a strided middle dim: x viewed as [outer, reduce, inner], one thread per
// (outer, inner) output; consecutive threads read consecutive inner elements (coalesced).
template <typename T, bool MAX>
__global__ __launch_bounds__(256) void reduce_cols(const typename T::S* __restrict__ x,
                                                   typename T::S* __restrict__ y, int64_t outer,
                                                   int64_t red_n, int64_t inner) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= outer * inner) return;
  const int64_t o = i / inner, c = i % inner;
  const typename T::S* p = x + o * red_n * inner + c;
  float a = MAX ? -INFINITY : 0.f;
  for (int64_t r = 0; r < red_n; ++r) {
    const float v = T::to_f(p[r * inner]);
    a = MAX ? nan_max(a, v) : a + v;
  }
  y[i] = T::from_f(a);
}

template <typename T, bool MAX>
static int launch_reduce(const void* x, void* y, int64_t outer, int64_t red_n, int64_t inner,
                         hipStream_t s) {
  using S = typename T::S;
  const S* xp = (const S*)x;
  S* yp = (S*)y;
  if (inner == 1) {
    const int64_t rows = outer, cols = red_n;
    RowPlan plan;
    const bool vec = cols % T::kVec == 0 && host_aligned16(x);
    bool handled = false;
    if (vec && plan_row(cols / T::kVec, T::kVec, &plan, 2)) {
      AK_ROW_SWITCH({
        const dim3 grid((unsigned)cdiv(rows, RowGeom<L>::kRowsPerBlock));
        reduce_rows<T, L, VPT, MAX><<<grid, RowGeom<L>::kThreads, 0, s>>>(xp, yp, rows, (int)cols);
      });
    }
    if (!handled) reduce_loop<T, MAX><<<(unsigned)rows, kLoopThreads, 0, s>>>(xp, yp, (int)cols);
  } else {
    reduce_cols<T, MAX><<<(unsigned)cdiv(outer * inner, 256), 256, 0, s>>>(xp, yp, outer, red_n, inner);
  }
  return record_launch();
}

}  // namespace ak

using namespace ak;

static bool bad_rows(int64_t rows, int64_t cols) {
  return rows < 0 || cols < 0 || cols > INT_MAX || rows > (int64_t)INT_MAX;
}

extern "C" int ak_rmsnorm(int dtype, const void* x, const void* w, void* y, int64_t rows,
                          int64_t cols, float eps, hipStream_t stream) {
  if (bad_rows(rows, cols)) return AK_EINVAL;
  if (rows == 0 || cols == 0) return AK_OK;
  if (!x || !w || !y) return AK_EINVAL;
  AK_DISPATCH(dtype, T, return launch_rmsnorm<T, 0>(x, w, y, rows, cols, eps, stream));
}

extern "C" int ak_rmsnorm_rsqrt(int dtype, const void* x, const void* w, void* y, int64_t rows,
                                int64_t cols, float eps, hipStream_t stream) {
  if (bad_rows(rows, cols)) return AK_EINVAL;
  if (rows == 0 || cols == 0) return AK_OK;
  if (!x || !w || !y) return AK_EINVAL;
  AK_DISPATCH(dtype, T, return launch_rmsnorm<T, 1>(x, w, y, rows, cols, eps, stream));
}

extern "C" int ak_layernorm(int dtype, const void* x, const void* w, const void* b, void* y,
                            int64_t rows, int64_t cols, float eps, hipStream_t stream) {
  if (bad_rows(rows, cols)) return AK_EINVAL;
  if (rows == 0 || cols == 0) return AK_OK;
  if (!x || !y) return AK_EINVAL;
  AK_DISPATCH(dtype, T, return launch_layernorm<T>(x, w, b, y, rows, cols, eps, stream));
}

extern "C" int ak_softmax(int dtype, const void* x, void* y, int64_t rows, int64_t cols,
                          hipStream_t stream) {
  // a call that launches nothing still consumes pending launch events (they never carry over)
  const bool launches = !bad_rows(rows, cols) && rows != 0 && cols != 0 && x && y &&
                        (dtype == AK_F32 || dtype == AK_F16 || dtype == AK_BF16);
  if (!launches) take_launch_events();
  if (bad_rows(rows, cols)) return AK_EINVAL;
  if (rows == 0 || cols == 0) return AK_OK;
  if (!x || !y) return AK_EINVAL;
  AK_DISPATCH(dtype, T, return launch_softmax<T>(x, y, rows, cols, stream));
}

extern "C" int ak_cross_entropy(int dtype, const void* logits, const int64_t* targets,
                                float* row_loss, void* out, int64_t rows, int64_t vocab,
                                int64_t ignore_index, hipStream_t stream) {
  if (bad_rows(rows, vocab)) return AK_EINVAL;
  if (!out) return AK_EINVAL;
  if (rows > 0 && (!logits || !targets || !row_loss || vocab == 0)) return AK_EINVAL;
  AK_DISPATCH(dtype, T, return launch_ce<T>(logits, targets, row_loss, out, rows, vocab, ignore_index, stream));
}

// ---------------------------------------------------------------------------------------------
// ak_cross_entropy_noalloc: ak_cross_entropy with the per-row losses in a file-scope device array
// instead of a caller workspace, for callers that cannot allocate. In host code `scratch` names a
// host-side stand-in, not device memory: its device address is looked up once per device with
// hipGetSymbolAddress (that device current) and cached; kernels only ever get that address.
// Every call writes the loss of each of its rows before ce_mean reads it, so nothing has to be
// cleared between calls; calls that overlap on one device share the array and race.
// ---------------------------------------------------------------------------------------------
static __device__ __align__(256) float scratch[AK_CE_NOALLOC_MAX_ROWS];

namespace {
constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
std::atomic<float*> g_scratch[kMaxDevices];

// Device address of `scratch` on the device that runs `stream` (the current device for the null
// stream); AK_OK or an error status.
int ce_scratch(hipStream_t stream, float** out) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e == hipSuccess && stream) e = hipStreamGetDevice(stream, &dev);
  if (e != hipSuccess) return record_hip_error(e);
  if (dev < 0 || dev >= kMaxDevices) return AK_EUNSUPPORTED;
  float* p = g_scratch[dev].load(std::memory_order_acquire);
  if (!p) {
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    p = g_scratch[dev].load(std::memory_order_relaxed);
    if (!p) {
      int cur = dev;
      e = hipGetDevice(&cur);
      if (e == hipSuccess && cur != dev) e = hipSetDevice(dev);
      void* addr = nullptr;
      if (e == hipSuccess) e = hipGetSymbolAddress(&addr, HIP_SYMBOL(scratch));
      if (cur != dev) {
        const hipError_t e2 = hipSetDevice(cur);
        if (e == hipSuccess) e = e2;
      }
      if (e != hipSuccess) return record_hip_error(e);
      if (!addr) return AK_EHIP;
      p = static_cast<float*>(addr);
      g_scratch[dev].store(p, std::memory_order_release);
    }
  }
  *out = p;
  return AK_OK;
}
}  // namespace

extern "C" int ak_cross_entropy_noalloc(int dtype, const void* logits, const int64_t* targets, void* out,
                                        int64_t rows, int64_t vocab, int64_t ignore_index, hipStream_t stream) {
  if (bad_rows(rows, vocab)) return AK_EINVAL;
  if (rows > AK_CE_NOALLOC_MAX_ROWS) return AK_EINVAL;
  if (!out) return AK_EINVAL;
  if (rows > 0 && (!logits || !targets || vocab == 0)) return AK_EINVAL;
  if (dtype != AK_F32 && dtype != AK_F16 && dtype != AK_BF16) return AK_EINVAL;
  float* loss = nullptr;
  const int st = ce_scratch(stream, &loss);
  if (st != AK_OK) return st;
  AK_DISPATCH(dtype, T, return launch_ce<T>(logits, targets, loss, out, rows, vocab, ignore_index, stream));
}

extern "C" int ak_reduce_sum(int dtype, const void* x, void* y, int64_t outer, int64_t reduce,
                             int64_t inner, hipStream_t stream) {
  if (outer < 0 || reduce < 0 || inner < 0 || reduce > INT_MAX || outer > (int64_t)INT_MAX * 256) return AK_EINVAL;
  if (outer == 0 || inner == 0) return AK_OK;
  if (!x || !y) return AK_EINVAL;
  AK_DISPATCH(dtype, T, return launch_reduce<T, false>(x, y, outer, reduce, inner, stream));
}

extern "C" int ak_reduce_max(int dtype, const void* x, void* y, int64_t outer, int64_t reduce,
                             int64_t inner, hipStream_t stream) {
  if (outer < 0 || reduce <= 0 || inner < 0 || reduce > INT_MAX || outer > (int64_t)INT_MAX * 256) return AK_EINVAL;
  if (outer == 0 || inner == 0) return AK_OK;
  if (!x || !y) return AK_EINVAL;
  AK_DISPATCH(dtype, T, return launch_reduce<T, true>(x, y, outer, reduce, inner, stream));
}
