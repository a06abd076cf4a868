// rope.hip -- interleaved rotary position embedding (reference.py:63-69) on gfx950.
//
// Pairs (x[2i], x[2i+1]) of each row rotate by table entry i of the row's position:
//   y[2i]   = rnd(rnd(x[2i]*cos[i]) - rnd(x[2i+1]*sin[i]))
//   y[2i+1] = rnd(rnd(x[2i]*sin[i]) + rnd(x[2i+1]*cos[i]))
// rnd() rounds to the element type, as each elementwise tensor op of the reference does; for
// fp32 no fused multiply-add is formed, so every element is bit-identical to the tensor ops.
// The fast path moves one 16-byte vector of x (4 pairs for f16 / bf16) per thread with two 8-byte
// table slices; table rows stay hot in L2 across heads. Index divisions use FastDiv (32-bit).
#include <limits.h>

#include "ak_common.h"

namespace ak {

#pragma clang fp contract(off)
template <typename T>
__device__ __forceinline__ void rope_pair(float x1, float x2, float c, float s, float* y1, float* y2) {
  *y1 = T::rnd(T::rnd(x1 * c) - T::rnd(x2 * s));
  *y2 = T::rnd(T::rnd(x1 * s) + T::rnd(x2 * c));
}

template <typename T>
__device__ __forceinline__ u32x4 rope_chunk(const u32x4& xv, const typename T::S* cp, const typename T::S* sp) {
  constexpr int kP = T::kVec / 2;  // pairs per 16-byte vector
  float cf[kP], sf[kP];
  if constexpr (kP == 4) {  // 2-byte types: 8 bytes of cos, 8 bytes of sin
    const u32x2 cv = *reinterpret_cast<const u32x2*>(cp);
    const u32x2 sv = *reinterpret_cast<const u32x2*>(sp);
    const u32x4 c4 = {cv[0], cv[1], 0u, 0u}, s4 = {sv[0], sv[1], 0u, 0u};
#pragma unroll
    for (int p = 0; p < kP; ++p) {
      cf[p] = T::lane_elem(c4, p);
      sf[p] = T::lane_elem(s4, p);
    }
  } else {  // fp32: 2 pairs per vector
#pragma unroll
    for (int p = 0; p < kP; ++p) {
      cf[p] = T::to_f(cp[p]);
      sf[p] = T::to_f(sp[p]);
    }
  }
  u32x4 yv;
#pragma unroll
  for (int p = 0; p < kP; ++p) {
    float y1, y2;
    rope_pair<T>(T::lane_elem(xv, 2 * p), T::lane_elem(xv, 2 * p + 1), cf[p], sf[p], &y1, &y2);
    T::set_elem(yv, 2 * p, y1);
    T::set_elem(yv, 2 * p + 1, y2);
  }
  return yv;
}

template <typename T>
__global__ __launch_bounds__(256) void rope_vec(const typename T::S* __restrict__ x,
                                                const typename T::S* __restrict__ ct,
                                                const typename T::S* __restrict__ st,
                                                typename T::S* __restrict__ y, int64_t nchunks,
                                                int chunks_per_row, int half, int64_t table_rows,
                                                int64_t rep_inner) {
  constexpr int kP = T::kVec / 2;
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= nchunks) return;
  const u32x4 xv = ld16(x + i * T::kVec);
  const int64_t row = i / chunks_per_row;
  const int c = (int)(i - row * chunks_per_row);
  const int64_t trow = (row / rep_inner) % table_rows;
  st16(y + i * T::kVec, rope_chunk<T>(xv, ct + trow * half + c * kP, st + trow * half + c * kP));
}

// The same with 32-bit indices (chunks, rows, table entries below 2^31) and the row, column and
// table-row divisions done by FastDiv: 6 % faster than 64-bit division at 34 MB (cold, rocprofv3).
template <typename T>
__global__ __launch_bounds__(256) void rope_vec32(const typename T::S* __restrict__ x,
                                                  const typename T::S* __restrict__ ct,
                                                  const typename T::S* __restrict__ st,
                                                  typename T::S* __restrict__ y, uint32_t nchunks, uint32_t cpr,
                                                  FastDiv f_cpr, uint32_t half, FastDiv f_rep, uint32_t table_rows,
                                                  FastDiv f_tab) {
  constexpr int kP = T::kVec / 2;
  const uint32_t i = blockIdx.x * 256u + threadIdx.x;
  if (i >= nchunks) return;
  const u32x4 xv = ld16(x + (int64_t)i * T::kVec);
  const uint32_t row = fdiv(i, f_cpr);
  const uint32_t c = i - row * cpr;
  const uint32_t q = fdiv(row, f_rep);
  const uint32_t toff = (q - fdiv(q, f_tab) * table_rows) * half + c * kP;
  st16(y + (int64_t)i * T::kVec, rope_chunk<T>(xv, ct + toff, st + toff));
}

// Any alignment: one pair per thread.
template <typename T>
__global__ __launch_bounds__(256) void rope_scalar(const typename T::S* __restrict__ x,
                                                   const typename T::S* __restrict__ ct,
                                                   const typename T::S* __restrict__ st,
                                                   typename T::S* __restrict__ y, int64_t npairs,
                                                   int half, int64_t table_rows, int64_t rep_inner) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= npairs) return;
  const int64_t row = i / half;
  const int p = (int)(i - row * half);
  const int64_t trow = (row / rep_inner) % table_rows;
  float y1, y2;
  rope_pair<T>(T::to_f(x[2 * i]), T::to_f(x[2 * i + 1]), T::to_f(ct[trow * half + p]),
               T::to_f(st[trow * half + p]), &y1, &y2);
  y[2 * i] = T::from_f(y1);
  y[2 * i + 1] = T::from_f(y2);
}
// Model form (the reference's LLaMA apply_rotary_emb, models/llama_7b.py:40-48): x upcast to
// fp32, rotated by fp32 cos / sin as a complex multiply, rounded once to x's dtype.
// x rows are grouped rep_inner (heads) to a token, token t starting at element t * x_tok_stride
// (dense when x_tok_stride = rep_inner * head_dim; larger when q / k are column slices of a fused
// QKV projection); y is dense.
template <typename T>
__global__ __launch_bounds__(256) void rope_f32t_vec(const typename T::S* __restrict__ x,
                                                    const float* __restrict__ ct,
                                                    const float* __restrict__ st,
                                                    typename T::S* __restrict__ y, int64_t nchunks,
                                                    int chunks_per_row, int half, int64_t table_rows,
                                                    int64_t rep_inner, int64_t x_tok_stride) {
  constexpr int kP = T::kVec / 2;
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= nchunks) return;
  const int64_t row = i / chunks_per_row;
  const int c = (int)(i - row * chunks_per_row);
  const int64_t tok = row / rep_inner;
  const int64_t trow = tok % table_rows;
  const int64_t xoff = tok * x_tok_stride + (row - tok * rep_inner) * (2 * half) + (int64_t)c * T::kVec;
  const u32x4 xv = ld16(x + xoff);
  const float* cp = ct + trow * half + c * kP;
  const float* sp = st + trow * half + c * kP;
  u32x4 yv;
#pragma unroll
  for (int p = 0; p < kP; ++p) {
    const float a = T::lane_elem(xv, 2 * p), b = T::lane_elem(xv, 2 * p + 1);
    const float cc = cp[p], ss = sp[p];
    T::set_elem(yv, 2 * p, a * cc - b * ss);
    T::set_elem(yv, 2 * p + 1, a * ss + b * cc);
  }
  st16(y + i * T::kVec, yv);
}
// rope_f32t_vec with 32-bit indices and FastDiv (chunks, rows, tokens and table entries below 2^31).
template <typename T>
__global__ __launch_bounds__(256) void rope_f32t_vec32(const typename T::S* __restrict__ x,
                                                      const float* __restrict__ ct,
                                                      const float* __restrict__ st,
                                                      typename T::S* __restrict__ y, uint32_t nchunks,
                                                      uint32_t cpr, FastDiv f_cpr, uint32_t half, uint32_t rep_inner,
                                                      FastDiv f_rep, uint32_t table_rows, FastDiv f_tab,
                                                      int64_t x_tok_stride) {
  constexpr int kP = T::kVec / 2;
  const uint32_t i = blockIdx.x * 256u + threadIdx.x;
  if (i >= nchunks) return;
  const uint32_t row = fdiv(i, f_cpr);
  const uint32_t c = i - row * cpr;
  const uint32_t tok = fdiv(row, f_rep);
  const uint32_t trow = tok - fdiv(tok, f_tab) * table_rows;
  const int64_t xoff = (int64_t)tok * x_tok_stride + (int64_t)(row - tok * rep_inner) * (2 * half) + c * T::kVec;
  const u32x4 xv = ld16(x + xoff);
  const float* cp = ct + trow * half + c * kP;
  const float* sp = st + trow * half + c * kP;
  u32x4 yv;
#pragma unroll
  for (int p = 0; p < kP; ++p) {
    const float a = T::lane_elem(xv, 2 * p), b = T::lane_elem(xv, 2 * p + 1);
    const float cc = cp[p], ss = sp[p];
    T::set_elem(yv, 2 * p, a * cc - b * ss);
    T::set_elem(yv, 2 * p + 1, a * ss + b * cc);
  }
  st16(y + (int64_t)i * T::kVec, yv);
}
#pragma clang fp contract(on)

template <typename T>
static int launch_rope(const void* x, const void* c, const void* s, void* y, int64_t rows,
                       int64_t d, int64_t table_rows, int64_t rep_inner, hipStream_t stream) {
  using S = typename T::S;
  const int half = (int)(d / 2);
  const bool vec = d % T::kVec == 0 && host_aligned16(x) && host_aligned16(y) &&
                   (((uintptr_t)c | (uintptr_t)s) & 7u) == 0;
  if (vec) {
    const int cpr = (int)(d / T::kVec);
    const int64_t n = rows * cpr;
    constexpr int64_t kLim = (int64_t)1 << 31;
    if (n < kLim && rep_inner < kLim && table_rows * half < kLim) {
      rope_vec32<T><<<(unsigned)cdiv(n, 256), 256, 0, stream>>>(
          (const S*)x, (const S*)c, (const S*)s, (S*)y, (uint32_t)n, (uint32_t)cpr, make_fastdiv((uint32_t)cpr),
          (uint32_t)half, make_fastdiv((uint32_t)rep_inner), (uint32_t)table_rows, make_fastdiv((uint32_t)table_rows));
    } else {
      rope_vec<T><<<(unsigned)cdiv(n, 256), 256, 0, stream>>>(
          (const S*)x, (const S*)c, (const S*)s, (S*)y, n, cpr, half, table_rows, rep_inner);
    }
  } else {
    const int64_t n = rows * half;
    rope_scalar<T><<<(unsigned)cdiv(n, 256), 256, 0, stream>>>((const S*)x, (const S*)c, (const S*)s,
                                                               (S*)y, n, half, table_rows, rep_inner);
  }
  return record_launch();
}

template <typename T>
static int launch_rope_f32t(const void* x, const float* c, const float* s, void* y, int64_t rows,
                            int64_t d, int64_t table_rows, int64_t rep_inner, int64_t x_tok_stride,
                            hipStream_t stream) {
  using S = typename T::S;
  const int cpr = (int)(d / T::kVec);
  const int64_t n = rows * cpr;
  constexpr int64_t kLim = (int64_t)1 << 31;
  if (n < kLim && rep_inner < kLim && table_rows * (d / 2) < kLim) {
    rope_f32t_vec32<T><<<(unsigned)cdiv(n, 256), 256, 0, stream>>>(
        (const S*)x, c, s, (S*)y, (uint32_t)n, (uint32_t)cpr, make_fastdiv((uint32_t)cpr), (uint32_t)(d / 2),
        (uint32_t)rep_inner, make_fastdiv((uint32_t)rep_inner), (uint32_t)table_rows,
        make_fastdiv((uint32_t)table_rows), x_tok_stride);
  } else {
    rope_f32t_vec<T><<<(unsigned)cdiv(n, 256), 256, 0, stream>>>((const S*)x, c, s, (S*)y, n, cpr,
                                                                   (int)(d / 2), table_rows, rep_inner,
                                                                   x_tok_stride);
  }
  return record_launch();
}

}  // namespace ak

using namespace ak;

extern "C" int ak_rope(int dtype, const void* x, const void* cos_t, const void* sin_t, void* y,
                       int64_t rows, int64_t head_dim, int64_t table_rows, int64_t rep_inner,
                       hipStream_t stream) {
  if (rows < 0 || head_dim < 0 || head_dim % 2 != 0 || head_dim > INT_MAX) return AK_EINVAL;
  if (rows == 0 || head_dim == 0) return AK_OK;
  if (!x || !cos_t || !sin_t || !y || table_rows <= 0 || rep_inner <= 0) return AK_EINVAL;
  if (rows * head_dim / 2 > (int64_t)UINT_MAX * 256) return AK_EINVAL;
  AK_DISPATCH(dtype, T, return launch_rope<T>(x, cos_t, sin_t, y, rows, head_dim, table_rows, rep_inner, stream));
}

extern "C" int ak_rope_f32_tables(int dtype, const void* x, const float* cos_t, const float* sin_t,
                                  void* y, int64_t rows, int64_t head_dim, int64_t table_rows,
                                  int64_t rep_inner, int64_t x_tok_stride, hipStream_t stream) {
  if (rows < 0 || head_dim < 0 || head_dim % 2 != 0 || head_dim > INT_MAX) return AK_EINVAL;
  if (rows == 0 || head_dim == 0) return AK_OK;
  if (!x || !cos_t || !sin_t || !y || table_rows <= 0 || rep_inner <= 0 || rows % rep_inner != 0) return AK_EINVAL;
  if (x_tok_stride < rep_inner * head_dim) return AK_EINVAL;
  if (dtype != AK_F16 && dtype != AK_BF16) return AK_EUNSUPPORTED;
  if (head_dim % 8 != 0 || x_tok_stride % 8 != 0 || !host_aligned16(x) || !host_aligned16(y)) return AK_EUNSUPPORTED;
  if (rows * head_dim / 8 > (int64_t)UINT_MAX * 256) return AK_EINVAL;
  if (dtype == AK_F16)
    return launch_rope_f32t<TF16>(x, cos_t, sin_t, y, rows, head_dim, table_rows, rep_inner, x_tok_stride, stream);
  return launch_rope_f32t<TBF16>(x, cos_t, sin_t, y, rows, head_dim, table_rows, rep_inner, x_tok_stride, stream);
}
