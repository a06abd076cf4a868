// gemm.hip -- LDS-tiled MFMA GEMM for gfx950 (f16 / bf16 in, fp32 accumulate), the dual-B
// SwiGLU gate/up kernel built on it, and a full-precision fp32 GEMM on v_mfma_f32_16x16x4_f32.
//
// f16 / bf16 design
//   * Block tile BM x BN (BN per B matrix; NB = 1 plain GEMM, NB = 2 gate and up sharing the A
//     tile). WM x WN waves; each wave owns a (BM/WM) x (BN/WN) sub-tile per B matrix made of
//     16x16 v_mfma_f32_16x16x32_{f16,bf16} tiles. The MFMA is issued with B as the "A" operand,
//     so a lane's accumulator holds four consecutive C columns of one row (8-byte stores).
//   * Main kernel (gemm_dma, K-contiguous B = nn.Linear weights, K % 64 == 0): operands reach LDS
//     by LDS DMA, two or three 64-deep stages (four 32-deep ones when the grid under-fills the
//     chip), so one or two tiles stream in while one is multiplied. Inside a tile the next
//     k-step's fragments load from LDS while the current MFMAs run, and the barrier that retires
//     a stage sits between the two halves of a k-step's MFMAs.
//   * Fallback kernel (gemm_mfma: any alignment, odd K, strided or [K, N] B): register-staged
//     loads into two LDS stages of [rows][64], chunks XOR-swizzled; [K, N] B is transposed in
//     registers on its way to LDS (8x8 blocks rebuilt as K-contiguous rows with v_perm_b32).
//   * Tile order is XCD-aware: hardware hands block i to XCD i % 8, so consecutive logical tiles
//     are given to one XCD and grouped along M to share A and B in that XCD's L2.
#include <limits.h>

#include "ak_common.h"

namespace ak {

constexpr int kBK = 64;           // k extent of one LDS tile
constexpr int kKC = kBK / 8;      // 16-byte chunks per tile row

// Physical chunk of logical chunk c in row `row`. Rows r and r + 8 get different patterns, so
// both the 16-row fragment reads and the transposed [K,N] writes (rows 8 apart) are conflict-free.
__device__ __forceinline__ int swz(int row, int c) { return c ^ ((row ^ (row >> 3)) & 7); }
// element offset of chunk c of row `row` in a [rows][64] tile
__device__ __forceinline__ int lds_off(int row, int c) { return row * kBK + swz(row, c) * 8; }

template <typename T>
__device__ __forceinline__ f32x4 mfma16x16x32(const u32x4& a, const u32x4& b, const f32x4& c);
template <>
__device__ __forceinline__ f32x4 mfma16x16x32<TF16>(const u32x4& a, const u32x4& b, const f32x4& c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a), __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
}
template <>
__device__ __forceinline__ f32x4 mfma16x16x32<TBF16>(const u32x4& a, const u32x4& b, const f32x4& c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
}

// The LDS-DMA kernel's MFMA: v_mfma_f32_16x16x32 (f32x4 accumulators), 8 consecutive k of one row
// per lane. (32x32x16 fragments were measured 4-10 % slower on every workload.)
template <int MF>
struct MfmaAcc {
  static_assert(MF == 16, "the LDS-DMA kernel uses 16x16x32 fragments");
  using type = f32x4;
};
template <typename T, int MF>
__device__ __forceinline__ typename MfmaAcc<MF>::type mfma_tile(const u32x4& a, const u32x4& b,
                                                                const typename MfmaAcc<MF>::type& c) {
  return mfma16x16x32<T>(a, b, c);
}

// Load 8 consecutive k of one row of a K-contiguous matrix (row stride ld). Out-of-range rows or
// k give zeros. VEC: K, ld and the base are multiples of 8 elements / 16 bytes.
template <bool VEC>
__device__ __forceinline__ u32x4 load_kchunk(const uint16_t* __restrict__ p, int64_t ld, int row, int rows,
                                             int k, int K) {
  if constexpr (VEC) {
    if (row < rows && k < K) return ld16(p + (int64_t)row * ld + k);
    return u32x4{0u, 0u, 0u, 0u};
  } else {
    u32x4 v = {0u, 0u, 0u, 0u};
    if (row < rows) {
      const uint16_t* q = p + (int64_t)row * ld;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const uint32_t h = (k + e < K) ? q[k + e] : 0u;
        v[e >> 1] |= h << ((e & 1) * 16);
      }
    }
    return v;
  }
}

// 4x8 transpose of 16-bit values: in[r] holds 8 n-values of k-row r; out[n] gets the 4 k-values
// of column n (v_perm_b32 picks the low or high halves of two words).
__device__ __forceinline__ void transpose4x8(const u32x4 (&in)[4], u32x2 (&out)[8]) {
#pragma unroll
  for (int n = 0; n < 8; ++n) {
    const int w = n >> 1;
    const uint32_t sel = (n & 1) ? 0x07060302u : 0x05040100u;
    out[n][0] = __builtin_amdgcn_perm(in[1][w], in[0][w], sel);
    out[n][1] = __builtin_amdgcn_perm(in[3][w], in[2][w], sel);
  }
}

// Tile scheduling: logical tile index for this block (XCD-aware, grouped along M).
__device__ __forceinline__ void tile_coords(int tiles_m, int tiles_n, int* tm, int* tn) {
  const int nb = gridDim.x;
  const int bid = blockIdx.x;
  const int full = nb & ~7;
  const int L = bid < full ? (bid & 7) * (full >> 3) + (bid >> 3) : bid;
  constexpr int GM = 4;
  const int per_group = GM * tiles_n;
  const int g = L / per_group;
  const int first_m = g * GM;
  const int gsz = min(tiles_m - first_m, GM);
  const int r = L - g * per_group;
  *tm = first_m + r % gsz;
  *tn = r / gsz;
}

// --------------------------------------------------------------------------------------------
// Epilogues (applied to fp32 accumulators; every step rounds like the reference's tensor ops)
// --------------------------------------------------------------------------------------------
enum Epi { kEpiStore = 0, kEpiSilu = 1, kEpiGelu = 2, kEpiRelu2 = 3, kEpiNone = 4, kEpiResidual = 5, kEpiRope = 6,
           kEpiPartial = 7, kEpiBias = 8, kEpiBiasGelu = 9, kEpiBiasResidual = 10 };

// Arguments of the rotary epilogue (kEpiRope), passed by value to every f16 / bf16 GEMM kernel:
// columns [0, rot_cols) of C form heads of head_dim columns whose (even, odd) pairs are rotated
// by the fp32 tables cos / sin [seq_len, head_dim / 2]; row m of C is token m % seq_len.
//
// Split-K (kEpiPartial): the grid's y dimension is the K slice; slice z multiplies A and B advanced
// by z * split_a / z * split_b elements and stores its fp32 accumulators to the workspace advanced by
// z * split_c floats (row stride ldc), for splitk_reduce to sum.
struct EpiArgs {
  const uint16_t* bias = nullptr;  // kEpiBiasResidual (R is the residual there)
  const float* cos = nullptr;
  const float* sin = nullptr;
  int head_dim = 0;
  int rot_cols = 0;
  int seq_len = 1;
  int splits = 1;
  int64_t split_a = 0, split_b = 0, split_c = 0;
  // Batched products (ak_gemm_batched): grid z is the batch item; item z reads A and B advanced by
  // z * batch_a / z * batch_b elements and writes C advanced by z * batch_c (a stride of 0 shares
  // the operand across the batch).
  int batch = 1;
  int64_t batch_a = 0, batch_b = 0, batch_c = 0;
};

// Bases of this block's batch item (grid z); one item when ep.batch == 1.
template <class PA, class PB, class PC>
__device__ __forceinline__ void batch_bases(PA& A, PB& B, PC& C, const EpiArgs& ep) {
  if (ep.batch > 1) {
    const int64_t z = blockIdx.z;
    A += z * ep.batch_a;
    B += z * ep.batch_b;
    C += z * ep.batch_c;
  }
}

// The model's rotation of one pair in fp32, each product and sum rounded on its own (no fused
// multiply-add), as separate fp32 tensor ops compute (a c - b s, a s + b c).
__device__ __forceinline__ void rope_rotate(float& a, float& b, float c, float s) {
#pragma clang fp contract(off)
  const float y1 = a * c - b * s;
  const float y2 = a * s + b * c;
  a = y1;
  b = y2;
}

// torch's exact GELU of one rounded value, in fp32: x * 0.5 * (1 + erf(x / sqrt(2)))
__device__ __forceinline__ float gelu_erf(float g) { return 0.5f * g * (1.0f + erff(g * 0.70710678118654752f)); }

template <typename T, int EPI>
__device__ __forceinline__ float gate_up(float g_acc, float u_acc) {
  const float g = T::rnd(g_acc);
  const float u = T::rnd(u_acc);
  float a;
  if constexpr (EPI == kEpiSilu) a = T::rnd(g / (1.0f + expf(-g)));
  else if constexpr (EPI == kEpiGelu) a = T::rnd(gelu_erf(g));
  else if constexpr (EPI == kEpiRelu2) { const float r = g > 0.f ? g : 0.f; a = T::rnd(r * r); }
  else a = g;
  return a * u;  // rounded by the store
}

// Epilogue of one lane's share of a block tile: for fragment (i, j) the lane holds the four
// consecutive outputs C[m][n .. n + 3], m = mb + MST i, n = nb + NST j, in acc[.][i][j] (NB == 2:
// gate and up accumulators, combined by gate_up).
//   kEpiResidual rounds the product to the element type, adds R[m][n + e] (R shares C's leading
//     dimension) and rounds again: the two roundings of torch's `R + A @ B`. fp32 holds the sum of
//     two f16 / bf16 values to 24 bits, at least 2p + 2 for both formats, so rounding it once more
//     gives the correctly rounded sum.
//   kEpiBias adds bias[n + e] (the element type, R points at it) to the fp32 accumulator and
//     rounds once: nn.Linear's fused bias (torch's addmm adds it in the fp32 compute type).
//   kEpiBiasGelu is kEpiBias's rounded value through exact GELU in fp32, rounded again: a biased
//     nn.Linear followed by nn.GELU (R points at the bias).
//   kEpiBiasResidual is kEpiBias's rounded value plus R[m][n + e] (the residual; the bias comes
//     from ep.bias), rounded again: torch's `R + linear(x)` for a biased Linear.
//   kEpiRope rounds the product to the element type, then (columns below rot_cols) rotates the
//     pairs (n, n + 1), (n + 2, n + 3) in fp32 by table row m % seq_len and rounds once: the
//     projection's output cast to fp32, rotated and cast back. n is a multiple of 4 and head_dim
//     of 4, so the four columns never straddle a head or the rot_cols boundary.
// The side values (R, or the cos / sin pairs) of every fragment are loaded first, then combined
// and stored, so their latency is paid once per tile rather than once per fragment.
// Stores: the results of fragments 2p and 2p + 1 (columns 32p + 4g + 0..3 and 32p + 16 + 4g + 0..3
// in lane group g = lane / 16) are packed to the element type and regrouped across the four lane
// groups (regroup8), so each lane stores 8 consecutive columns 32p + 8g + 0..7 of its row: one
// 16-byte store where C is 16-byte aligned, which fills the 64-byte requests (4 lanes x 16 bytes
// per row) that 8-byte stores half-fill.
// VEC: a lane's 8 in-range columns of C are one 16-byte store at any alignment (store_cols), so
// any leading dimension works (an odd ldc, e.g. a 50257-column vocabulary projection); R's four
// columns load as one 8-byte access where that is 8-byte aligned, as elements otherwise.
// Regroup two fragments' packed columns across the 16-lane groups of a wave. On entry lane group g
// (lanes 16g .. 16g + 15) holds 4-column group g of fragment x and of fragment y, i.e. groups g and
// 4 + g of their 32 columns; on exit it holds group 2g in x and group 2g + 1 in y. Lanes keep their
// row (lane % 16). permlane32_swap exchanges x's upper half-wave with y's lower one
// (x = [x0 x1 y0 y1], y = [x2 x3 y2 y3] by lane group), permlane16_swap x's odd lane groups with
// y's even ones (x = [x0 x2 y0 y2], y = [x1 x3 y1 y3]).
__device__ __forceinline__ void regroup8(uint32_t& x, uint32_t& y) {
  const auto h = __builtin_amdgcn_permlane32_swap(x, y, false, false);
  const auto q = __builtin_amdgcn_permlane16_swap(h[0], h[1], false, false);
  x = q[0];
  y = q[1];
}

// Store the first W (4 or 8) 16-bit elements of o (element e in dword e / 2, low half first) to
// cp[0 .. W - 1], the first `valid` of them only. With all W in range (VEC) it is one 16- or 8-byte
// store at whatever 2-byte alignment cp has: global memory on this target takes multi-dword
// accesses at any alignment (the HSA code object is built with unaligned-access-mode, which is why
// the compiler emits one global_store_dwordx4 for a 2-byte-aligned pointer here). Rows whose start
// is not 16-byte aligned (an odd ldc, e.g. a 50257-column vocabulary projection) took 47 % longer
// with stores narrowed to their alignment.
typedef u32x4 u32x4_a2 __attribute__((aligned(2)));
typedef u32x2 u32x2_a2 __attribute__((aligned(2)));
template <bool VEC, int W>
__device__ __forceinline__ void store_cols(uint16_t* cp, int valid, const u32x4& o) {
  if (VEC && valid >= W) {
    if constexpr (W == 8) *reinterpret_cast<u32x4_a2*>(cp) = o;
    else *reinterpret_cast<u32x2_a2*>(cp) = u32x2{o[0], o[1]};
    return;
  }
#pragma unroll
  for (int e = 0; e < W; ++e)
    if (e < valid) cp[e] = (uint16_t)(o[e >> 1] >> ((e & 1) * 16));
}

template <typename T, int NB, int EPI, bool VEC, int FM, int FN, int MST = 16, int NST = 16>
__device__ __forceinline__ void tile_epilogue(uint16_t* __restrict__ C, const uint16_t* __restrict__ R,
                                              int64_t ldc, int M, int N, int mb, int nb,
                                              const f32x4 (&acc)[NB][FM][FN], const EpiArgs& ep) {
  typedef float f32x2 __attribute__((ext_vector_type(2)));
  constexpr bool kRes = NB == 1 && (EPI == kEpiResidual || EPI == kEpiBiasResidual);
  constexpr bool kRope = NB == 1 && EPI == kEpiRope;
  constexpr bool kBias = NB == 1 && (EPI == kEpiBias || EPI == kEpiBiasGelu || EPI == kEpiBiasResidual);
  if constexpr (NB == 1 && EPI == kEpiPartial) {
    // fp32 accumulators as they are (C is the fp32 workspace; N % 4 == 0 and ldc % 4 == 0)
    float* Cf = reinterpret_cast<float*>(C);
#pragma unroll
    for (int i = 0; i < FM; ++i) {
      const int m = mb + i * MST;
      if (m >= M) continue;
#pragma unroll
      for (int j = 0; j < FN; ++j) {
        const int n = nb + j * NST;
        if (n < N) *reinterpret_cast<f32x4*>(Cf + (int64_t)m * ldc + n) = acc[0][i][j];
      }
    }
    return;
  }
  u32x2 side_r[kRes ? FM : 1][kRes ? FN : 1];
  float side_b[kBias ? FN : 1][4];
  if constexpr (kBias) {
    const uint16_t* bias = EPI == kEpiBiasResidual ? ep.bias : R;
#pragma unroll
    for (int j = 0; j < FN; ++j) {
      const int n = nb + j * NST;
#pragma unroll
      for (int e = 0; e < 4; ++e) side_b[j][e] = n + e < N ? T::to_f(bias[n + e]) : 0.f;
    }
  }
  f32x2 side_c[kRope ? FM : 1][kRope ? FN : 1], side_s[kRope ? FM : 1][kRope ? FN : 1];
  if constexpr (kRes) {
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
      for (int j = 0; j < FN; ++j) {
        const int m = mb + i * MST, n = nb + j * NST;
        const uint16_t* rp = R + (int64_t)m * ldc + n;
        u32x2 r = {0u, 0u};
        if (m < M) {
          if (VEC && n + 3 < N && ((uintptr_t)rp & 7u) == 0) {
            r = *reinterpret_cast<const u32x2*>(rp);
          } else {
#pragma unroll
            for (int e = 0; e < 4; ++e)
              if (n + e < N) r[e >> 1] |= (uint32_t)rp[e] << ((e & 1) * 16);
          }
        }
        side_r[i][j] = r;
      }
  }
  if constexpr (kRope) {
    const int half = ep.head_dim >> 1;
#pragma unroll
    for (int i = 0; i < FM; ++i) {
      const int m = mb + i * MST;
      const int64_t row = (int64_t)((m < M ? m : 0) % ep.seq_len) * half;
#pragma unroll
      for (int j = 0; j < FN; ++j) {
        const int n = nb + j * NST;
        f32x2 c = {1.f, 1.f}, sn = {0.f, 0.f};
        if (n < ep.rot_cols) {
          const int64_t t = row + ((n % ep.head_dim) >> 1);  // even: 8-byte aligned pairs
          c = *reinterpret_cast<const f32x2*>(ep.cos + t);
          sn = *reinterpret_cast<const f32x2*>(ep.sin + t);
        }
        side_c[i][j] = c;
        side_s[i][j] = sn;
      }
    }
  }
  static_assert(NST == 16, "fragment pairs regroup 16-column fragments");
#pragma unroll
  for (int i = 0; i < FM; ++i) {
    const int m = mb + i * MST;
    uint32_t lo[FN], hi[FN];  // packed columns 0, 1 and 2, 3 of each fragment
#pragma unroll
    for (int j = 0; j < FN; ++j) {
      const int n = nb + j * NST;
      float v[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        if constexpr (NB == 2) v[e] = gate_up<T, EPI>(acc[0][i][j][e], acc[1][i][j][e]);
        else if constexpr ((kRes && !kBias) || kRope) v[e] = T::rnd(acc[0][i][j][e]);
        else v[e] = acc[0][i][j][e];
      }
      if constexpr (kBias) {
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          v[e] += side_b[j][e];
          if constexpr (EPI != kEpiBias) v[e] = T::rnd(v[e]);
          if constexpr (EPI == kEpiBiasGelu) v[e] = gelu_erf(v[e]);
        }
      }
      if constexpr (kRes) {
#pragma unroll
        for (int e = 0; e < 4; ++e) v[e] += T::to_f((uint16_t)(side_r[i][j][e >> 1] >> ((e & 1) * 16)));
      }
      if constexpr (kRope) {
        if (n < ep.rot_cols) {
          rope_rotate(v[0], v[1], side_c[i][j][0], side_s[i][j][0]);
          rope_rotate(v[2], v[3], side_c[i][j][1], side_s[i][j][1]);
        }
      }
      lo[j] = (uint32_t)T::from_f(v[0]) | ((uint32_t)T::from_f(v[1]) << 16);
      hi[j] = (uint32_t)T::from_f(v[2]) | ((uint32_t)T::from_f(v[3]) << 16);
    }
    // fragment pairs: 8 consecutive columns per lane (the shuffles run on every lane, before the
    // row test)
    const int g = (lane_id() >> 4) & 3;
    const int nq = nb - 4 * g + 8 * g;  // lane group g's first column of pair 0
#pragma unroll
    for (int j = 0; j + 1 < FN; j += 2) {
      regroup8(lo[j], lo[j + 1]);
      regroup8(hi[j], hi[j + 1]);
      if (m < M) {
        const u32x4 o = {lo[j], hi[j], lo[j + 1], hi[j + 1]};
        const int n = nq + j * NST;
        store_cols<VEC, 8>(C + (int64_t)m * ldc + n, N - n, o);
      }
    }
    if constexpr (FN % 2 == 1) {
      if (m < M) {
        const int n = nb + (FN - 1) * NST;
        const u32x4 o = {lo[FN - 1], hi[FN - 1], 0u, 0u};
        store_cols<VEC, 4>(C + (int64_t)m * ldc + n, N - n, o);
      }
    }
  }
}

// --------------------------------------------------------------------------------------------
// The f16 / bf16 kernel
// --------------------------------------------------------------------------------------------
template <typename T, bool BT, bool VEC, int BM, int BN, int WM, int WN, int NB, int EPI>
__global__ __launch_bounds__(WM* WN* kWave) void gemm_mfma(
    const uint16_t* __restrict__ A, const uint16_t* __restrict__ B0, const uint16_t* __restrict__ B1,
    uint16_t* __restrict__ C, int M, int N, int K, int64_t lda, int64_t ldb, int64_t ldc,
    int tiles_m, int tiles_n, EpiArgs ep) {
  constexpr int kThreads = WM * WN * kWave;
  constexpr int WTM = BM / WM, WTN = BN / WN;
  constexpr int FM = WTM / 16, FN = WTN / 16;
  constexpr int A_CH = BM * kKC / kThreads;  // A chunks per thread
  static_assert(BM * kKC % kThreads == 0, "A tile must split evenly");
  constexpr int BT_CH = (BN * kKC + kThreads - 1) / kThreads;      // [N,K] B chunks per thread
  constexpr int BN_UNITS = (kBK / 4) * (BN / 8);                   // [K,N] B 4x8 units per matrix
  constexpr int BN_U = (BN_UNITS + kThreads - 1) / kThreads;

  __shared__ __attribute__((aligned(16))) uint16_t sA[2][BM * kBK];
  __shared__ __attribute__((aligned(16))) uint16_t sB[2][NB][BN * kBK];
  batch_bases(A, B0, C, ep);

  int tm, tn;
  tile_coords(tiles_m, tiles_n, &tm, &tn);
  const int m0 = tm * BM, n0 = tn * BN;
  const int tid = threadIdx.x;
  const int lane = lane_id();
  const int wid = wave_id();
  const int wm = wid / WN, wn = wid % WN;
  const uint16_t* Bm[2] = {B0, B1};

  // ---- global -> register staging ----
  u32x4 ra[A_CH];
  u32x4 rbt[NB][BT ? BT_CH : 1];
  u32x4 rbn[BT ? 1 : BN_U][4];

  auto gload = [&](int k0) {
#pragma unroll
    for (int i = 0; i < A_CH; ++i) {
      const int q = tid + i * kThreads;
      const int row = q / kKC, c = q % kKC;
      ra[i] = load_kchunk<VEC>(A, lda, m0 + row, M, k0 + c * 8, K);
    }
    if constexpr (BT) {
#pragma unroll
      for (int b = 0; b < NB; ++b)
#pragma unroll
        for (int i = 0; i < BT_CH; ++i) {
          const int q = tid + i * kThreads;
          const int row = q / kKC, c = q % kKC;
          if (q < BN * kKC) rbt[b][i] = load_kchunk<VEC>(Bm[b], ldb, n0 + row, N, k0 + c * 8, K);
        }
    } else {
#pragma unroll
      for (int i = 0; i < BN_U; ++i) {
        const int u = tid + i * kThreads;
        // consecutive lanes take consecutive 8-column groups of the same 4 k-rows (coalesced)
        const int ng = u % (BN / 8), kq = u / (BN / 8);
        if (u < BN_UNITS) {
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const int k = k0 + kq * 4 + r;
            const int n = n0 + ng * 8;
            u32x4 v = {0u, 0u, 0u, 0u};
            if (k < K) {
              const uint16_t* p = B0 + (int64_t)k * ldb + n;
              if constexpr (VEC) {
                if (n < N) v = ld16(p);
              } else {
#pragma unroll
                for (int e = 0; e < 8; ++e) {
                  const uint32_t h = (n + e < N) ? p[e] : 0u;
                  v[e >> 1] |= h << ((e & 1) * 16);
                }
              }
            }
            rbn[i][r] = v;
          }
        }
      }
    }
  };
  auto sstore = [&](int st) {
#pragma unroll
    for (int i = 0; i < A_CH; ++i) {
      const int q = tid + i * kThreads;
      const int row = q / kKC, c = q % kKC;
      *reinterpret_cast<u32x4*>(&sA[st][lds_off(row, c)]) = ra[i];
    }
    if constexpr (BT) {
#pragma unroll
      for (int b = 0; b < NB; ++b)
#pragma unroll
        for (int i = 0; i < BT_CH; ++i) {
          const int q = tid + i * kThreads;
          const int row = q / kKC, c = q % kKC;
          if (q < BN * kKC) *reinterpret_cast<u32x4*>(&sB[st][b][lds_off(row, c)]) = rbt[b][i];
        }
    } else {
#pragma unroll
      for (int i = 0; i < BN_U; ++i) {
        const int u = tid + i * kThreads;
        const int ng = u % (BN / 8), kq = u / (BN / 8);
        if (u < BN_UNITS) {
          u32x2 t[8];
          transpose4x8(rbn[i], t);
#pragma unroll
          for (int n = 0; n < 8; ++n)
            *reinterpret_cast<u32x2*>(&sB[st][0][lds_off(ng * 8 + n, kq >> 1) + (kq & 1) * 4]) = t[n];
        }
      }
    }
  };

  f32x4 acc[NB][FM][FN];
#pragma unroll
  for (int b = 0; b < NB; ++b)
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
      for (int j = 0; j < FN; ++j) acc[b][i][j] = f32x4{0.f, 0.f, 0.f, 0.f};

  const int KT = (K + kBK - 1) / kBK;
  gload(0);
  sstore(0);
  __syncthreads();

  const int fr = lane & 15;        // fragment row owned by this lane
  const int fc = lane >> 4;        // 8-element k group inside a 32-k step
  for (int kt = 0; kt < KT; ++kt) {
    const int cur = kt & 1;
    if (kt + 1 < KT) gload((kt + 1) * kBK);
#pragma unroll
    for (int s = 0; s < kBK / 32; ++s) {
      u32x4 fa[FM], fb[NB][FN];
#pragma unroll
      for (int i = 0; i < FM; ++i) {
        const int row = wm * WTM + i * 16 + fr;
        fa[i] = *reinterpret_cast<const u32x4*>(&sA[cur][lds_off(row, s * 4 + fc)]);
      }
#pragma unroll
      for (int b = 0; b < NB; ++b)
#pragma unroll
        for (int j = 0; j < FN; ++j) {
          const int row = wn * WTN + j * 16 + fr;
          fb[b][j] = *reinterpret_cast<const u32x4*>(&sB[cur][b][lds_off(row, s * 4 + fc)]);
        }
#pragma unroll
      for (int b = 0; b < NB; ++b)
#pragma unroll
        for (int i = 0; i < FM; ++i)
#pragma unroll
          for (int j = 0; j < FN; ++j) acc[b][i][j] = mfma16x16x32<T>(fb[b][j], fa[i], acc[b][i][j]);
    }
    if (kt + 1 < KT) sstore(cur ^ 1);
    __syncthreads();
  }

  // ---- epilogue: lane holds C[m][n .. n+3] for each (i, j) ----
  tile_epilogue<T, NB, EPI, VEC, FM, FN>(C, B1, ldc, M, N, m0 + wm * WTM + fr, n0 + wn * WTN + fc * 4, acc, ep);
}

// --------------------------------------------------------------------------------------------
// The f16 / bf16 kernel for K-contiguous B ([N, K], nn.Linear weights) with K % 64 == 0.
// Tiles move global -> LDS with gfx950's LDS DMA (global_load_lds_dwordx4): no staging registers
// and no LDS store instructions. One DMA instruction writes 64 lanes x 16 bytes = 1 KB of
// consecutive tile rows; each lane fetches the logical chunk that the XOR swizzle maps to its
// physical slot. Rows past M / N are clamped to the last row (their results are never stored).
// gfx950 serves a 64-lane ds_read_b128 in 8-lane phases, so the swizzles put the 8 rows of a phase
// in 8 distinct 16-byte bank slots (measured for 128-byte rows: SQ_LDS_BANK_CONFLICT 0 with
// chunk c ^ (row & 7), 50% with an extra row-bit-3 term, 75% unswizzled).
// --------------------------------------------------------------------------------------------
// LDS-DMA helpers (lds_void, wait_vmcnt, dma_barrier) live in ak_common.h.

// The same transfer as inline assembly. The compiler then does not track it: its wait-count pass
// inserts no waits for it (a conservative full wait at a loop head otherwise drains the whole
// four-stage pipeline once per iteration), and every wait is the caller's explicit vmcnt. M0
// holds the wave-uniform LDS destination. It is an input operand bound to M0 ("{m0}"), so the
// compiler writes M0 itself and knows its value; the statement changes no register behind the
// compiler's back. One wait state separates the M0 write from the load.
__device__ __forceinline__ void dma16_asm(const char* base, uint32_t off, uint16_t* lds_row_base) {
  const uint32_t lds = (uint32_t)(uintptr_t)(lds_void*)lds_row_base;
  asm volatile(
      "s_nop 0\n\t"
      "global_load_lds_dwordx4 %0, %1"
      :
      : "v"(off), "s"(base), "{m0}"(lds)
      : "memory");
}

// Multi-stage variant: NS LDS stages of BKD-deep tiles (BKD 64: 128-byte rows, chunk c of row r
// at c ^ (r & 7), 8 rows per DMA instruction; BKD 32: 64-byte rows, chunk c at c ^ ((r >> 2) & 1),
// 16 rows per instruction; either way the 8 rows of one ds_read_b128 phase hit 8 distinct 16-byte
// bank slots). NS - 1 tiles are in flight while one is multiplied. Tile t lives in stage t % NS;
// the loop runs in groups of NS tiles with a uniform guard on the tail.
template <int BKD>
struct DmaGeom;
template <>
struct DmaGeom<64> {
  static constexpr int RPI = 8;  // rows per 1 KB DMA instruction
  __device__ static __forceinline__ int swz(int r, int c) { return c ^ (r & 7); }
};
template <>
struct DmaGeom<32> {
  static constexpr int RPI = 16;
  __device__ static __forceinline__ int swz(int r, int c) { return c ^ ((r >> 2) & 1); }
};

// [K, N] B (N contiguous, torch.matmul's B) is staged as [k][n] tile rows. The MFMA operand needs
// 8 consecutive k of one n per lane: two ds_read_b64_tr_b16 each give 4. That instruction
// transposes across each group of 16 lanes: output lane i, element e = element (i % 4) of source
// lane (i / 4 + 4 e); so source lane j addresses B[k0 + j / 4][n0 + 4 (j % 4)] and output lane i
// receives B[k0 + e][n0 + i]. 16-byte chunk c of tile row k is stored at c ^ bkn_swz<BN>(k): the 16
// rows of one tr read (4 per lane group) land on distinct banks for lane groups {0,1}, {2,3},
// {0,2} and {1,3}.
// A 64-element tile row (BN = 64) has 8 chunks and 128 bytes, so rows r and r + 2 share banks: the
// pattern 2 ((k >> 1) & 1) + 4 (((k >> 3) ^ (k >> 4)) & 1) keeps each read's chunk pair inside the row
// and gives rows {0, 2, 8, 10}, {0, 2, 16, 18} and {8, 10, 24, 26} distinct chunk pairs (rows + 4,
// the second read, share the pattern).
template <int BN>
__device__ __forceinline__ int bkn_swz(int k) {
  if constexpr (BN == 64) return 2 * (((k >> 1) & 1) + 2 * (((k >> 3) ^ (k >> 4)) & 1));
  else return 2 * ((k & 3) + 4 * (((k >> 3) ^ (k >> 4)) & 1));
}

typedef short gemm_s16x4 __attribute__((ext_vector_type(4)));
__device__ __forceinline__ u32x2 lds_tr16(const uint16_t* p) {
  return __builtin_bit_cast(
      u32x2, __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) gemm_s16x4*)(p)));
}

// B-side DMA geometry: BKN (B is [K, N]) stages BKD rows of BN elements, else BN rows of BKD.
template <int BN, int BKD, bool BKN>
struct DmaB {
  static constexpr int kRowElems = BKN ? BN : BKD;
  static constexpr int RPI = 512 / kRowElems;    // tile rows per 1 KB transfer
  static constexpr int kRows = BKN ? BKD : BN;   // tile rows per stage
};

template <typename T, int BM, int BN, int WM, int WN, int NB, int BKD, int NS, bool BKN, int MF>
__device__ __forceinline__ void gemm_dma_ns_kloop(
    typename MfmaAcc<MF>::type (&acc)[NB][BM / WM / MF][BN / WN / MF], const uint16_t* A, const uint16_t* B0,
    const uint16_t* B1, const uint32_t* oa, const uint32_t* ob, uint32_t kb_step_b, int K, int wid,
    int wm, int wn, int lane, uint16_t* s0, uint16_t* s1, uint16_t* s2, uint16_t* s3) {
  using G = DmaGeom<BKD>;
  using GB = DmaB<BN, BKD, BKN>;
  constexpr int NW = WM * WN;
  constexpr int WTM = BM / WM, WTN = BN / WN;
  constexpr int FM = WTM / MF, FN = WTN / MF;
  constexpr int A_INS = BM / G::RPI / NW;
  constexpr int B_INS = GB::kRows / GB::RPI / NW;
  constexpr int INS = A_INS + NB * B_INS;
  constexpr int H = FM / 2;
  constexpr int KS = 32;  // k per MFMA
  constexpr int STEPS = BKD / KS;         // k-steps per tile
  static_assert(NS >= 2 && NS <= 4, "stages");
  const uint16_t* Bm[2] = {B0, B1};
  // fragment row (lane % MF) and 16-byte k chunk (lane / MF) of this lane
  const int fr = lane & (MF - 1), fc = lane / MF;
  uint16_t* const st[4] = {s0, s1, s2, s3};

  auto issue = [&](int kt, uint16_t* sp) {
    const uint32_t kb = 2u * (uint32_t)(kt * BKD);
    const uint32_t kbb = BKN ? (uint32_t)kt * kb_step_b : kb;
#pragma unroll
    for (int i = 0; i < A_INS; ++i)
      dma16_asm(reinterpret_cast<const char*>(A), oa[i] + kb, sp + (i * NW + wid) * 512);
#pragma unroll
    for (int b = 0; b < NB; ++b)
#pragma unroll
      for (int i = 0; i < B_INS; ++i)
        dma16_asm(reinterpret_cast<const char*>(Bm[b]), ob[i] + kbb, sp + (BM + b * BN) * BKD + (i * NW + wid) * 512);
  };
  u32x4 fa[FM], fb[NB][FN], fbn[NB][FN];
  auto frag = [&](const uint16_t* base, int row, int s) -> u32x4 {
    return *reinterpret_cast<const u32x4*>(&base[row * BKD + G::swz(row, s * (KS / 8) + fc) * 8]);
  };
  auto load_a = [&](const uint16_t* sp, int s, int i0, int i1) {
#pragma unroll
    for (int i = i0; i < i1; ++i) fa[i] = frag(sp, wm * WTM + i * MF + fr, s);
  };
  auto load_b = [&](const uint16_t* sp, int s, u32x4 (*dst)[FN]) {
#pragma unroll
    for (int b = 0; b < NB; ++b)
#pragma unroll
      for (int j = 0; j < FN; ++j) {
        if constexpr (BKN) {
          // k = 32 s + 8 (lane / 16) + 0..3 and + 4..7 for n = wn * WTN + 16 j + lane % 16
          const uint16_t* bs = sp + (BM + b * BN) * BKD;
          const int row = s * 32 + 8 * fc + (fr >> 2);
          const int col = wn * WTN + j * 16 + 4 * (fr & 3);
          const uint16_t* p = bs + row * BN + (((col >> 3) ^ bkn_swz<BN>(row)) * 8) + (col & 7);
          const u32x2 lo = lds_tr16(p);
          const u32x2 hi = lds_tr16(p + 4 * BN);  // rows + 4 share the swizzle
          dst[b][j] = u32x4{lo[0], lo[1], hi[0], hi[1]};
        } else {
          dst[b][j] = frag(sp + (BM + b * BN) * BKD, wn * WTN + j * MF + fr, s);
        }
      }
  };
  auto mfma_rows = [&](int i0, int i1) {
#pragma unroll
    for (int b = 0; b < NB; ++b)
#pragma unroll
      for (int i = i0; i < i1; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j) acc[b][i][j] = mfma_tile<T, MF>(fb[b][j], fa[i], acc[b][i][j]);
  };
  const int KT = K / BKD;
  // One k-step: first half of the MFMAs; at a tile's last step (cross) wait until the next tile
  // has landed (NS - 2 later tiles may still be in flight), barrier (every wave holds this tile's
  // fragments, so its stage is free) and refill the stage with tile refill_kt (clamped: past the
  // end it re-fetches the last tile into a stage nobody reads again); the next step's fragments
  // load around the second half.
  auto kstep = [&](const uint16_t* nsp, int ns, bool cross, uint16_t* rsp, int refill_kt) {
    mfma_rows(0, H);
    __builtin_amdgcn_sched_barrier(0);
    if (cross) {
      dma_barrier<(NS - 2) * INS>();
      issue(refill_kt, rsp);
    }
    load_a(nsp, ns, 0, H);
    load_b(nsp, ns, fbn);
    __builtin_amdgcn_sched_barrier(0);
    mfma_rows(H, FM);
    __builtin_amdgcn_sched_barrier(0);
    load_a(nsp, ns, H, FM);
#pragma unroll
    for (int b = 0; b < NB; ++b)
#pragma unroll
      for (int j = 0; j < FN; ++j) fb[b][j] = fbn[b][j];
  };
#pragma unroll
  for (int i = 0; i < NS; ++i) issue(min(i, KT - 1), st[i]);
  dma_barrier<(NS - 1) * INS>();
  load_a(s0, 0, 0, FM);
  load_b(s0, 0, fb);
  for (int kt = 0; kt < KT; kt += NS) {
#pragma unroll
    for (int u = 0; u < NS; ++u) {
      const int t = kt + u;
      if (t < KT) {  // uniform over the block
#pragma unroll
        for (int s = 0; s < STEPS; ++s) {
          if (s + 1 < STEPS) kstep(st[u], s + 1, false, st[u], 0);
          else kstep(st[(u + 1) % NS], 0, true, st[u], min(t + NS, KT - 1));
        }
      }
    }
  }
  wait_vmcnt<0>();  // no DMA may still target this block's LDS when its waves end
}

template <typename T, int BM, int BN, int WM, int WN, int NB, int EPI, int BKD, int NS, bool BKN, int MF>
__global__ __launch_bounds__(WM* WN* kWave) void gemm_dma(
    const uint16_t* __restrict__ A, const uint16_t* __restrict__ B0, const uint16_t* __restrict__ B1,
    uint16_t* __restrict__ C, int M, int N, int K, int64_t lda, int64_t ldb, int64_t ldc,
    int tiles_m, int tiles_n, EpiArgs ep) {
  constexpr int NW = WM * WN;
  constexpr int WTM = BM / WM, WTN = BN / WN;
  constexpr int FM = WTM / MF, FN = WTN / MF;  // MFMA fragments per wave along M and N
  constexpr int RPI = DmaGeom<BKD>::RPI;  // tile rows per DMA instruction (1 KB)
  using GB = DmaB<BN, BKD, BKN>;
  constexpr int A_INS = BM / RPI / NW;  // DMA instructions per wave per tile for A
  constexpr int B_INS = GB::kRows / GB::RPI / NW;  // ... per B matrix
  static_assert(A_INS * RPI * NW == BM && B_INS * GB::RPI * NW == GB::kRows, "tile rows split over waves");
  static_assert(4 * (A_INS + NB * B_INS) < 64, "outstanding DMA fits vmcnt");
  static_assert(FM % 2 == 0, "two MFMA halves per k-step");
  constexpr int kStage = (BM + NB * BN) * BKD;  // elements per stage
  __shared__ __attribute__((aligned(1024))) uint16_t sS0[kStage];
  __shared__ __attribute__((aligned(1024))) uint16_t sS1[kStage];
  __shared__ __attribute__((aligned(1024))) uint16_t sS2[NS > 2 ? kStage : 1];
  __shared__ __attribute__((aligned(1024))) uint16_t sS3[NS > 3 ? kStage : 1];

  if constexpr (EPI == kEpiPartial) {
    const int z = (int)blockIdx.y;  // K slice
    A += z * ep.split_a;
    B0 += z * ep.split_b;
    C += 2 * z * ep.split_c;  // fp32 workspace addressed in 16-bit units
  }
  batch_bases(A, B0, C, ep);
  int tm, tn;
  tile_coords(tiles_m, tiles_n, &tm, &tn);
  const int m0 = tm * BM, n0 = tn * BN;
  const int lane = lane_id();
  const int wid = __builtin_amdgcn_readfirstlane(wave_id());  // wave-uniform: LDS bases in SGPRs
  const int wm = wid / WN, wn = wid % WN;
  const int r_in = lane / (64 / RPI), pc = lane % (64 / RPI);

  // Per-lane byte offsets (fixed over k; the host guarantees M * lda and N * ldb elements fit
  // 31 bits, so bytes fit 32) of the row and chunk each DMA instruction fetches: physical chunk pc
  // of a row holds logical chunk swz(row, pc) (each XOR pattern is its own inverse).
  uint32_t oa[A_INS];
#pragma unroll
  for (int i = 0; i < A_INS; ++i) {
    const int row = (i * NW + wid) * RPI + r_in;
    const int lc = DmaGeom<BKD>::swz(row, pc);
    oa[i] = 2u * (uint32_t)(min(m0 + row, M - 1) * (int)lda + lc * 8);
  }
  uint32_t ob[B_INS];
#pragma unroll
  for (int i = 0; i < B_INS; ++i) {
    if constexpr (BKN) {
      // tile row = k (relative to the tile's first k), BN / 8 chunks per row; columns past N are
      // clamped onto the last full chunk (their results are never stored)
      constexpr int CPR = BN / 8;
      const int row = (i * NW + wid) * GB::RPI + lane / CPR;
      const int lc = (lane % CPR) ^ bkn_swz<BN>(row);
      ob[i] = 2u * (uint32_t)(row * (int)ldb + min(n0 + lc * 8, N - 8));
    } else {
      const int row = (i * NW + wid) * RPI + r_in;
      const int lc = DmaGeom<BKD>::swz(row, pc);
      ob[i] = 2u * (uint32_t)(min(n0 + row, N - 1) * (int)ldb + lc * 8);
    }
  }
  const uint32_t kb_step_b = 2u * (uint32_t)BKD * (uint32_t)ldb;  // B bytes per k-tile ([K, N] B)

  using Acc = typename MfmaAcc<MF>::type;
  Acc acc[NB][FM][FN];
#pragma unroll
  for (int b = 0; b < NB; ++b)
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
      for (int j = 0; j < FN; ++j)
#pragma unroll
        for (int e = 0; e < (int)(sizeof(Acc) / 4); ++e) acc[b][i][j][e] = 0.f;

  gemm_dma_ns_kloop<T, BM, BN, WM, WN, NB, BKD, NS, BKN, MF>(acc, A, B0, B1, oa, ob, kb_step_b, K, wid, wm, wn,
                                                             lane, sS0, sS1, sS2, sS3);

  // 16x16 fragment: lane holds C[m0' + lane % 16][n0' + 4 (lane / 16) + 0..3]
  const int fr = lane & 15, fc = lane >> 4;
  tile_epilogue<T, NB, EPI, true, FM, FN>(C, B1, ldc, M, N, m0 + wm * WTM + fr, n0 + wn * WTN + fc * 4, acc, ep);
}

// --------------------------------------------------------------------------------------------
// fp32 GEMM: v_mfma_f32_16x16x4_f32 keeps full fp32 products (no reduced-precision inputs).
// Block 128x128x16, 4 waves of 64x64. A: [BM][BK+1] (padded), B: [BK][BN+16] for [K,N] input or
// [BN][BK+1] for [N,K] input.
// --------------------------------------------------------------------------------------------
constexpr int kF32BM = 128, kF32BN = 128, kF32BK = 16;

// s += v with the lost low-order bits kept in c (Kahan). No multiplies, so no contraction applies.
__device__ __forceinline__ void kahan_add(f32x4& s, f32x4& c, const f32x4& v) {
  const f32x4 y = v - c;
  const f32x4 t = s + y;
  c = (t - s) - y;
  s = t;
}

template <bool BT>
__global__ __launch_bounds__(256) void gemm_f32(const float* __restrict__ A, const float* __restrict__ B,
                                                float* __restrict__ C, int M, int N, int K,
                                                int64_t lda, int64_t ldb, int64_t ldc, int tiles_m,
                                                int tiles_n, int64_t batch_a, int64_t batch_b,
                                                int64_t batch_c) {
  constexpr int BM = kF32BM, BN = kF32BN, BK = kF32BK;
  constexpr int PA = BK + 1;
  constexpr int PBN = BN + 16;
  __shared__ float sA[2][BM * PA];
  __shared__ float sB[2][BT ? BN * PA : BK * PBN];
  if (gridDim.z > 1) {  // batch item blockIdx.z (ak_gemm_batched)
    const int64_t z = blockIdx.z;
    A += z * batch_a;
    B += z * batch_b;
    C += z * batch_c;
  }
  int tm, tn;
  tile_coords(tiles_m, tiles_n, &tm, &tn);
  const int m0 = tm * BM, n0 = tn * BN;
  const int tid = threadIdx.x, lane = lane_id(), wid = wave_id();
  const int wm = wid >> 1, wn = wid & 1;
  float ra[8], rb[8];
  auto gload = [&](int k0) {
#pragma unroll
    for (int i = 0; i < 8; ++i) {  // A: 128 x 16, element e = tid + i*256
      const int e = tid + i * 256;
      const int row = e / BK, k = e % BK;
      ra[i] = (m0 + row < M && k0 + k < K) ? A[(int64_t)(m0 + row) * lda + k0 + k] : 0.f;
    }
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int e = tid + i * 256;
      if constexpr (BT) {  // [N,K]: 128 x 16
        const int row = e / BK, k = e % BK;
        rb[i] = (n0 + row < N && k0 + k < K) ? B[(int64_t)(n0 + row) * ldb + k0 + k] : 0.f;
      } else {  // [K,N]: 16 x 128
        const int k = e / BN, n = e % BN;
        rb[i] = (k0 + k < K && n0 + n < N) ? B[(int64_t)(k0 + k) * ldb + n0 + n] : 0.f;
      }
    }
  };
  auto sstore = [&](int st) {
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int e = tid + i * 256;
      sA[st][(e / BK) * PA + e % BK] = ra[i];
      if constexpr (BT) sB[st][(e / BK) * PA + e % BK] = rb[i];
      else sB[st][(e / BN) * PBN + e % BN] = rb[i];
    }
  };
  f32x4 acc[4][4], comp[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = comp[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};
  const int KT = (K + BK - 1) / BK;
  gload(0);
  sstore(0);
  __syncthreads();
  const int fr = lane & 15, fk = lane >> 4;
  for (int kt = 0; kt < KT; ++kt) {
    const int cur = kt & 1;
    if (kt + 1 < KT) gload((kt + 1) * BK);
    // Two-level sum: each k-tile accumulates from zero and is then added to the total, which
    // keeps fp32 rounding error of long dot products about sqrt(BK) times smaller.
    f32x4 part[4][4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int j = 0; j < 4; ++j) part[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int s = 0; s < BK / 4; ++s) {
      const int k = s * 4 + fk;
      float fa[4], fb[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) fa[i] = sA[cur][(wm * 64 + i * 16 + fr) * PA + k];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int n = wn * 64 + j * 16 + fr;
        fb[j] = BT ? sB[cur][n * PA + k] : sB[cur][k * PBN + n];
      }
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) part[i][j] = __builtin_amdgcn_mfma_f32_16x16x4f32(fb[j], fa[i], part[i][j], 0, 0, 0);
    }
    // Kahan-compensated outer sum over k-tiles: the running total's rounding error is carried
    // in `comp` and fed back, so long K (8192+) stays within the fp32 tolerance.
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int j = 0; j < 4; ++j) kahan_add(acc[i][j], comp[i][j], part[i][j]);
    if (kt + 1 < KT) sstore(cur ^ 1);
    __syncthreads();
  }
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int m = m0 + wm * 64 + i * 16 + fr;
    if (m >= M) continue;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int n = n0 + wn * 64 + j * 16 + fk * 4;
#pragma unroll
      for (int e = 0; e < 4; ++e)
        if (n + e < N) C[(int64_t)m * ldc + n + e] = acc[i][j][e];
    }
  }
}

// --------------------------------------------------------------------------------------------
// Host dispatch
// --------------------------------------------------------------------------------------------
struct TileCfg {
  int bm, bn;
};

// Pick the tile that keeps the 256 CUs busiest: fraction of CU-slots doing useful work over the
// launch, weighted by the per-tile efficiency of smaller tiles (more LDS and L2 traffic per flop).
// wide192: also consider 256x192 tiles (the LDS-DMA kernel with nn.Linear-layout B; 2048 x 6144,
// a fused QKV projection, is then exactly one tile per CU). small64: also consider 64x64 tiles
// (the same kernel, for grids that 128x128 tiles leave mostly idle).
static TileCfg pick_tile(int64_t M, int64_t N, int nb, bool wide192 = false, bool small64 = false,
                         int64_t batch = 1) {
  const TileCfg cands[] = {{256, 256}, {256, 128}, {128, 128}, {256, 192}, {64, 64}};
  // relative per-flop throughput of the tiles (bf16, MI355X): 4096^3 on 256x256 1230 TF/s,
  // 2048x4096x4096 on 256x128 1084 TF/s, 2048x6144x4096 on 128x128 786 TF/s, on 256x192 1108 TF/s;
  // 64x64 weighted so that it wins only where 128x128 tiles fill under a third of the CUs (cold,
  // f16: 2048x768x768 16.4 -> 13.8 us, 2048x768x3072 41.7 -> 37.3 us, 1024^3 NN 17.3 -> 15.5 us,
  // 4096x768x768 unchanged at 15.1 us; with a weight of 0.5 it was also picked there and took
  // 16.3 us)
  const double eff[] = {1.0, 0.88, 0.64, 0.88, 0.35};
  const int cus = 256;
  TileCfg best = cands[2];
  double best_s = -1.0;
  for (int i = 0; i < 5; ++i) {
    if ((i == 3 && !(wide192 && nb == 1)) || (i == 4 && !(small64 && nb == 1))) continue;
    const int bn = cands[i].bn / (nb == 2 ? 2 : 1);
    const int64_t tiles = cdiv(M, cands[i].bm) * cdiv(N, bn) * batch;
    const int64_t waves = cdiv(tiles, cus);
    const double used = (double)tiles / (double)(waves * cus);
    // padding waste inside edge tiles
    const double pad = (double)(M * N) / (double)(cdiv(M, cands[i].bm) * cands[i].bm * cdiv(N, bn) * bn);
    const double s = used * pad * eff[i];
    if (s > best_s + 1e-9) {
      best_s = s;
      best = cands[i];
    }
  }
  return best;
}

template <typename T, bool BT, bool VEC, int BM, int BN, int WM, int WN, int NB, int EPI>
static void launch_gemm_cfg(const void* A, const void* B0, const void* B1, void* C, int M, int N,
                            int K, int64_t lda, int64_t ldb, int64_t ldc, hipStream_t s, const EpiArgs& ep) {
  const int tiles_m = (int)cdiv(M, BM), tiles_n = (int)cdiv(N, BN);
  gemm_mfma<T, BT, VEC, BM, BN, WM, WN, NB, EPI><<<dim3(tiles_m * tiles_n, 1, ep.batch), WM * WN * kWave, 0, s>>>(
      (const uint16_t*)A, (const uint16_t*)B0, (const uint16_t*)B1, (uint16_t*)C, M, N, K, lda, ldb,
      ldc, tiles_m, tiles_n, ep);
}

// Waves along N of the 256x256 tile: 4 (8 waves of 128x64; measured faster than 4 waves of
// 128x128, one wave per SIMD with accumulators in AGPRs).
constexpr int kBigWN = 4;

template <typename T, bool BT, bool VEC, int NB, int EPI>
static void launch_gemm_tiled(const void* A, const void* B0, const void* B1, void* C, int M, int N,
                              int K, int64_t lda, int64_t ldb, int64_t ldc, hipStream_t s, const EpiArgs& ep) {
  const TileCfg t = pick_tile(M, N, NB, false, false, ep.batch);
  if constexpr (NB == 1) {
    if (t.bm == 256 && t.bn == 256)
      launch_gemm_cfg<T, BT, VEC, 256, 256, 2, kBigWN, 1, EPI>(A, B0, B1, C, M, N, K, lda, ldb, ldc, s, ep);
    else if (t.bm == 256)
      launch_gemm_cfg<T, BT, VEC, 256, 128, 4, 2, 1, EPI>(A, B0, B1, C, M, N, K, lda, ldb, ldc, s, ep);
    else
      launch_gemm_cfg<T, BT, VEC, 128, 128, 2, 2, 1, EPI>(A, B0, B1, C, M, N, K, lda, ldb, ldc, s, ep);
  } else {
    if (t.bm == 256 && t.bn == 256)
      launch_gemm_cfg<T, BT, VEC, 256, 128, 2, 4, 2, EPI>(A, B0, B1, C, M, N, K, lda, ldb, ldc, s, ep);
    else if (t.bm == 256)
      launch_gemm_cfg<T, BT, VEC, 256, 64, 4, 2, 2, EPI>(A, B0, B1, C, M, N, K, lda, ldb, ldc, s, ep);
    else
      launch_gemm_cfg<T, BT, VEC, 128, 64, 2, 2, 2, EPI>(A, B0, B1, C, M, N, K, lda, ldb, ldc, s, ep);
  }
}

constexpr int kCUs = 256;  // MI355X compute units

template <typename T, int BM, int BN, int WM, int WN, int NB, int EPI, int BKD, int NS, bool BKN>
static void launch_dma_kernel(const void* A, const void* B0, const void* B1, void* C, int M, int N, int K,
                              int64_t lda, int64_t ldb, int64_t ldc, int tiles_m, int tiles_n, hipStream_t s,
                              const EpiArgs& ep) {
  // MFMA shape 16x16x32 (32x32x16 fragments measured 4-10 % slower on every workload)
  constexpr int MF = 16;
  gemm_dma<T, BM, BN, WM, WN, NB, EPI, BKD, NS, BKN, MF><<<dim3(tiles_m * tiles_n, ep.splits, ep.batch), WM * WN * kWave, 0, s>>>(
      (const uint16_t*)A, (const uint16_t*)B0, (const uint16_t*)B1, (uint16_t*)C, M, N, K, lda, ldb, ldc,
      tiles_m, tiles_n, ep);
}

// Pipeline plan per tile shape: stage bytes (BM + NB * BN) * BKD * 2 and the 160 KB of LDS fix
// how many stages fit.
// Waves along N of the 128x128 tile: 4 (8 waves of 64x32, two per SIMD). Measured, cold, 2048^3
// (256 tiles, one per CU): f16 NN 26.8 us against 36.5 us with 4 waves of 64x64 (stock hipBLASLt
// 32.0), bf16 NT 26.4 against 36.0 (28.9); three or four stages for the 4-wave tile reach
// 28.2-29.4 us. Shapes on other tiles are unchanged.
constexpr int kSmallWN = 4;

template <int BM, int BN, int NB, int NW>
struct DmaPlan {
  static constexpr int kStage64 = (BM + NB * BN) * 64 * 2;
  static constexpr int kFit64 = 163840 / kStage64;
  static constexpr bool kOk32 = BM % (16 * NW) == 0 && BN % (16 * NW) == 0;
  // Three 64-deep stages where they fit beside 8 waves, else two. Measured (bf16, NT):
  // 2048x4096x4096 on 256x128 tiles 83.5 us two-stage -> 63.4 us three-stage; 4096^3 on 256x256
  // 107.4 us two-stage (four 32-deep stages: 121.2 us, the doubled barrier count outweighs the
  // deeper queue). The 64x64 tile (4 waves, 16 KB stages, picked for grids that larger tiles leave
  // mostly idle) waits on transfer latency, not MFMAs: four stages keep three tiles in flight
  // (cold, f16: 1024^3 15.5 -> 10.8 us, 2048x768x3072 37.0 -> 29.8 us, 2048x1024x1024 16.6 ->
  // 14.6 us; four stages on 128x128 tiles gained nothing).
  static constexpr int BKD = 64;
  static constexpr int NS = BM == 64 ? 4 : (kFit64 >= 3 && NW == 8) ? 3 : 2;
};

template <typename T, int BM, int BN, int WM, int WN, int NB, int EPI, bool BKN>
static void launch_dma_cfg(const void* A, const void* B0, const void* B1, void* C, int M, int N, int K,
                           int64_t lda, int64_t ldb, int64_t ldc, hipStream_t s, const EpiArgs& ep) {
  const int tiles_m = (int)cdiv(M, BM), tiles_n = (int)cdiv(N, BN);
  using P = DmaPlan<BM, BN, NB, WM * WN>;
  // Four 32-deep stages when the grid fills at most half the CUs (each block's own DMA latency is
  // then exposed; measured 2048x1024x4096: 50.9 us against 59.0 us two-stage). With more tiles the
  // 64-deep pair is faster per tile (2048x6144x4096 on 192 tiles of 256x256: 109.9 us against
  // 127.5 us).
  constexpr bool kOk32 = P::kOk32;
  if (kOk32 && 2 * tiles_m * tiles_n * ep.splits * ep.batch <= kCUs) {
    if constexpr (kOk32)
      launch_dma_kernel<T, BM, BN, WM, WN, NB, EPI, 32, 4, BKN>(A, B0, B1, C, M, N, K, lda, ldb, ldc, tiles_m,
                                                                tiles_n, s, ep);
    return;
  }
  launch_dma_kernel<T, BM, BN, WM, WN, NB, EPI, P::BKD, P::NS, BKN>(A, B0, B1, C, M, N, K, lda, ldb, ldc, tiles_m,
                                                                    tiles_n, s, ep);
}

template <typename T, int NB, int EPI, bool BKN>
static void launch_gemm_dma(const void* A, const void* B0, const void* B1, void* C, int M, int N, int K,
                            int64_t lda, int64_t ldb, int64_t ldc, hipStream_t s, const EpiArgs& ep) {
  // 256x192 needs [N, K] B: a [K, N] B tile row of 192 elements does not split into 1 KB transfers
  const TileCfg t = pick_tile(M, N, NB, !BKN, EPI != kEpiPartial, ep.batch);
  if constexpr (NB == 1) {
    if constexpr (!BKN) {
      if (t.bm == 256 && t.bn == 192) {
        launch_dma_cfg<T, 256, 192, 2, 4, 1, EPI, false>(A, B0, B1, C, M, N, K, lda, ldb, ldc, s, ep);
        return;
      }
    }
    if (t.bm == 64) {
      launch_dma_cfg<T, 64, 64, 2, 2, 1, EPI, BKN>(A, B0, B1, C, M, N, K, lda, ldb, ldc, s, ep);
      return;
    }
    if (t.bm == 256 && t.bn == 256)
      launch_dma_cfg<T, 256, 256, 2, kBigWN, 1, EPI, BKN>(A, B0, B1, C, M, N, K, lda, ldb, ldc, s, ep);
    else if (t.bm == 256) launch_dma_cfg<T, 256, 128, 4, 2, 1, EPI, BKN>(A, B0, B1, C, M, N, K, lda, ldb, ldc, s, ep);
    else launch_dma_cfg<T, 128, 128, 2, kSmallWN, 1, EPI, BKN>(A, B0, B1, C, M, N, K, lda, ldb, ldc, s, ep);
  } else {
    static_assert(!BKN, "gate/up weights are [H, D]");
    if (t.bm == 256 && t.bn == 256)
      launch_dma_cfg<T, 256, 128, 2, kBigWN, 2, EPI, false>(A, B0, B1, C, M, N, K, lda, ldb, ldc, s, ep);
    else if (t.bm == 256) launch_dma_cfg<T, 256, 64, 4, 2, 2, EPI, false>(A, B0, B1, C, M, N, K, lda, ldb, ldc, s, ep);
    else launch_dma_cfg<T, 128, 64, 2, 2, 2, EPI, false>(A, B0, B1, C, M, N, K, lda, ldb, ldc, s, ep);
  }
}

template <typename T, int NB, int EPI>
static int launch_gemm16(const void* A, const void* B0, const void* B1, void* C, int64_t M,
                         int64_t N, int64_t K, int64_t lda, int64_t ldb, int64_t ldc, bool bt,
                         hipStream_t s, const EpiArgs& ep = EpiArgs{}) {
  // vec: A and B load as 16-byte k-chunks (C's alignment does not matter: the epilogue checks each
  // 8-byte store)
  bool vec = K % 8 == 0 && lda % 8 == 0 && ldb % 8 == 0 && host_aligned16(A) && host_aligned16(B0) &&
             (!B1 || EPI == kEpiBias || EPI == kEpiBiasGelu || host_aligned16(B1)) && ep.batch_a % 8 == 0 &&
             ep.batch_b % 8 == 0;
  if (!bt) vec = vec && N % 8 == 0;
  const int m = (int)M, n = (int)N, k = (int)K;
  // LDS-DMA path: nn.Linear-layout B, K a multiple of 64, 32-bit element offsets
  const bool fits32 = M * lda < INT_MAX && N * ldb < INT_MAX;
  if (bt && vec && K % kBK == 0 && K > 0 && fits32) {
    launch_gemm_dma<T, NB, EPI, false>(A, B0, B1, C, m, n, k, lda, ldb, ldc, s, ep);
    return record_launch();
  }
  // [K, N] B (torch.matmul's layout) on the same pipeline, fragments read through LDS transposes
  if constexpr (NB == 1) {
    const bool fits32_kn = M * lda < INT_MAX && K * ldb < INT_MAX;
    if (!bt && vec && K % kBK == 0 && K > 0 && N >= 8 && fits32_kn) {
      launch_gemm_dma<T, 1, EPI, true>(A, B0, B1, C, m, n, k, lda, ldb, ldc, s, ep);
      return record_launch();
    }
  }
  if (bt) {
    if (vec) launch_gemm_tiled<T, true, true, NB, EPI>(A, B0, B1, C, m, n, k, lda, ldb, ldc, s, ep);
    else launch_gemm_tiled<T, true, false, NB, EPI>(A, B0, B1, C, m, n, k, lda, ldb, ldc, s, ep);
  } else {
    if constexpr (NB == 1) {
      if (vec) launch_gemm_tiled<T, false, true, 1, EPI>(A, B0, B1, C, m, n, k, lda, ldb, ldc, s, ep);
      else launch_gemm_tiled<T, false, false, 1, EPI>(A, B0, B1, C, m, n, k, lda, ldb, ldc, s, ep);
    } else {
      return AK_EINVAL;
    }
  }
  return record_launch();
}

// ---------------------------------------------------------------------------------------------
// Split-K for grids that leave most CUs idle (few output tiles, long K): slice z of the K range runs
// as grid row z of the LDS-DMA kernel and stores fp32 partial tiles to the caller's workspace
// [splits][M][N]; splitk_reduce then adds the slices in order z = 0, 1, ... and rounds once, so the
// result is deterministic and keeps "fp32 accumulation, one output rounding".
// ---------------------------------------------------------------------------------------------
template <typename T>
__global__ __launch_bounds__(256) void splitk_reduce(const float* __restrict__ ws, uint16_t* __restrict__ C, int M,
                                                     int N, int64_t ldc, int splits) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;  // one 4-column group per thread
  const int groups_per_row = N / 4;
  if (i >= (int64_t)M * groups_per_row) return;
  const int m = (int)(i / groups_per_row), n = (int)(i % groups_per_row) * 4;
  const int64_t plane = (int64_t)M * N;
  const float* p = ws + (int64_t)m * N + n;
  f32x4 acc = *reinterpret_cast<const f32x4*>(p);
  for (int z = 1; z < splits; ++z) {
    const f32x4 v = *reinterpret_cast<const f32x4*>(p + z * plane);
#pragma unroll
    for (int e = 0; e < 4; ++e) acc[e] += v[e];
  }
  u32x2 o;
  o[0] = (uint32_t)T::from_f(acc[0]) | ((uint32_t)T::from_f(acc[1]) << 16);
  o[1] = (uint32_t)T::from_f(acc[2]) | ((uint32_t)T::from_f(acc[3]) << 16);
  *reinterpret_cast<u32x2*>(C + (int64_t)m * ldc + n) = o;
}

// K slices for a plain f16 / bf16 GEMM on the LDS-DMA path, 1 when splitting does not pay: the
// chosen tiling must fill at most half the CUs, each slice keeps at least 1024 of K (sixteen
// 64-deep tiles) and a multiple of 64, and slices stop doubling once tiles x slices would pass the
// CU count.
static int splitk_slices(int64_t M, int64_t N, int64_t K, int64_t lda, int64_t ldb, int64_t ldc, bool bt) {
  if (M <= 0 || N <= 0 || K <= 0 || N % 4 != 0 || ldc % 4 != 0 || lda % 8 != 0 || ldb % 8 != 0) return 1;
  if (M * lda >= INT_MAX || (bt ? N : K) * ldb >= INT_MAX || M * N * 8 >= INT_MAX) return 1;
  // [K, N] B runs the LDS-DMA kernel only with N a multiple of 8 (its 16-byte column chunks), the
  // same rule as the unsplit path
  if (!bt && N % 8 != 0) return 1;
  const TileCfg t = pick_tile(M, N, 1, !bt);
  const int64_t tiles = cdiv(M, t.bm) * cdiv(N, t.bn);
  if (2 * tiles > kCUs) return 1;
  int s = 1;
  // Slices stay at least 1024 deep: shorter ones lose more to the pipeline fill and the fp32
  // partial round trip than the extra CUs win (1024^3 f16: 11.9 us unsplit, 18.0 us in 4 slices;
  // 1024x1024x4096: 32.5 us unsplit, 22.8 us in 4 slices).
  while (s < 8 && tiles * s * 2 <= kCUs && K % (64 * s * 2) == 0 && K / (s * 2) >= 1024) s *= 2;
  return s;
}

template <typename T>
static int launch_gemm16_splitk(const void* A, const void* B, void* C, int64_t M, int64_t N, int64_t K,
                                int64_t lda, int64_t ldb, int64_t ldc, bool bt, int splits, float* ws,
                                hipStream_t s) {
  EpiArgs ep;
  ep.splits = splits;
  const int64_t ks = K / splits;
  ep.split_a = ks;
  ep.split_b = bt ? ks : ks * ldb;
  ep.split_c = M * N;
  // partial tiles: the workspace is the output, row stride N
  if (bt) launch_gemm_dma<T, 1, kEpiPartial, false>(A, B, nullptr, ws, (int)M, (int)N, (int)ks, lda, ldb, N, s, ep);
  else launch_gemm_dma<T, 1, kEpiPartial, true>(A, B, nullptr, ws, (int)M, (int)N, (int)ks, lda, ldb, N, s, ep);
  const int64_t groups = M * (N / 4);
  splitk_reduce<T><<<(unsigned)cdiv(groups, 256), 256, 0, s>>>(ws, (uint16_t*)C, (int)M, (int)N, ldc, splits);
  return record_launch();
}

// batch > 1: grid z is the batch item, whose operands start z * batch_x elements further
static int launch_gemm32(const void* A, const void* B, void* C, int64_t M, int64_t N, int64_t K,
                         int64_t lda, int64_t ldb, int64_t ldc, bool bt, hipStream_t s, int batch = 1,
                         int64_t batch_a = 0, int64_t batch_b = 0, int64_t batch_c = 0) {
  const int tiles_m = (int)cdiv(M, kF32BM), tiles_n = (int)cdiv(N, kF32BN);
  const dim3 grid(tiles_m * tiles_n, 1, batch);
  if (bt)
    gemm_f32<true><<<grid, 256, 0, s>>>((const float*)A, (const float*)B, (float*)C, (int)M, (int)N, (int)K, lda,
                                        ldb, ldc, tiles_m, tiles_n, batch_a, batch_b, batch_c);
  else
    gemm_f32<false><<<grid, 256, 0, s>>>((const float*)A, (const float*)B, (float*)C, (int)M, (int)N, (int)K, lda,
                                         ldb, ldc, tiles_m, tiles_n, batch_a, batch_b, batch_c);
  return record_launch();
}

// fp32 gate/up: two fp32 GEMMs into a caller-visible layout is not possible without a
// workspace, so the fp32 fused MLP is served by a small elementwise-epilogue kernel over two
// fp32 GEMM outputs computed in place: h <- gate, then a second pass combines with up computed
// tile by tile. For simplicity and exactness fp32 uses one dedicated kernel instead.
__global__ __launch_bounds__(256) void gate_up_f32(const float* __restrict__ X, const float* __restrict__ Wg,
                                                   const float* __restrict__ Wu, float* __restrict__ Hout,
                                                   int M, int H, int D, int act, int tiles_m, int tiles_n) {
  // 64x64 tile, 4 waves of 32x32 (2x2 MFMA 16x16x4 per matrix)
  constexpr int BM = 64, BN = 64, BK = 16, PA = BK + 1;
  __shared__ float sX[BM * PA], sG[BN * PA], sU[BN * PA];
  int tm, tn;
  tile_coords(tiles_m, tiles_n, &tm, &tn);
  const int m0 = tm * BM, n0 = tn * BN;
  const int tid = threadIdx.x, lane = lane_id(), wid = wave_id();
  const int wm = wid >> 1, wn = wid & 1;
  const int fr = lane & 15, fk = lane >> 4;
  f32x4 ag[2][2], au[2][2], cg[2][2], cu[2][2];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j) ag[i][j] = au[i][j] = cg[i][j] = cu[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};
  for (int k0 = 0; k0 < D; k0 += BK) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int e = tid + i * 256;
      const int row = e / BK, k = e % BK;
      const bool kin = k0 + k < D;
      sX[row * PA + k] = (m0 + row < M && kin) ? X[(int64_t)(m0 + row) * D + k0 + k] : 0.f;
      sG[row * PA + k] = (n0 + row < H && kin) ? Wg[(int64_t)(n0 + row) * D + k0 + k] : 0.f;
      sU[row * PA + k] = (n0 + row < H && kin) ? Wu[(int64_t)(n0 + row) * D + k0 + k] : 0.f;
    }
    __syncthreads();
    f32x4 pg[2][2], pu[2][2];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int j = 0; j < 2; ++j) pg[i][j] = pu[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int s = 0; s < BK / 4; ++s) {
      const int k = s * 4 + fk;
      float fx[2], fg[2], fu[2];
#pragma unroll
      for (int i = 0; i < 2; ++i) fx[i] = sX[(wm * 32 + i * 16 + fr) * PA + k];
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        fg[j] = sG[(wn * 32 + j * 16 + fr) * PA + k];
        fu[j] = sU[(wn * 32 + j * 16 + fr) * PA + k];
      }
#pragma unroll
      for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j) {
          pg[i][j] = __builtin_amdgcn_mfma_f32_16x16x4f32(fg[j], fx[i], pg[i][j], 0, 0, 0);
          pu[i][j] = __builtin_amdgcn_mfma_f32_16x16x4f32(fu[j], fx[i], pu[i][j], 0, 0, 0);
        }
    }
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        kahan_add(ag[i][j], cg[i][j], pg[i][j]);
        kahan_add(au[i][j], cu[i][j], pu[i][j]);
      }
    __syncthreads();
  }
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const int m = m0 + wm * 32 + i * 16 + fr;
    if (m >= M) continue;
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int n = n0 + wn * 32 + j * 16 + fk * 4;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        if (n + e >= H) continue;
        float v;
        switch (act) {
          case kEpiSilu: v = gate_up<TF32, kEpiSilu>(ag[i][j][e], au[i][j][e]); break;
          case kEpiGelu: v = gate_up<TF32, kEpiGelu>(ag[i][j][e], au[i][j][e]); break;
          case kEpiRelu2: v = gate_up<TF32, kEpiRelu2>(ag[i][j][e], au[i][j][e]); break;
          default: v = gate_up<TF32, kEpiNone>(ag[i][j][e], au[i][j][e]); break;
        }
        Hout[(int64_t)m * H + n + e] = v;
      }
    }
  }
}

}  // namespace ak

using namespace ak;

extern "C" int ak_gemm(int dtype, const void* A, const void* B, void* C, int64_t M, int64_t N,
                       int64_t K, int64_t lda, int64_t ldb, int64_t ldc, int b_trans,
                       hipStream_t stream) {
  if (M < 0 || N < 0 || K < 0 || M > INT_MAX || N > INT_MAX || K > INT_MAX) return AK_EINVAL;
  if (M == 0 || N == 0) return AK_OK;
  if (!A || !B || !C) return AK_EINVAL;
  if (lda < K || ldc < N || ldb < (b_trans ? K : N)) return AK_EINVAL;
  if (cdiv(M, 128) * cdiv(N, 128) > INT_MAX) return AK_EINVAL;
  const bool bt = b_trans != 0;
  switch (dtype) {
    case AK_F32: return launch_gemm32(A, B, C, M, N, K, lda, ldb, ldc, bt, stream);
    case AK_F16: return launch_gemm16<TF16, 1, kEpiStore>(A, B, nullptr, C, M, N, K, lda, ldb, ldc, bt, stream);
    case AK_BF16: return launch_gemm16<TBF16, 1, kEpiStore>(A, B, nullptr, C, M, N, K, lda, ldb, ldc, bt, stream);
    default: return AK_EINVAL;
  }
}

extern "C" int ak_gemm_batched(int dtype, const void* A, const void* B, void* C, int64_t batch, int64_t M,
                               int64_t N, int64_t K, int64_t lda, int64_t ldb, int64_t ldc, int64_t stride_a,
                               int64_t stride_b, int64_t stride_c, int b_trans, hipStream_t stream) {
  if (batch < 0 || M < 0 || N < 0 || K < 0 || M > INT_MAX || N > INT_MAX || K > INT_MAX) return AK_EINVAL;
  if (batch == 0 || M == 0 || N == 0) return AK_OK;
  if (!A || !B || !C) return AK_EINVAL;
  if (lda < K || ldc < N || ldb < (b_trans ? K : N) || stride_a < 0 || stride_b < 0) return AK_EINVAL;
  // the batch items of C must not overlap (each is written once, in parallel)
  if (batch > 1 && stride_c < (M - 1) * ldc + N) return AK_EINVAL;
  if (cdiv(M, 128) * cdiv(N, 128) > INT_MAX) return AK_EINVAL;
  const bool bt = b_trans != 0;
  const int esz = dtype == AK_F32 ? 4 : 2;
  // grid z holds at most 65535 items: larger batches run in chunks
  constexpr int64_t kMaxZ = 65535;
  for (int64_t z0 = 0; z0 < batch; z0 += kMaxZ) {
    const int64_t nz = batch - z0 < kMaxZ ? batch - z0 : kMaxZ;
    const char* a = (const char*)A + z0 * stride_a * esz;
    const char* b = (const char*)B + z0 * stride_b * esz;
    char* c = (char*)C + z0 * stride_c * esz;
    int st = AK_OK;
    if (dtype == AK_F32) {
      st = launch_gemm32(a, b, c, M, N, K, lda, ldb, ldc, bt, stream, (int)nz, stride_a, stride_b, stride_c);
    } else {
      EpiArgs ep;
      ep.batch = (int)nz;
      ep.batch_a = stride_a;
      ep.batch_b = stride_b;
      ep.batch_c = stride_c;
      if (dtype == AK_F16) st = launch_gemm16<TF16, 1, kEpiStore>(a, b, nullptr, c, M, N, K, lda, ldb, ldc, bt, stream, ep);
      else if (dtype == AK_BF16) st = launch_gemm16<TBF16, 1, kEpiStore>(a, b, nullptr, c, M, N, K, lda, ldb, ldc, bt, stream, ep);
      else return AK_EINVAL;
    }
    if (st != AK_OK) return st;
  }
  return AK_OK;
}

extern "C" int64_t ak_gemm_workspace_bytes(int dtype, int64_t M, int64_t N, int64_t K, int64_t lda, int64_t ldb,
                                           int64_t ldc, int b_trans) {
  if (dtype != AK_F16 && dtype != AK_BF16) return 0;
  if (M < 0 || N < 0 || K < 0 || M > INT_MAX || N > INT_MAX || K > INT_MAX) return 0;
  const int sl = splitk_slices(M, N, K, lda, ldb, ldc, b_trans != 0);
  return sl > 1 ? (int64_t)sl * M * N * (int64_t)sizeof(float) : 0;
}

extern "C" int ak_gemm_ws(int dtype, const void* A, const void* B, void* C, int64_t M, int64_t N, int64_t K,
                          int64_t lda, int64_t ldb, int64_t ldc, int b_trans, void* workspace,
                          int64_t workspace_bytes, hipStream_t stream) {
  const int64_t need = ak_gemm_workspace_bytes(dtype, M, N, K, lda, ldb, ldc, b_trans);
  const bool aligned = host_aligned16(A) && host_aligned16(B) && (((uintptr_t)C) & 7u) == 0 &&
                       host_aligned16(workspace);
  if (need == 0 || !workspace || workspace_bytes < need || !aligned || lda < K || ldc < N ||
      ldb < (b_trans ? K : N))
    return ak_gemm(dtype, A, B, C, M, N, K, lda, ldb, ldc, b_trans, stream);
  const int sl = (int)(need / (M * N * (int64_t)sizeof(float)));
  if (dtype == AK_F16)
    return launch_gemm16_splitk<TF16>(A, B, C, M, N, K, lda, ldb, ldc, b_trans != 0, sl, (float*)workspace, stream);
  return launch_gemm16_splitk<TBF16>(A, B, C, M, N, K, lda, ldb, ldc, b_trans != 0, sl, (float*)workspace, stream);
}

extern "C" int ak_gemm_residual(int dtype, const void* A, const void* B, const void* R, void* C, int64_t M,
                                int64_t N, int64_t K, int64_t lda, int64_t ldb, int64_t ldc, int b_trans,
                                hipStream_t stream) {
  if (M < 0 || N < 0 || K < 0 || M > INT_MAX || N > INT_MAX || K > INT_MAX) return AK_EINVAL;
  if (M == 0 || N == 0) return AK_OK;
  if (!A || !B || !R || !C) return AK_EINVAL;
  if (lda < K || ldc < N || ldb < (b_trans ? K : N)) return AK_EINVAL;
  if (cdiv(M, 128) * cdiv(N, 128) > INT_MAX) return AK_EINVAL;
  // R is read and C written element by element in one pass: they must not overlap
  const uintptr_t r0 = (uintptr_t)R, c0 = (uintptr_t)C;
  const uintptr_t span = (uintptr_t)(((M - 1) * ldc + N) * 2);
  if (r0 < c0 + span && c0 < r0 + span) return AK_EINVAL;
  const bool bt = b_trans != 0;
  switch (dtype) {
    case AK_F16: return launch_gemm16<TF16, 1, kEpiResidual>(A, B, R, C, M, N, K, lda, ldb, ldc, bt, stream);
    case AK_BF16: return launch_gemm16<TBF16, 1, kEpiResidual>(A, B, R, C, M, N, K, lda, ldb, ldc, bt, stream);
    case AK_F32: return AK_EUNSUPPORTED;
    default: return AK_EINVAL;
  }
}

extern "C" int ak_gemm_bias(int dtype, const void* A, const void* B, const void* bias, void* C, int64_t M,
                            int64_t N, int64_t K, int64_t lda, int64_t ldb, int64_t ldc, int b_trans,
                            hipStream_t stream) {
  if (M < 0 || N < 0 || K < 0 || M > INT_MAX || N > INT_MAX || K > INT_MAX) return AK_EINVAL;
  if (M == 0 || N == 0) return AK_OK;
  if (!A || !B || !bias || !C) return AK_EINVAL;
  if (lda < K || ldc < N || ldb < (b_trans ? K : N)) return AK_EINVAL;
  if (cdiv(M, 128) * cdiv(N, 128) > INT_MAX) return AK_EINVAL;
  const bool bt = b_trans != 0;
  switch (dtype) {
    case AK_F16: return launch_gemm16<TF16, 1, kEpiBias>(A, B, bias, C, M, N, K, lda, ldb, ldc, bt, stream);
    case AK_BF16: return launch_gemm16<TBF16, 1, kEpiBias>(A, B, bias, C, M, N, K, lda, ldb, ldc, bt, stream);
    case AK_F32: return AK_EUNSUPPORTED;
    default: return AK_EINVAL;
  }
}

extern "C" int ak_gemm_bias_gelu(int dtype, const void* A, const void* B, const void* bias, void* C, int64_t M,
                                 int64_t N, int64_t K, int64_t lda, int64_t ldb, int64_t ldc, int b_trans,
                                 hipStream_t stream) {
  if (M < 0 || N < 0 || K < 0 || M > INT_MAX || N > INT_MAX || K > INT_MAX) return AK_EINVAL;
  if (M == 0 || N == 0) return AK_OK;
  if (!A || !B || !bias || !C) return AK_EINVAL;
  if (lda < K || ldc < N || ldb < (b_trans ? K : N)) return AK_EINVAL;
  if (cdiv(M, 128) * cdiv(N, 128) > INT_MAX) return AK_EINVAL;
  const bool bt = b_trans != 0;
  switch (dtype) {
    case AK_F16: return launch_gemm16<TF16, 1, kEpiBiasGelu>(A, B, bias, C, M, N, K, lda, ldb, ldc, bt, stream);
    case AK_BF16: return launch_gemm16<TBF16, 1, kEpiBiasGelu>(A, B, bias, C, M, N, K, lda, ldb, ldc, bt, stream);
    case AK_F32: return AK_EUNSUPPORTED;
    default: return AK_EINVAL;
  }
}

extern "C" int ak_gemm_bias_residual(int dtype, const void* A, const void* B, const void* bias, const void* R,
                                     void* C, int64_t M, int64_t N, int64_t K, int64_t lda, int64_t ldb,
                                     int64_t ldc, int b_trans, hipStream_t stream) {
  if (M < 0 || N < 0 || K < 0 || M > INT_MAX || N > INT_MAX || K > INT_MAX) return AK_EINVAL;
  if (M == 0 || N == 0) return AK_OK;
  if (!A || !B || !bias || !R || !C) return AK_EINVAL;
  if (lda < K || ldc < N || ldb < (b_trans ? K : N)) return AK_EINVAL;
  if (cdiv(M, 128) * cdiv(N, 128) > INT_MAX) return AK_EINVAL;
  // R is read and C written element by element in one pass: they must not overlap
  const uintptr_t r0 = (uintptr_t)R, c0 = (uintptr_t)C;
  const uintptr_t span = (uintptr_t)(((M - 1) * ldc + N) * 2);
  if (r0 < c0 + span && c0 < r0 + span) return AK_EINVAL;
  const bool bt = b_trans != 0;
  EpiArgs ep;
  ep.bias = (const uint16_t*)bias;
  switch (dtype) {
    case AK_F16: return launch_gemm16<TF16, 1, kEpiBiasResidual>(A, B, R, C, M, N, K, lda, ldb, ldc, bt, stream, ep);
    case AK_BF16: return launch_gemm16<TBF16, 1, kEpiBiasResidual>(A, B, R, C, M, N, K, lda, ldb, ldc, bt, stream, ep);
    case AK_F32: return AK_EUNSUPPORTED;
    default: return AK_EINVAL;
  }
}

extern "C" int ak_gemm_rope(int dtype, const void* A, const void* B, void* C, int64_t M, int64_t N, int64_t K,
                            int64_t lda, int64_t ldb, int64_t ldc, int b_trans, const float* cos_t,
                            const float* sin_t, int64_t seq_len, int64_t head_dim, int64_t rot_cols,
                            hipStream_t stream) {
  if (M < 0 || N < 0 || K < 0 || M > INT_MAX || N > INT_MAX || K > INT_MAX) return AK_EINVAL;
  if (head_dim <= 0 || head_dim % 4 != 0 || head_dim > INT_MAX) return AK_EINVAL;
  if (rot_cols < 0 || rot_cols > N || rot_cols % head_dim != 0) return AK_EINVAL;
  if (seq_len <= 0 || seq_len > INT_MAX) return AK_EINVAL;
  if (M == 0 || N == 0) return AK_OK;
  if (!A || !B || !C || (rot_cols > 0 && (!cos_t || !sin_t))) return AK_EINVAL;
  if ((((uintptr_t)cos_t) | ((uintptr_t)sin_t)) & 7u) return AK_EINVAL;  // pairs load as 8 bytes
  if (lda < K || ldc < N || ldb < (b_trans ? K : N)) return AK_EINVAL;
  if (cdiv(M, 128) * cdiv(N, 128) > INT_MAX) return AK_EINVAL;
  EpiArgs ep;
  ep.cos = cos_t;
  ep.sin = sin_t;
  ep.head_dim = (int)head_dim;
  ep.rot_cols = (int)rot_cols;
  ep.seq_len = (int)seq_len;
  const bool bt = b_trans != 0;
  switch (dtype) {
    case AK_F16: return launch_gemm16<TF16, 1, kEpiRope>(A, B, nullptr, C, M, N, K, lda, ldb, ldc, bt, stream, ep);
    case AK_BF16: return launch_gemm16<TBF16, 1, kEpiRope>(A, B, nullptr, C, M, N, K, lda, ldb, ldc, bt, stream, ep);
    case AK_F32: return AK_EUNSUPPORTED;
    default: return AK_EINVAL;
  }
}

extern "C" int ak_mlp_gate_up(int dtype, const void* x, const void* w_gate, const void* w_up, void* h,
                              int64_t M, int64_t H, int64_t D, int activation, hipStream_t stream) {
  if (M < 0 || H < 0 || D < 0 || M > INT_MAX || H > INT_MAX || D > INT_MAX) return AK_EINVAL;
  if (M == 0 || H == 0) return AK_OK;
  if (!x || !w_gate || !w_up || !h) return AK_EINVAL;
  int epi;
  switch (activation) {
    case AK_ACT_SILU: epi = kEpiSilu; break;
    case AK_ACT_GELU: epi = kEpiGelu; break;
    case AK_ACT_RELU2: epi = kEpiRelu2; break;
    case AK_ACT_NONE: epi = kEpiNone; break;
    default: return AK_EINVAL;
  }
  if (dtype == AK_F32) {
    const int tiles_m = (int)cdiv(M, 64), tiles_n = (int)cdiv(H, 64);
    gate_up_f32<<<tiles_m * tiles_n, 256, 0, stream>>>((const float*)x, (const float*)w_gate, (const float*)w_up,
                                                       (float*)h, (int)M, (int)H, (int)D, epi, tiles_m, tiles_n);
    return record_launch();
  }
#define AK_GU(TT)                                                                                          \
  switch (epi) {                                                                                           \
    case kEpiSilu: return launch_gemm16<TT, 2, kEpiSilu>(x, w_gate, w_up, h, M, H, D, D, D, H, true, stream);   \
    case kEpiGelu: return launch_gemm16<TT, 2, kEpiGelu>(x, w_gate, w_up, h, M, H, D, D, D, H, true, stream);   \
    case kEpiRelu2: return launch_gemm16<TT, 2, kEpiRelu2>(x, w_gate, w_up, h, M, H, D, D, D, H, true, stream); \
    default: return launch_gemm16<TT, 2, kEpiNone>(x, w_gate, w_up, h, M, H, D, D, D, H, true, stream);         \
  }
  if (dtype == AK_F16) { AK_GU(TF16) }
  if (dtype == AK_BF16) { AK_GU(TBF16) }
#undef AK_GU
  return AK_EINVAL;
}
