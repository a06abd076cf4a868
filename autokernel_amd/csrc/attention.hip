// attention.hip -- flash-attention forward for gfx950 (f16 / bf16, head_dim 64 or 128).
//
// Semantics of reference.py:32-42: O = softmax(Q K^T * sm_scale, causal mask j > i) V, computed
// without materialising the score matrix (online softmax, fp32 statistics and accumulators).
//
// Work split: one block = 4 waves = 128 query rows of one (batch, head); each wave owns 32 query
// rows. Keys stream through LDS in tiles of 64 (double-buffered, register prefetch).
//   * S^T = K Q^T on v_mfma_f32_32x32x16: the query index is the MFMA column, so each lane owns
//     one query and 16 of its 32 key scores per 32-key block; the row max needs one xor-32
//     exchange and the running sum stays lane-local until the end.
//   * O^T += V^T P^T on the same MFMA: the score accumulator layout is used directly as the B
//     operand (P^T) after rounding to f16 / bf16. Inside each 16-key group the MFMA's k order
//     is a fixed permutation of the keys; V^T is stored in LDS with the same permutation, so
//     the contraction is unchanged. O^T also has the query as its column, so the online-softmax
//     rescale is lane-local.
//   * V is transposed on its way into LDS (4 keys x 8 dims per thread through v_perm_b32; the 8
//     lanes of a write phase cover 8 key-quads of one V^T row); K stays [key][d]. Both use the
//     XOR chunk swizzle c ^ (row & 7), under which fragment reads and these writes are
//     conflict-free.
//   * Causal: key tiles past a block's last query are never loaded, tiles past a wave's last
//     query are skipped by that wave, and blocks are issued heaviest-first over all heads.
//   * f16 inputs: the reference rounds Q K^T to f16 and scales in f16, so scores beyond the f16
//     range become +-inf (and produce its NaN rows). Per tile, a wave-wide test of the largest
//     |score| enables an exact per-element emulation only when such a score exists.
#include <limits.h>

#include "ak_common.h"

namespace ak {

constexpr int kFaBKV = 64;   // keys per tile
// fa_fwd2's lazy exp2 base: a row's base is raised only when a tile's max passes it by more than
// this (log2 units), so P <= 2^8 (exact range in f16 / bf16) and, after a row's first tile, the
// O rescale is almost never needed.
constexpr float kFa2Slack = 8.0f;

constexpr int kFaWaves = 4;                  // waves per block, 32 query rows each
constexpr int kFaBQ = 32 * kFaWaves;         // query rows per block
constexpr int kFaThreads = kFaWaves * 64;
constexpr float kFaLog2e = 1.4426950408889634f;

// 16-byte chunk c of an LDS row is stored at chunk c ^ (row & 7): a ds_read_b128 phase of 8 lanes
// reading 8 consecutive rows at one logical chunk hits 8 different slots.
__device__ __forceinline__ int fa_swz(int row, int c) { return c ^ (row & 7); }

// Physical position of key offset o (0..15) inside its 16-key group in V^T: the MFMA's logical
// k index h*8 + e (lane half h, element e) carries key 4h + (e & 3) + 8 * (e >> 2).
__device__ __forceinline__ int fa_kperm(int o) { return o ^ ((((o >> 2) ^ (o >> 3)) & 1) * 12); }

template <typename T>
__device__ __forceinline__ f32x16 mfma32x32x16(const u32x4& a, const u32x4& b, const f32x16& c);
template <>
__device__ __forceinline__ f32x16 mfma32x32x16<TF16>(const u32x4& a, const u32x4& b, const f32x16& c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, a), __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
}
template <>
__device__ __forceinline__ f32x16 mfma32x32x16<TBF16>(const u32x4& a, const u32x4& b, const f32x16& c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
}

template <typename T, int D>
__global__ __launch_bounds__(kFaThreads, 8 / kFaWaves) void fa_fwd(
    const uint16_t* __restrict__ Q, const uint16_t* __restrict__ K, const uint16_t* __restrict__ V,
    uint16_t* __restrict__ O, int Hq, int group, int Sq, int Sk, int64_t qsb, int64_t qsh,
    int64_t qss, int64_t ksb, int64_t ksh, int64_t kss, int64_t vsb, int64_t vsh, int64_t vss,
    int64_t osb, int64_t osh, int64_t oss, int causal, float scale_log2, float ovf_thresh, int nbh) {
  constexpr int DC = D / 8;              // 16-byte chunks per K row
  constexpr int NDB = D / 32;            // 32-wide d blocks of O^T
  constexpr int NS = D / 16;             // 16-deep d steps of S^T
  constexpr int K_CH = kFaBKV * DC / kFaThreads;          // K chunks per thread per tile
  constexpr int V_UNITS = (kFaBKV / 4) * (D / 8);         // 4(key) x 8(d) V units per tile
  constexpr int V_U = (V_UNITS + kFaThreads - 1) / kFaThreads;
  static_assert(K_CH * kFaThreads == kFaBKV * DC, "tile split");

  __shared__ __attribute__((aligned(16))) uint16_t sK[2][kFaBKV * D];
  __shared__ __attribute__((aligned(16))) uint16_t sV[2][D * kFaBKV];

  // 1-D grid ordered by q-block, heaviest first across all (batch, head): blocks are dispatched in
  // index order, so under a causal mask the long blocks start first and short ones fill the tail.
  const int bh = (int)(blockIdx.x % (unsigned)nbh);
  const int qi = (int)(blockIdx.x / (unsigned)nbh);
  const int nqb = (Sq + kFaBQ - 1) / kFaBQ;
  const int qb = causal ? (nqb - 1 - qi) : qi;
  const int h = bh % Hq, b = bh / Hq;
  const int hk = h / group;
  const int tid = threadIdx.x, lane = lane_id(), w = wave_id();
  const int l32 = lane & 31, hh = lane >> 5;
  const int q0 = qb * kFaBQ;
  const int qw0 = q0 + w * 32;         // this wave's first query
  const int my_q = qw0 + l32;          // this lane's query

  const uint16_t* Qb = Q + b * qsb + h * qsh;
  const uint16_t* Kb = K + b * ksb + hk * ksh;
  const uint16_t* Vb = V + b * vsb + hk * vsh;
  uint16_t* Ob = O + b * osb + h * osh;

  // Q fragments: B operand of S^T, lane holds q = l32, d = s*16 + hh*8 .. +8
  u32x4 qf[NS];
#pragma unroll
  for (int s = 0; s < NS; ++s)
    qf[s] = (my_q < Sq) ? ld16(Qb + (int64_t)my_q * qss + s * 16 + hh * 8) : u32x4{0u, 0u, 0u, 0u};

  // key range
  int kend = Sk;
  if (causal) kend = min(Sk, q0 + kFaBQ);
  const int ntiles = (kend + kFaBKV - 1) / kFaBKV;

  u32x4 rk[K_CH];
  u32x4 rv[V_U][4];
  auto gload = [&](int k0) {
#pragma unroll
    for (int i = 0; i < K_CH; ++i) {
      const int q = tid + i * kFaThreads;
      const int row = q / DC, c = q % DC;
      const int key = k0 + row;
      rk[i] = key < Sk ? ld16(Kb + (int64_t)key * kss + c * 8) : u32x4{0u, 0u, 0u, 0u};
    }
#pragma unroll
    for (int i = 0; i < V_U; ++i) {
      const int u = tid + i * kFaThreads;
      const int kq = u % (kFaBKV / 4), dg = u / (kFaBKV / 4);
      if (u < V_UNITS) {
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int key = k0 + kq * 4 + r;
          rv[i][r] = key < Sk ? ld16(Vb + (int64_t)key * vss + dg * 8) : u32x4{0u, 0u, 0u, 0u};
        }
      }
    }
  };
  auto sstore = [&](int st) {
#pragma unroll
    for (int i = 0; i < K_CH; ++i) {
      const int q = tid + i * kFaThreads;
      const int row = q / DC, c = q % DC;
      // swizzle the low 3 bits of the chunk index only (stays inside the row)
      const int pc = (c & ~7) | fa_swz(row, c & 7);
      *reinterpret_cast<u32x4*>(&sK[st][row * D + pc * 8]) = rk[i];
    }
#pragma unroll
    for (int i = 0; i < V_U; ++i) {
      const int u = tid + i * kFaThreads;
      const int kq = u % (kFaBKV / 4), dg = u / (kFaBKV / 4);
      if (u >= V_UNITS) continue;
      const int pos = (kq >> 2) * 16 + fa_kperm((kq & 3) * 4);  // physical key position
      const int c = pos >> 3, off = pos & 7;
#pragma unroll
      for (int n = 0; n < 8; ++n) {
        const int wd = n >> 1;
        const uint32_t sel = (n & 1) ? 0x07060302u : 0x05040100u;
        u32x2 t;
        t[0] = __builtin_amdgcn_perm(rv[i][1][wd], rv[i][0][wd], sel);
        t[1] = __builtin_amdgcn_perm(rv[i][3][wd], rv[i][2][wd], sel);
        const int d = dg * 8 + n;
        *reinterpret_cast<u32x2*>(&sV[st][d * kFaBKV + fa_swz(d, c) * 8 + off]) = t;
      }
    }
  };

  f32x16 o[NDB];
#pragma unroll
  for (int i = 0; i < NDB; ++i)
#pragma unroll
    for (int v = 0; v < 16; ++v) o[i][v] = 0.f;
  float m_run = -INFINITY, l_run = 0.f;

  if (ntiles > 0) {
    gload(0);
    sstore(0);
  }
  __syncthreads();

  for (int kt = 0; kt < ntiles; ++kt) {
    const int cur = kt & 1;
    const int k0 = kt * kFaBKV;
    if (kt + 1 < ntiles) gload(k0 + kFaBKV);

    const bool wave_needs = !causal || k0 <= qw0 + 31;
    if (wave_needs) {
      // ---- S^T for two 32-key blocks ----
      f32x16 s[2];
#pragma unroll
      for (int kb = 0; kb < 2; ++kb) {
#pragma unroll
        for (int v = 0; v < 16; ++v) s[kb][v] = 0.f;
        const int row = kb * 32 + l32;
#pragma unroll
        for (int st = 0; st < NS; ++st) {
          const int c = st * 2 + hh;
          const int pc = (c & ~7) | fa_swz(row, c & 7);
          const u32x4 kf = *reinterpret_cast<const u32x4*>(&sK[cur][row * D + pc * 8]);
          s[kb] = mfma32x32x16<T>(kf, qf[st], s[kb]);
        }
      }
      // ---- f16 overflow emulation (reference rounds Q K^T and its scaled value to f16) ----
      if constexpr (T::kCode == AK_F16) {
        float amax = 0.f;
#pragma unroll
        for (int kb = 0; kb < 2; ++kb)
#pragma unroll
          for (int v = 0; v < 16; ++v) amax = fmaxf(amax, fabsf(s[kb][v]));
        if (__builtin_amdgcn_ballot_w64(amax >= ovf_thresh)) {
#pragma unroll
          for (int kb = 0; kb < 2; ++kb)
#pragma unroll
            for (int v = 0; v < 16; ++v)
              if (fabsf(s[kb][v]) >= ovf_thresh) s[kb][v] = __builtin_copysignf(INFINITY, s[kb][v]);
        }
      }
      // ---- scale and mask. Fast path (positive scale, no masked key in the tile): the scale is
      // folded into the exp2 argument. Otherwise scores are scaled first and masked keys set to
      // -inf afterwards, as the reference masks the scaled scores.
      const bool need_mask = (causal && k0 + kFaBKV - 1 > qw0) || (k0 + kFaBKV > Sk);
      const bool fused = scale_log2 > 0.f && !need_mask;
      if (!fused) {
#pragma unroll
        for (int kb = 0; kb < 2; ++kb)
#pragma unroll
          for (int v = 0; v < 16; ++v) {
            const int key = k0 + kb * 32 + (v >> 2) * 8 + hh * 4 + (v & 3);
            const bool masked = key >= Sk || (causal && key > my_q);
            s[kb][v] = masked ? -INFINITY : s[kb][v] * scale_log2;
          }
      }
      // ---- online softmax (log2 domain) ----
      float mt = -INFINITY;
#pragma unroll
      for (int kb = 0; kb < 2; ++kb)
#pragma unroll
        for (int v = 0; v < 16; ++v) mt = fmaxf(mt, s[kb][v]);
      mt = fmaxf(mt, __shfl_xor(mt, 32, kWave));
      const float m_tile = fused ? mt * scale_log2 : mt;
      // the exp2 base is the exact running max (P <= 1), raised on every tile whose max passes it
      // (a NaN tile max propagates)
      const float m_new = !(m_tile == m_tile) ? m_tile : fmaxf(m_run, m_tile);
      const float base = (m_new == -INFINITY) ? 0.f : m_new;
      const float alpha = (m_new == m_run) ? 1.0f : __builtin_amdgcn_exp2f(m_run - base);
      const float mul = fused ? scale_log2 : 1.0f;
      float ps = 0.f;
      u32x4 pf[4];
#pragma unroll
      for (int kb = 0; kb < 2; ++kb) {
#pragma unroll
        for (int half = 0; half < 2; ++half) {
          float p[8];
#pragma unroll
          for (int e = 0; e < 8; ++e) {
            p[e] = __builtin_amdgcn_exp2f(__builtin_fmaf(s[kb][half * 8 + e], mul, -base));
            ps += p[e];
          }
          u32x4 pk;
#pragma unroll
          for (int e = 0; e < 4; ++e)
            pk[e] = (uint32_t)T::from_f(p[2 * e]) | ((uint32_t)T::from_f(p[2 * e + 1]) << 16);
          pf[kb * 2 + half] = pk;
        }
      }
      l_run = l_run * alpha + ps;
      m_run = m_new;
      if (__builtin_amdgcn_ballot_w64(alpha != 1.0f)) {
#pragma unroll
        for (int i = 0; i < NDB; ++i)
#pragma unroll
          for (int v = 0; v < 16; ++v) o[i][v] *= alpha;
      }
      // ---- O^T += V^T P^T ----
#pragma unroll
      for (int t = 0; t < 4; ++t) {
#pragma unroll
        for (int db = 0; db < NDB; ++db) {
          const int d = db * 32 + l32;
          const int c = t * 2 + hh;
          const u32x4 vf = *reinterpret_cast<const u32x4*>(&sV[cur][d * kFaBKV + fa_swz(d, c) * 8]);
          o[db] = mfma32x32x16<T>(vf, pf[t], o[db]);
        }
      }
    }
    if (kt + 1 < ntiles) sstore(cur ^ 1);
    __syncthreads();
  }

  // ---- epilogue: O[q][d] = O^T[d][q] / l ----
  const float l_tot = l_run + __shfl_xor(l_run, 32, kWave);
  if (my_q < Sq) {
    uint16_t* orow = Ob + (int64_t)my_q * oss;
#pragma unroll
    for (int db = 0; db < NDB; ++db)
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int d = db * 32 + g * 8 + hh * 4;
        u32x2 pk;
        pk[0] = (uint32_t)T::from_f(o[db][g * 4 + 0] / l_tot) | ((uint32_t)T::from_f(o[db][g * 4 + 1] / l_tot) << 16);
        pk[1] = (uint32_t)T::from_f(o[db][g * 4 + 2] / l_tot) | ((uint32_t)T::from_f(o[db][g * 4 + 3] / l_tot) << 16);
        *reinterpret_cast<u32x2*>(orow + d) = pk;
      }
  }
}

// ============================================================================================
// fa_fwd2: the main forward kernel (positive scale; one head's K / V rows addressable with
// 32-bit byte offsets). Same work split and arithmetic as fa_fwd, built for gfx950's pipes:
//   * K and V tiles reach LDS by LDS DMA (buffer_load_dwordx4 ... lds): no staging registers, no
//     ds_write. The buffer resource of each tile ends at the last valid key, so rows past Sk
//     arrive as zeros (their scores are masked; zero V rows add nothing).
//   * V stays in its natural [key][d] layout. The V^T fragments of O^T += V^T P^T are read with
//     ds_read_b64_tr_b16, which transposes a 4 x 16 block of 16-bit values across each group of
//     16 lanes: output lane i, element e = element (i % 4) of source lane (i / 4 + 4 e). So source
//     lane j of a group addresses V[key0 + j / 4][d0 + 4 (j % 4)] and output lane i receives
//     V[key0 + e][d0 + i], e = 0..3: four consecutive keys of one d, as the MFMA's A operand needs.
//   * Software pipeline per wave, one tile per iteration j:
//       phase 1: O^T += V_{j-1}^T P_{j-1}^T (MFMA)   with   row max of S_j, exponent arguments (VALU)
//       phase 2: S_{j+1} = K_{j+1} Q^T (MFMA)        with   P_j = exp2(...), packing, row sums and the
//                                                           rescale O^T <- alpha_j O^T (VALU)
//     so every MFMA burst has independent softmax work beside it. Two barriers per tile (after
//     each phase); each tile's DMA is issued 1.5 iterations before it is read.
//   * Scores stay in raw units (Q K^T); the scale is folded into the exp2 argument. The
//     reference's f16 overflow of Q K^T (or of its scaled value) turns a row into NaN exactly when
//     some unmasked score reaches the overflow threshold (an inf score) or when every unmasked
//     score is at or below minus the threshold (a row of -inf); both are decided once per row from
//     the true row max.
//   * Lazy exp2 base: a row's base is raised only when a tile's max passes it by more than
//     kFa2Slack (log2 units), so P <= 2^8 is rounded to f16 / bf16 for the P V product and the row
//     sums add those rounded values (v_dot2 against ones: the weights that multiply V are the ones
//     normalised). Past a row's first tile the base almost never moves, so the O rescale sits
//     behind a wave-uniform branch after phase 2 instead of 64 multiplies per tile. Measured against
//     the exact running max (P <= 1, unrounded fp32 row sums: SDPA's rounding, 99.8 % bit-equal to
//     it), one process, f16: [1, 32, 8192, 128] 576.7 -> 549.5 us, [4, 32, 2048, 128] 183.3 ->
//     181.5 us, [1, 32/8, 2048, 128] 61.2 -> 57.8 us.
// LDS swizzles (16-byte chunk c of row r):
//   K: c ^ (r & 15) for D = 128, c ^ ((r >> 1) & 7) for D = 64. gfx950 serves a ds_read_b128 in
//      16-lane phases (256 bytes); the 16 lanes of a phase read rows r..r+15 at one chunk.
//   V: c ^ (4 (r & 3) + 2 ((r >> 2) & 1)) for D = 128 (256-byte rows), c ^ (4 ((r >> 1) & 1) +
//      2 ((r >> 2) & 1)) for D = 64 (128-byte rows). A tr read's 16-lane groups cover rows r..r+3
//      (groups 0, 1) or r+4..r+7 (groups 2, 3) at 32 bytes each; any two of its groups land on
//      distinct banks.
// ============================================================================================
template <int D>
__device__ __forceinline__ int fa2_kswz(int r) {
  if constexpr (D == 128) return r & 15;
  else return (r >> 1) & 7;
}
template <int D>
__device__ __forceinline__ int fa2_vswz(int r) {
  if constexpr (D == 128) return 4 * (r & 3) + 2 * ((r >> 2) & 1);
  else return 4 * ((r >> 1) & 1) + 2 * ((r >> 2) & 1);
}

// Raw buffer resource: loads at byte offsets >= nbytes return zeros.
__device__ __forceinline__ u32x4 fa2_rsrc(const void* base, uint32_t nbytes) {
  const uint64_t a = (uint64_t)(uintptr_t)base;
  u32x4 r;
  r[0] = __builtin_amdgcn_readfirstlane((uint32_t)a);
  r[1] = __builtin_amdgcn_readfirstlane((uint32_t)(a >> 32) & 0xffffu);  // stride 0
  r[2] = __builtin_amdgcn_readfirstlane(nbytes);
  r[3] = 0x00020000u;  // 32-bit data format, untyped access
  return r;
}

// One 1 KB LDS-DMA transfer: lane L's 16 bytes from rsrc + voff land at LDS byte lds + 16 L.
// Inline assembly, so the compiler inserts no waits for it: every wait is an explicit vmcnt. The
// LDS destination is an input operand bound to M0 ("{m0}"): the compiler writes M0 itself, so no
// register changes behind its back. One wait state separates the M0 write from the load.
__device__ __forceinline__ void fa2_dma16(const u32x4& rsrc, uint32_t voff, uint32_t lds) {
  asm volatile(
      "s_nop 0\n\t"
      "buffer_load_dwordx4 %0, %1, 0 offen lds"
      :
      : "v"(voff), "s"(rsrc), "{m0}"(lds)
      : "memory");
}

typedef short fa2_s16x4 __attribute__((ext_vector_type(4)));
__device__ __forceinline__ u32x2 fa2_tr16(const uint16_t* p) {
  return __builtin_bit_cast(
      u32x2, __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) fa2_s16x4*)(p)));
}

template <typename T>
__device__ __forceinline__ uint32_t fa2_pack(float a, float b);
template <>
__device__ __forceinline__ uint32_t fa2_pack<TF16>(float a, float b) {
  typedef float f2 __attribute__((ext_vector_type(2)));
  return __builtin_bit_cast(uint32_t, __builtin_convertvector((f2){a, b}, f16x2));
}
template <>
__device__ __forceinline__ uint32_t fa2_pack<TBF16>(float a, float b) {
  typedef float f2 __attribute__((ext_vector_type(2)));
  typedef __bf16 b2 __attribute__((ext_vector_type(2)));
  return __builtin_bit_cast(uint32_t, __builtin_convertvector((f2){a, b}, b2));
}
// acc + p.lo + p.hi (p: two packed values)
template <typename T>
__device__ __forceinline__ float fa2_sum2(uint32_t p, float acc);
template <>
__device__ __forceinline__ float fa2_sum2<TF16>(uint32_t p, float acc) {
  const f16x2 one = {(_Float16)1.0f, (_Float16)1.0f};
  return __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2, p), one, acc, false);
}
template <>
__device__ __forceinline__ float fa2_sum2<TBF16>(uint32_t p, float acc) {
  typedef __bf16 b2 __attribute__((ext_vector_type(2)));
  const b2 one = {(__bf16)1.0f, (__bf16)1.0f};
  return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(b2, p), one, acc, false);
}
// Keeps the computation of x ahead of this point (an empty use the compiler cannot move).
__device__ __forceinline__ void fa2_pin(const f32x16& x) { asm volatile("" ::"v"(x)); }
// max over the two 32-lane halves (every lane gets the same value, combined in the same order)
// NaN-propagating max (v_maximum3_f32 / v_maximum_f32). fmaxf would ignore a NaN score, and on
// MFMA results the compiler then quiets each operand first (one v_max_f32 per operand: 11 more
// instructions per 64-key tile). A row whose scores hold a NaN comes out NaN either way: its true
// max fails the overflow test below.
__device__ __forceinline__ float fa2_max(float a, float b) { return __builtin_elementwise_maximum(a, b); }
__device__ __forceinline__ float fa2_halves_max(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return fa2_max(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float fa2_halves_sum(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

// fa_fwd2 work split: kFa2Waves waves of 32 query rows per block, two waves per SIMD.
constexpr int kFa2Waves = 4;
constexpr int kFa2BQ = 32 * kFa2Waves;
constexpr int kFa2Threads = 64 * kFa2Waves;
constexpr int kFa2Layer = 256;  // blocks per layer: one per MI355X compute unit

// NH = 2 (grids of at most one block per CU): a block is 8 waves, and waves 4..7 take the second
// half of the block's key tiles for the same 128 queries, in LDS stages of their own. Every wave
// runs the same number of iterations (the first half's tile count) with two barriers each, so the
// halves meet at every barrier; the DMA issue and wait counts follow each half's real tile count,
// so no transfer reads past the block's last key. At the end the second half hands its O^T, exp2
// base, row sums and true row max to the first through LDS, which combines them and stores O.
template <typename T, int D, int NH>
__global__ __launch_bounds__(kFa2Threads * NH, NH == 1 ? 8 / kFa2Waves : 1) void fa_fwd2(
    const uint16_t* __restrict__ Q, const uint16_t* __restrict__ K, const uint16_t* __restrict__ V,
    uint16_t* __restrict__ O, int Hq, int group, int Sq, int Sk, int64_t qsb, int64_t qsh,
    int64_t qss, int64_t ksb, int64_t ksh, int kss, int64_t vsb, int64_t vsh, int vss,
    int64_t osb, int64_t osh, int64_t oss, int causal, float c_log2, float thr, int nbh) {
  static_assert((kFa2Waves == 4 || kFa2Waves == 8) && kFaBKV == 64 && (NH == 1 || NH == 2), "fa_fwd2 tiling");
  constexpr int DC = D / 8;             // 16-byte chunks per row
  constexpr int RPI = 64 / DC;          // rows per 1 KB DMA transfer
  constexpr int NIW = kFaBKV / RPI / kFa2Waves;  // transfers per wave per tile, per matrix
  constexpr int NS = D / 16;            // 16-deep d steps of S^T
  constexpr int NDB = D / 32;           // 32-row d blocks of O^T
  constexpr int TILE = kFaBKV * D;      // elements of one K or V tile
  static_assert(NIW * RPI * kFa2Waves == kFaBKV, "tile rows split over waves");
  __shared__ __attribute__((aligned(1024))) uint16_t sKa[NH * 2 * TILE];
  __shared__ __attribute__((aligned(1024))) uint16_t sVa[NH * 2 * TILE];

  // Causal work order: blocks come heaviest first (greedy balance over many rounds). A grid of at
  // most two layers of kFa2Layer blocks (one block per CU each) reverses its second layer, so the
  // two blocks that share a CU pair a heavy and a light query block (measured [1, 32, 2048, 128]:
  // 56.2 -> 53.2 us; longer grids lose about 2 % with it). A bijection of block indices.
  int L = (int)blockIdx.x;
  if (causal && gridDim.x <= 2u * kFa2Layer) {
    const int layer = L / kFa2Layer, base = layer * kFa2Layer;
    if (layer & 1) L = base + min(kFa2Layer, (int)gridDim.x - base) - 1 - (L - base);
  }
  const int bh = L % nbh;
  const int qi = L / nbh;
  const int nqb = (Sq + kFa2BQ - 1) / kFa2BQ;
  const int qb = causal ? (nqb - 1 - qi) : qi;
  const int h = bh % Hq, b = bh / Hq;
  const int hk = h / group;
  const int lane = lane_id();
  const int wid = __builtin_amdgcn_readfirstlane(wave_id());
  const int half = NH == 2 ? wid / kFa2Waves : 0;  // key half (wave-uniform)
  const int w = wid % kFa2Waves;                    // wave within the half: query rows w * 32 ..
  uint16_t* const sK = sKa + half * 2 * TILE;       // this half's two K stages
  uint16_t* const sV = sVa + half * 2 * TILE;
  const int l32 = lane & 31, hh = lane >> 5;
  const int q0 = qb * kFa2BQ;
  const int qw0 = q0 + w * 32;
  const int my_q = qw0 + l32;

  const uint16_t* Qb = Q + b * qsb + h * qsh;
  const uint16_t* Kb = K + b * ksb + hk * ksh;
  const uint16_t* Vb = V + b * vsb + hk * vsh;
  uint16_t* Ob = O + b * osb + h * osh;

  // Q fragments (B operand of S^T): lane holds query l32, d = s * 16 + hh * 8 .. + 8
  u32x4 qf[NS];
#pragma unroll
  for (int s = 0; s < NS; ++s)
    qf[s] = (my_q < Sq) ? ld16(Qb + (int64_t)my_q * qss + s * 16 + hh * 8) : u32x4{0u, 0u, 0u, 0u};

  const int kend = causal ? min(Sk, q0 + kFa2BQ) : Sk;
  const int ntb = (kend + kFaBKV - 1) / kFaBKV;          // the block's key tiles, >= 1 (>= 2 when NH = 2)
  // This half's tiles are jbase + 0 .. jbase + nt - 1 (nt >= 1); j below is relative to jbase.
  // Every wave iterates ntl times: the second half's last iteration is empty when ntb is odd.
  const int ntl = NH == 2 ? (ntb + 1) / 2 : ntb;
  const int jbase = half * ntl;
  const int nt = NH == 2 ? (half ? ntb - ntl : ntl) : ntb;
  // this wave's last tile in this half (negative when every key of the half is past its queries)
  const int jw = min(nt - 1, (causal ? min(ntb - 1, (qw0 + 31) / kFaBKV) : ntb - 1) - jbase);

  // Per-lane byte offsets of the DMA transfers inside a tile (the tile base is in the resource):
  // transfer n = i * 4 + w covers tile rows n * RPI ..; lane L writes physical chunk L % DC of row
  // n * RPI + L / DC and so fetches the logical chunk the swizzle maps there (XOR: its own inverse).
  uint32_t offk[NIW], offv[NIW];
#pragma unroll
  for (int i = 0; i < NIW; ++i) {
    const int row = (i * kFa2Waves + w) * RPI + lane / DC;
    const int pc = lane % DC;
    offk[i] = (uint32_t)(row * kss * 2 + ((pc ^ fa2_kswz<D>(row)) * 16));
    offv[i] = (uint32_t)(row * vss * 2 + ((pc ^ fa2_vswz<D>(row)) * 16));
  }
  const uint32_t sK_lds = (uint32_t)(uintptr_t)(lds_void*)sK;
  const uint32_t sV_lds = (uint32_t)(uintptr_t)(lds_void*)sV;

  auto issue_k = [&](int j, int stage) {
    const int k0 = (jbase + j) * kFaBKV;
    const u32x4 rs = fa2_rsrc(Kb + (int64_t)k0 * kss, (uint32_t)(((Sk - 1 - k0) * kss + D) * 2));
#pragma unroll
    for (int i = 0; i < NIW; ++i) fa2_dma16(rs, offk[i], sK_lds + stage * TILE * 2 + (i * kFa2Waves + w) * 1024);
  };
  auto issue_v = [&](int j, int stage) {
    const int k0 = (jbase + j) * kFaBKV;
    const u32x4 rs = fa2_rsrc(Vb + (int64_t)k0 * vss, (uint32_t)(((Sk - 1 - k0) * vss + D) * 2));
#pragma unroll
    for (int i = 0; i < NIW; ++i) fa2_dma16(rs, offv[i], sV_lds + stage * TILE * 2 + (i * kFa2Waves + w) * 1024);
  };

  // S^T = K Q^T for the 64 keys of a tile: two 32-key accumulators, issued alternately
  auto qk = [&](const uint16_t* ks, f32x16 (&s)[2]) {
#pragma unroll
    for (int kb = 0; kb < 2; ++kb)
#pragma unroll
      for (int v = 0; v < 16; ++v) s[kb][v] = 0.f;
#pragma unroll
    for (int st = 0; st < NS; ++st)
#pragma unroll
      for (int kb = 0; kb < 2; ++kb) {
        const int r = kb * 32 + l32;
        const int c = st * 2 + hh;
        const u32x4 kf = *reinterpret_cast<const u32x4*>(&ks[r * D + (c ^ fa2_kswz<D>(r)) * 8]);
        s[kb] = mfma32x32x16<T>(kf, qf[st], s[kb]);
      }
  };

  // O^T += V^T P^T over the 64 keys of a tile: 16-key step t, lane-half hh carries keys
  // 16 t + 4 hh + 0..3 and 16 t + 8 + 4 hh + 0..3 (the S^T accumulator order, see softmax below).
  f32x16 o[NDB];
#pragma unroll
  for (int i = 0; i < NDB; ++i)
#pragma unroll
    for (int v = 0; v < 16; ++v) o[i][v] = 0.f;
  const int g16 = lane >> 4, i16 = lane & 15;
  const int vrow = 4 * (g16 >> 1) + (i16 >> 2);          // + 16 t (+ 8 for the second read)
  const int vcol = 16 * (g16 & 1) + 4 * (i16 & 3);       // + 32 db
  const int vsw = fa2_vswz<D>(vrow);                      // same for rows + 8, + 16 t
  u32x4 pf[4];
  // O^T += V^T P^T over the 64 keys of a tile, one 32-row d block at a time (O^T already carries the
  // tile's exp2 base: it was rescaled in the previous phase).
  auto pv = [&](const uint16_t* vs) {
#pragma unroll
    for (int db = 0; db < NDB; ++db) {
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        const int col = db * 32 + vcol;
        const uint16_t* p = vs + (16 * t + vrow) * D + (((col >> 3) ^ vsw) * 8) + (col & 7);
        const u32x2 lo = fa2_tr16(p);
        const u32x2 hi = fa2_tr16(p + 8 * D);
        const u32x4 vf = {lo[0], lo[1], hi[0], hi[1]};
        o[db] = mfma32x32x16<T>(vf, pf[t], o[db]);
      }
    }
  };

  float m_run = -INFINITY, l_run = 0.f, m_true = -INFINITY;
  // row statistics of S_j: mask, tile max (raw units), lazy base update (alpha = 1 unless it moved)
  auto stats = [&](f32x16 (&s)[2], int k0, bool masked, float& alpha, float& base) {
    if (masked) {
      // key k0 + hh * 4 + off is masked when it is at or past lim (Sk, or my_q + 1 when causal):
      // one compare against the compile-time offset per score
      const int lim = causal ? min(Sk, my_q + 1) : Sk;
      const int t = lim - (k0 + hh * 4);
#pragma unroll
      for (int kb = 0; kb < 2; ++kb)
#pragma unroll
        for (int v = 0; v < 16; ++v) {
          const int off = kb * 32 + (v >> 2) * 8 + (v & 3);
          if (off >= t) s[kb][v] = -INFINITY;
        }
    }
    // four independent max3 chains over 7 scores each, then one max3 chain over their results and
    // the four scores left (16 three-input maxima for 32 scores)
    float m4[4];
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      const int kb = c >> 1, v0 = (c & 1) * 8;
      float m = fa2_max(fa2_max(s[kb][v0], s[kb][v0 + 1]), s[kb][v0 + 2]);
      m = fa2_max(fa2_max(m, s[kb][v0 + 3]), s[kb][v0 + 4]);
      m4[c] = fa2_max(fa2_max(m, s[kb][v0 + 5]), s[kb][v0 + 6]);
    }
    float mt = fa2_max(fa2_max(m4[0], s[0][7]), m4[1]);
    mt = fa2_max(fa2_max(mt, s[0][15]), m4[2]);
    mt = fa2_max(fa2_max(mt, s[1][7]), m4[3]);
    mt = fa2_max(mt, s[1][15]);
    mt = fa2_halves_max(mt);
    m_true = fa2_max(m_true, mt);
    const float mts = mt * c_log2;
    const float m_new = (mts > m_run + kFa2Slack || m_run == -INFINITY) ? fmaxf(m_run, mts) : m_run;
    base = (m_new == -INFINITY) ? 0.f : m_new;
    alpha = (m_new == m_run) ? 1.0f : __builtin_amdgcn_exp2f(m_run - base);
    m_run = m_new;
  };
  // Exponent arguments in place: S_j * c - base (log2 units).
  auto exp_args = [&](f32x16 (&s)[2], float base) {
#pragma unroll
    for (int kb = 0; kb < 2; ++kb)
#pragma unroll
      for (int v = 0; v < 16; ++v) s[kb][v] = __builtin_fmaf(s[kb][v], c_log2, -base);
  };
  // P_j = exp2(argument), rounded to the element type and packed as the B operand of the O^T
  // update; returns the row-half sum of the rounded values.
  auto exp_pack = [&](const f32x16 (&s)[2]) -> float {
    float ps = 0.f;
#pragma unroll
    for (int t = 0; t < 4; ++t)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int v = 8 * (t & 1) + 2 * e;
        const float x0 = __builtin_amdgcn_exp2f(s[t >> 1][v]);
        const float x1 = __builtin_amdgcn_exp2f(s[t >> 1][v + 1]);
        pf[t][e] = fa2_pack<T>(x0, x1);
        ps = fa2_sum2<T>(pf[t][e], ps);
      }
    return ps;
  };

  // end of iteration j: every wave is done with V_{j-1} and K_{j+1}, and V_j and K_{j+2} (issued
  // one iteration ago) have landed; refill the two free stages.
  // DMA schedule (two LDS stages each for K and V; tile t lives in stage t & 1):
  //   mid(j), after phase 1 of iteration j: every wave is done with V_{j-1}; V_{j+1} goes into its
  //     stage. K_{j+1}, read in phase 2, must have landed.
  //   end(j), after phase 2: every wave is done with K_{j+1}; K_{j+3} goes into its stage. V_j,
  //     read in phase 1 of iteration j + 1, must have landed.
  // Each transfer so has 1.5 iterations to land. vmcnt retires transfers in issue order, so a
  // wait lets exactly the transfers issued after the needed one stay in flight (two groups of
  // NIW in the steady state, fewer near the end).
  auto barrier_after = [&](int later) {
    if (later >= 2) dma_barrier<2 * NIW>();
    else if (later == 1) dma_barrier<NIW>();
    else dma_barrier<0>();
  };
  // At j = 0 the prologue has already waited for K_0, K_1 and V_0; only K_2 (issued after that
  // wait) and V_1 (mid 0) can be in flight, and neither is needed before iteration 1.
  auto sync_mid = [&](int j, int par) {
    // issued after K_{j+1}: V_j (mid j-1) and K_{j+2}
    barrier_after(j == 0 ? (nt > 2) : 1 + (j + 2 < nt));
    if (j + 1 < nt) issue_v(j + 1, par ^ 1);
  };
  auto sync_end = [&](int j, int par) {
    // issued after V_j: K_{j+2} (end j-1) and V_{j+1} (mid j)
    barrier_after((j + 2 < nt) + (j + 1 < nt));
    if (j + 3 < nt) issue_k(j + 3, par ^ 1);
  };
  f32x16 sa[2], sb[2];
  // General iteration j (parity par = j & 1): S holds S_j, Sn receives S_{j+1}. Each phase runs
  // only where this wave needs it (causal tail, first tile), and diagonal / partial tiles are
  // masked.
  auto iter = [&](int j, int par, f32x16 (&S)[2], f32x16 (&Sn)[2]) {
    const int k0 = (jbase + j) * kFaBKV;
    if (j > 0 && j - 1 <= jw) pv(sV + (par ^ 1) * TILE);  // V_{j-1}
    float alpha = 1.0f, base = 0.f;
    const bool act = j <= jw;
    if (act) {
      const bool masked = (causal && k0 + kFaBKV - 1 > qw0) || (k0 + kFaBKV > Sk);
      stats(S, k0, masked, alpha, base);
    }
    sync_mid(j, par);
    if (j + 1 <= jw) qk(sK + (par ^ 1) * TILE, Sn);  // K_{j+1}
    if (act) {
      exp_args(S, base);
      const float ps = exp_pack(S);
      l_run = l_run * alpha + ps;
      if (__builtin_amdgcn_ballot_w64(alpha != 1.0f)) {
#pragma unroll
        for (int db = 0; db < NDB; ++db)
#pragma unroll
          for (int v = 0; v < 16; ++v) o[db][v] *= alpha;
      }
    }
    sync_end(j, par);
  };
  // Steady-state iteration (1 <= j, tile j unmasked, j + 1 <= jw): all four parts run, with no
  // branch between them, so the MFMAs of one part and the VALU work of the other share one block.
  // Interleave pattern of the steady state: each phase has D / 8 MFMAs (16 at D = 128, 8 at D = 64)
  // beside about the same softmax work, so the VALU instructions per MFMA follow D (measured at
  // D = 64 against the D = 128 pattern: [1, 32, 4096, 64] 104.7 -> 103.4 us, [2, 32, 2048, 64]
  // 62.6 -> 61.2 us, smaller shapes within 1 %).
  constexpr int kPhaseMfma = D / 8;
  constexpr int kP1Valu = D == 128 ? 4 : 8;
  constexpr int kP2Valu = D == 128 ? 5 : 9;
  auto iter_fast = [&](int j, int par, f32x16 (&S)[2], f32x16 (&Sn)[2]) {
    // phase 1: O^T += V_{j-1}^T P_{j-1}^T beside the row max of S_j and its exponent arguments
    // (pinned here, so that phase 2 holds only the exponentials, the packing and the row sums).
    // Nothing in this phase waits on VALU results, so one MFMA, two fragment reads and kP1Valu VALU
    // instructions interleave throughout; fragment reads run one MFMA ahead of their use.
    pv(sV + (par ^ 1) * TILE);
    float alpha, base;
    stats(S, (jbase + j) * kFaBKV, false, alpha, base);
    exp_args(S, base);
#pragma unroll
    for (int kb = 0; kb < 2; ++kb) asm volatile("" ::"v"(S[kb]));
    __builtin_amdgcn_sched_group_barrier(0x100, 4, 0);
#pragma unroll
    for (int i = 0; i < kPhaseMfma - 2; ++i) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // 1 MFMA
      __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);  // the V^T fragment of MFMA i + 2
      __builtin_amdgcn_sched_group_barrier(0x002, kP1Valu, 0);
    }
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
      __builtin_amdgcn_sched_group_barrier(0x002, kP1Valu, 0);
    }
    __builtin_amdgcn_sched_barrier(0);
    sync_mid(j, par);
    // phase 2: S_{j+1} = K_{j+1} Q^T beside P_j = exp2(...) and its row sum
    qk(sK + (par ^ 1) * TILE, Sn);
    const float ps = exp_pack(S);
    // keep P_j's computation here (otherwise it sinks to its first use after the barrier)
#pragma unroll
    for (int t = 0; t < 4; ++t) asm volatile("" ::"v"(pf[t]));
    asm volatile("" ::"v"(ps));
    __builtin_amdgcn_sched_group_barrier(0x100, 2, 1);
#pragma unroll
    for (int i = 0; i < kPhaseMfma - 2; ++i) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 1);  // 1 MFMA
      __builtin_amdgcn_sched_group_barrier(0x100, 1, 1);  // the K fragment of MFMA i + 2
      __builtin_amdgcn_sched_group_barrier(0x402, kP2Valu, 1);  // VALU / transcendental
    }
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 1);
      __builtin_amdgcn_sched_group_barrier(0x402, kP2Valu, 1);
    }
    __builtin_amdgcn_sched_barrier(0);
    // O^T <- alpha_j O^T (O^T is not touched by phase 2's MFMAs), only when some row's base moved
    if (__builtin_amdgcn_ballot_w64(alpha != 1.0f)) {
#pragma unroll
      for (int db = 0; db < NDB; ++db)
#pragma unroll
        for (int v = 0; v < 16; ++v) o[db][v] *= alpha;
    }
    l_run = l_run * alpha + ps;
    sync_end(j, par);
  };

  issue_k(0, 0);
  if (nt > 1) issue_k(1, 1);
  issue_v(0, 0);
  dma_barrier<0>();
  qk(sK, sa);  // S_0 (jw >= 0 except for a second-half wave whose queries precede all its keys)
  dma_barrier<0>();
  if (nt > 2) issue_k(2, 0);
  // first masked tile of this wave (diagonal or partial), and the end of the steady range
  const int jm_s = Sk / kFaBKV - jbase;
  const int jm = causal ? min((qw0 + 1) / kFaBKV - jbase, jm_s) : jm_s;
  const int jf = max(1, min(jm, jw));
  // Register roles are fixed at compile time: S_j is in sb at odd j of the steady loop, in sa
  // at even j; the general iterations always take S_j from sa and leave S_{j+1} in sa.
  iter(0, 0, sa, sb);
  int j = 1;
  for (; j + 1 < jf; j += 2) {
    iter_fast(j, 1, sb, sa);
    iter_fast(j + 1, 0, sa, sb);
  }
  if (j < jf) {
    iter_fast(j, 1, sb, sa);
    ++j;
  } else {
#pragma unroll
    for (int kb = 0; kb < 2; ++kb) sa[kb] = sb[kb];
  }
  for (; j < ntl; ++j) {
    iter(j, j & 1, sa, sb);
#pragma unroll
    for (int kb = 0; kb < 2; ++kb) sa[kb] = sb[kb];
  }
  if (ntl - 1 <= jw) pv(sV + ((ntl - 1) & 1) * TILE);
  wait_vmcnt<0>();  // (no transfer is outstanding here; kept so none can outlive the block)

  if constexpr (NH == 2) {
    // Hand-over: every wave is done with its K / V stages, so they hold the second half's
    // results, [wave][value][lane] (conflict-free): O^T in the K stages, the three row scalars
    // in the V stages.
    dma_barrier<0>();
    float* xo = reinterpret_cast<float*>(sKa) + w * (NDB * 16) * 64 + lane;
    float* xs = reinterpret_cast<float*>(sVa) + w * 3 * 64 + lane;
    if (half == 1) {
#pragma unroll
      for (int db = 0; db < NDB; ++db)
#pragma unroll
        for (int v = 0; v < 16; ++v) xo[(db * 16 + v) * 64] = o[db][v];
      xs[0] = m_run;
      xs[64] = l_run;
      xs[128] = m_true;
    }
    dma_barrier<0>();
    if (half == 1) return;
    // O = (O_0 2^(b_0 - b) + O_1 2^(b_1 - b)) / (l_0 2^(b_0 - b) + l_1 2^(b_1 - b)), b = max(b_0, b_1);
    // a half with no key for this query has base -inf, O = 0 and l = 0
    const float m1 = xs[0], l1 = xs[64], t1 = xs[128];
    const float mb = fmaxf(m_run, m1);
    const float a0 = m_run == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(m_run - mb);
    const float a1 = m1 == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(m1 - mb);
#pragma unroll
    for (int db = 0; db < NDB; ++db)
#pragma unroll
      for (int v = 0; v < 16; ++v) o[db][v] = o[db][v] * a0 + xo[(db * 16 + v) * 64] * a1;
    l_run = l_run * a0 + l1 * a1;
    m_true = fa2_max(m_true, t1);
  }

  // ---- epilogue: O[q][d] = O^T[d][q] / l; NaN rows where the reference's scores overflow ----
  // one correctly rounded reciprocal per row, then products (a NaN row multiplies by NaN)
  const bool nan_row = !(m_true < thr && m_true > -thr);
  const float inv = nan_row ? __builtin_nanf("") : 1.0f / fa2_halves_sum(l_run);
  if (my_q < Sq) {
    uint16_t* orow = Ob + (int64_t)my_q * oss;
#pragma unroll
    for (int db = 0; db < NDB; ++db)
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int d = db * 32 + g * 8 + hh * 4;
        u32x2 pk;
        pk[0] = fa2_pack<T>(o[db][g * 4 + 0] * inv, o[db][g * 4 + 1] * inv);
        pk[1] = fa2_pack<T>(o[db][g * 4 + 2] * inv, o[db][g * 4 + 3] * inv);
        *reinterpret_cast<u32x2*>(orow + d) = pk;
      }
  }
}

// ============================================================================================
// fa_general: every case the two MFMA kernels do not serve -- fp32, and head_dim other than 64 or
// 128 (any D up to 256) -- with the reference's arithmetic step by step (reference.py:32-42):
//   s = rnd(rnd(q . k) * sm_scale)     the score matrix and its scaled value in the element type
//   masked keys (causal, j > i) = -inf; P = rnd(softmax(s)) with fp32 statistics
//   O = rnd(P V)                       fp32 accumulation, one rounding
// rnd is the identity for fp32. Scores, products and sums are fp32 VALU work (f16 / bf16 products
// are exact in fp32). Two passes over the keys: the first takes each query row's max and sum, the
// second forms the normalised P, rounds it as F.softmax's output is rounded, and accumulates P V.
// A row whose max is +-inf or NaN comes out NaN, as softmax makes it.
// Work split: a block is 8 waves (two per SIMD) and 64 queries (8 per wave) of one (batch, head). Key tiles of
// KT = 64 keys (32 for head_dim above 128, so the tiles fit LDS) are staged in LDS as fp32; for the
// scores lane L takes key L % KT against the wave's query slots L / KT, L / KT + 64 / KT, ..., reading
// each 16-byte chunk of its K row once for all of them; for P V lane L owns dims L, L + 64, ... and
// reads P four keys at a time. K rows are padded by 4 floats, so the 16-byte reads of 8 rows (one
// LDS phase) land on 32 distinct banks.
// ============================================================================================
constexpr int kFgWaves = 8, kFgQW = 8, kFgQB = kFgWaves * kFgQW;

template <typename T, int DMAX>
__global__ __launch_bounds__(kFgWaves * 64) void fa_general(
    const typename T::S* __restrict__ Q, const typename T::S* __restrict__ K,
    const typename T::S* __restrict__ V, typename T::S* __restrict__ O, int Hq, int group, int Sq, int Sk,
    int D, int64_t qsb, int64_t qsh, int64_t qss, int64_t ksb, int64_t ksh, int64_t kss, int64_t vsb,
    int64_t vsh, int64_t vss, int64_t osb, int64_t osh, int64_t oss, int causal, float scale, int nbh,
    int vec4) {
  typedef float f32x4v __attribute__((ext_vector_type(4)));
  constexpr int KT = DMAX > 128 ? 32 : 64;  // LDS holds fp32: 256-wide rows take 32-key tiles
  constexpr int QPP = 64 / KT;               // queries scored side by side in one wave
  constexpr int NQ = kFgQW / QPP;            // query slots per lane: qs = i * QPP + lane / KT
  constexpr int KP = DMAX + 4;               // padded K row (floats): 16-byte reads conflict-free
  constexpr int RD = DMAX / 64;              // dims per lane in P V
  static_assert(DMAX % 64 == 0 && kFgQW % QPP == 0 && KT % 4 == 0, "fa_general tiling");
  __shared__ __attribute__((aligned(16))) float sQ[kFgQB * DMAX];
  __shared__ __attribute__((aligned(16))) float sK[KT * KP];
  __shared__ __attribute__((aligned(16))) float sV[KT * DMAX];
  __shared__ __attribute__((aligned(16))) float sP[kFgWaves][kFgQW][KT];

  const int nqb = (Sq + kFgQB - 1) / kFgQB;
  const int bh = (int)(blockIdx.x % (unsigned)nbh);
  const int qi = (int)(blockIdx.x / (unsigned)nbh);
  const int qb = causal ? (nqb - 1 - qi) : qi;  // causal: heaviest query blocks first
  const int h = bh % Hq, b = bh / Hq, hk = h / group;
  const int tid = threadIdx.x, lane = lane_id(), w = wave_id();
  const int q0 = qb * kFgQB;
  const int kk = lane % KT, qsub = lane / KT;
  const int D4 = (D + 3) & ~3;  // dims read in 16-byte steps (zeros past D)

  const typename T::S* Qb = Q + b * qsb + h * qsh;
  const typename T::S* Kb = K + b * ksb + hk * ksh;
  const typename T::S* Vb = V + b * vsb + hk * vsh;

  // rows of `rows` x DMAX floats from a [*, D] matrix with row stride ld into LDS (row pitch
  // pitch), zeros past D and past `valid` rows; vec4: D, the strides and the base are multiples of
  // 4 elements, so 4 consecutive elements load together
  auto stage = [&](float* dst, int pitch, const typename T::S* src, int64_t ld, int rows, int valid) {
    if (vec4) {
      using S = typename T::S;
      for (int e = tid; e < rows * (DMAX / 4); e += kFgWaves * 64) {
        const int r = e / (DMAX / 4), d = (e % (DMAX / 4)) * 4;
        f32x4v v = {0.f, 0.f, 0.f, 0.f};
        if (r < valid && d < D) {
          const S* p = src + (int64_t)r * ld + d;
          if constexpr (sizeof(S) == 4) {
            v = *reinterpret_cast<const f32x4v*>(p);
          } else {
            const u32x2 h = *reinterpret_cast<const u32x2*>(p);
            v = f32x4v{T::to_f((S)(h[0] & 0xffffu)), T::to_f((S)(h[0] >> 16)), T::to_f((S)(h[1] & 0xffffu)),
                       T::to_f((S)(h[1] >> 16))};
          }
        }
        *reinterpret_cast<f32x4v*>(dst + r * pitch + d) = v;
      }
    } else {
      for (int e = tid; e < rows * DMAX; e += kFgWaves * 64) {
        const int r = e / DMAX, d = e % DMAX;
        dst[r * pitch + d] = (r < valid && d < D) ? T::to_f(src[(int64_t)r * ld + d]) : 0.f;
      }
    }
  };
  stage(sQ, DMAX, Qb + (int64_t)q0 * qss, qss, kFgQB, Sq - q0);
  const int kend = causal ? min(Sk, q0 + kFgQB) : Sk;
  const int ntiles = (kend + KT - 1) / KT;

  // scores of key k0 + kk against this lane's NQ query slots, with the reference's roundings;
  // each K chunk is read once for all of them (the dot products run in d order)
  auto scores = [&](int k0, float (&sc)[NQ]) {
    float dot[NQ];
#pragma unroll
    for (int i = 0; i < NQ; ++i) dot[i] = 0.f;
    const float* kr = &sK[kk * KP];
    const float* qr = &sQ[(w * kFgQW + qsub) * DMAX];
    for (int d = 0; d < D4; d += 4) {
      const f32x4v kv = *reinterpret_cast<const f32x4v*>(kr + d);
#pragma unroll
      for (int i = 0; i < NQ; ++i) {
        const f32x4v qv = *reinterpret_cast<const f32x4v*>(qr + i * QPP * DMAX + d);
        dot[i] = __builtin_fmaf(qv[0], kv[0], dot[i]);
        dot[i] = __builtin_fmaf(qv[1], kv[1], dot[i]);
        dot[i] = __builtin_fmaf(qv[2], kv[2], dot[i]);
        dot[i] = __builtin_fmaf(qv[3], kv[3], dot[i]);
      }
    }
    const int key = k0 + kk;
#pragma unroll
    for (int i = 0; i < NQ; ++i) {
      const int q = q0 + w * kFgQW + i * QPP + qsub;
      float v = T::rnd(T::rnd(dot[i]) * scale);
      if (key >= Sk || (causal && key > q)) v = -INFINITY;
      sc[i] = v;
    }
  };
  auto load_k = [&](int k0) { stage(sK, KP, Kb + (int64_t)k0 * kss, kss, KT, Sk - k0); };
  auto load_v = [&](int k0) { stage(sV, DMAX, Vb + (int64_t)k0 * vss, vss, KT, Sk - k0); };

  // pass 1: row max (NaN-propagating) and sum of exp(s - max), kept identical in every lane
  float m[kFgQW], l[kFgQW];
#pragma unroll
  for (int i = 0; i < kFgQW; ++i) {
    m[i] = -INFINITY;
    l[i] = 0.f;
  }
  for (int t = 0; t < ntiles; ++t) {
    __syncthreads();
    load_k(t * KT);
    __syncthreads();
    float sc[NQ];
    scores(t * KT, sc);
#pragma unroll
    for (int i = 0; i < NQ; ++i)
#pragma unroll
      for (int u = 0; u < QPP; ++u) {
        // lanes u * KT .. u * KT + KT - 1 hold query slot i * QPP + u
        const int qs = i * QPP + u;
        const float tm = __shfl(seg_reduce<KT>(sc[i], OpNanMax()), u * KT, 64);
        const float mn = nan_max(m[qs], tm);
        float e = (qsub == u && mn != -INFINITY) ? __builtin_amdgcn_exp2f((sc[i] - mn) * kFaLog2e) : 0.f;
        e = __shfl(seg_reduce<KT>(e, OpAdd()), u * KT, 64);
        l[qs] = (mn == -INFINITY) ? 0.f : l[qs] * __builtin_amdgcn_exp2f((m[qs] - mn) * kFaLog2e) + e;
        m[qs] = mn;
      }
  }

  // pass 2: P = rnd(exp(s - max) / sum), O += P V
  float acc[kFgQW][RD];
#pragma unroll
  for (int i = 0; i < kFgQW; ++i)
#pragma unroll
    for (int r = 0; r < RD; ++r) acc[i][r] = 0.f;
  for (int t = 0; t < ntiles; ++t) {
    __syncthreads();
    load_k(t * KT);
    load_v(t * KT);
    __syncthreads();
    float sc[NQ];
    scores(t * KT, sc);
#pragma unroll
    for (int i = 0; i < NQ; ++i) {
      // this lane's slot i * QPP + qsub: pick its statistics (qsub is 0 when QPP == 1)
      float mq = m[i * QPP], lq = l[i * QPP];
#pragma unroll
      for (int u = 1; u < QPP; ++u)
        if (qsub == u) {
          mq = m[i * QPP + u];
          lq = l[i * QPP + u];
        }
      const float pe = (sc[i] == -INFINITY) ? 0.f : __builtin_amdgcn_exp2f((sc[i] - mq) * kFaLog2e);
      sP[w][i * QPP + qsub][kk] = T::rnd(pe / lq);
    }
    __syncthreads();
    for (int j = 0; j < KT; j += 4) {
      float vv[4][RD];
#pragma unroll
      for (int t4 = 0; t4 < 4; ++t4)
#pragma unroll
        for (int r = 0; r < RD; ++r) vv[t4][r] = sV[(j + t4) * DMAX + lane + 64 * r];
#pragma unroll
      for (int qs = 0; qs < kFgQW; ++qs) {
        const f32x4v pj = *reinterpret_cast<const f32x4v*>(&sP[w][qs][j]);
#pragma unroll
        for (int t4 = 0; t4 < 4; ++t4)
#pragma unroll
          for (int r = 0; r < RD; ++r) acc[qs][r] = __builtin_fmaf(pj[t4], vv[t4][r], acc[qs][r]);
      }
    }
  }

  typename T::S* Ob = O + b * osb + h * osh;
#pragma unroll
  for (int qs = 0; qs < kFgQW; ++qs) {
    const int q = q0 + w * kFgQW + qs;
    if (q >= Sq) continue;
    const bool nan_row = !(m[qs] > -INFINITY && m[qs] < INFINITY);
#pragma unroll
    for (int r = 0; r < RD; ++r) {
      const int d = lane + 64 * r;
      if (d < D) Ob[(int64_t)q * oss + d] = T::from_f(nan_row ? __builtin_nanf("") : acc[qs][r]);
    }
  }
}

template <typename T>
static int launch_fa_general(const void* Q, const void* K, const void* V, void* O, int64_t B, int64_t Hq,
                             int64_t Hkv, int64_t Sq, int64_t Sk, int64_t D, const int64_t* qs, const int64_t* ks,
                             const int64_t* vs, const int64_t* os, int causal, float sm_scale, hipStream_t st) {
  using S = typename T::S;
  const int64_t nblocks = cdiv(Sq, kFgQB) * Hq * B;
  if (nblocks > INT_MAX) return AK_EINVAL;
  // 4-element loads: D and every row / head / batch stride multiples of 4, bases aligned to 4 elements
  int vec4 = D % 4 == 0;
  const int64_t* all[3] = {qs, ks, vs};
  for (int i = 0; i < 3; ++i)
    for (int j = 0; j < 3; ++j)
      if (all[i][j] % 4 != 0) vec4 = 0;
  const uintptr_t al = 4 * sizeof(S) - 1;
  if ((((uintptr_t)Q) | ((uintptr_t)K) | ((uintptr_t)V)) & al) vec4 = 0;
#define AK_FG(DM)                                                                                           \
  fa_general<T, DM><<<dim3((unsigned)nblocks), kFgWaves * 64, 0, st>>>(                                     \
      (const S*)Q, (const S*)K, (const S*)V, (S*)O, (int)Hq, (int)(Hq / Hkv), (int)Sq, (int)Sk, (int)D,     \
      qs[0], qs[1], qs[2], ks[0], ks[1], ks[2], vs[0], vs[1], vs[2], os[0], os[1], os[2], causal, sm_scale, \
      (int)(Hq * B), vec4)
  if (D <= 64) AK_FG(64);
  else if (D <= 128) AK_FG(128);
  else AK_FG(256);
#undef AK_FG
  return record_launch();
}

template <typename T, int D>
static int launch_fa(const void* Q, const void* K, const void* V, void* O, int64_t B, int64_t Hq,
                     int64_t Hkv, int64_t Sq, int64_t Sk, const int64_t* qs, const int64_t* ks,
                     const int64_t* vs, const int64_t* os, int causal, float sm_scale, hipStream_t st) {
  const int64_t nblocks = cdiv(Sq, kFaBQ) * Hq * B;
  const int64_t nblocks2 = cdiv(Sq, kFa2BQ) * Hq * B;
  if (nblocks > INT_MAX) return AK_EINVAL;
  const dim3 grid((unsigned)nblocks);
  // Scores whose f16 rounding (or f16 scaling by sm_scale) overflows become +-inf.
  const float thr = 65520.0f / fmaxf(1.0f, fabsf(sm_scale));
  // fa_fwd2 folds a positive scale into exp2 and addresses one head's K / V rows with 32-bit
  // byte offsets; anything else takes fa_fwd.
  const int64_t span = (int64_t)2 * Sk * (ks[2] > vs[2] ? ks[2] : vs[2]);
  if (sm_scale > 0.f && span < ((int64_t)1 << 31) && ks[2] >= D && vs[2] >= D) {
    // A grid of at most one block per CU splits each block's keys over two wave groups (the
    // block's serial walk over its key tiles bounds such a grid). Sk >= 256 gives every block at
    // least two key tiles (a causal block's keys reach at least its first 128 queries), so each
    // half has one.
#define AK_FA2(NH)                                                                                  \
  fa_fwd2<T, D, NH><<<dim3((unsigned)nblocks2), kFa2Threads * NH, 0, st>>>(                         \
      (const uint16_t*)Q, (const uint16_t*)K, (const uint16_t*)V, (uint16_t*)O, (int)Hq,            \
      (int)(Hq / Hkv), (int)Sq, (int)Sk, qs[0], qs[1], qs[2], ks[0], ks[1], (int)ks[2], vs[0],     \
      vs[1], (int)vs[2], os[0], os[1], os[2], causal, sm_scale * kFaLog2e,                         \
      T::kCode == AK_F16 ? thr : INFINITY, (int)(Hq * B))
    if (nblocks2 <= kFa2Layer && Sk >= 4 * kFaBKV) AK_FA2(2);
    else AK_FA2(1);
#undef AK_FA2
    return record_launch();
  }
  fa_fwd<T, D><<<grid, kFaThreads, 0, st>>>(
      (const uint16_t*)Q, (const uint16_t*)K, (const uint16_t*)V, (uint16_t*)O, (int)Hq,
      (int)(Hq / Hkv), (int)Sq, (int)Sk, qs[0], qs[1], qs[2], ks[0], ks[1], ks[2], vs[0], vs[1],
      vs[2], os[0], os[1], os[2], causal, sm_scale * kFaLog2e, thr, (int)(Hq * B));
  return record_launch();
}

}  // namespace ak

using namespace ak;

extern "C" int ak_flash_attn_fwd(int dtype, const void* Q, const void* K, const void* V, void* O,
                                 int64_t B, int64_t Hq, int64_t Hkv, int64_t Sq, int64_t Sk,
                                 int64_t D, const int64_t* q_strides, const int64_t* k_strides,
                                 const int64_t* v_strides, const int64_t* o_strides, int causal,
                                 float sm_scale, hipStream_t stream) {
  if (B < 0 || Hq < 0 || Hkv <= 0 || Sq < 0 || Sk < 0 || D <= 0) return AK_EINVAL;
  if (Hq % Hkv != 0) return AK_EINVAL;
  if (!q_strides || !k_strides || !v_strides || !o_strides) return AK_EINVAL;
  if (dtype != AK_F32 && dtype != AK_F16 && dtype != AK_BF16) return AK_EINVAL;
  if (D > 256) return AK_EUNSUPPORTED;
  if (B == 0 || Hq == 0 || Sq == 0) return AK_OK;
  if (!Q || !K || !V || !O) return AK_EINVAL;
  if (B * Hq > INT_MAX || Sq > INT_MAX || Sk > INT_MAX) return AK_EINVAL;
  if (Sk == 0) return AK_EUNSUPPORTED;  // softmax over an empty key set
  const bool c = causal != 0;
  // The MFMA kernels: f16 / bf16, D 64 or 128, 16-byte aligned rows (every stride a multiple of 8
  // elements, 16-byte aligned bases). Everything else runs fa_general.
  bool fast = dtype != AK_F32 && (D == 64 || D == 128);
  const int64_t* all[4] = {q_strides, k_strides, v_strides, o_strides};
  for (int i = 0; i < 4; ++i)
    for (int j = 0; j < 3; ++j)
      if (all[i][j] % 8 != 0) fast = false;
  if (!host_aligned16(Q) || !host_aligned16(K) || !host_aligned16(V) || !host_aligned16(O)) fast = false;
  if (!fast) {
    if (dtype == AK_F32)
      return launch_fa_general<TF32>(Q, K, V, O, B, Hq, Hkv, Sq, Sk, D, q_strides, k_strides, v_strides, o_strides, c, sm_scale, stream);
    if (dtype == AK_F16)
      return launch_fa_general<TF16>(Q, K, V, O, B, Hq, Hkv, Sq, Sk, D, q_strides, k_strides, v_strides, o_strides, c, sm_scale, stream);
    return launch_fa_general<TBF16>(Q, K, V, O, B, Hq, Hkv, Sq, Sk, D, q_strides, k_strides, v_strides, o_strides, c, sm_scale, stream);
  }
  if (dtype == AK_F16) {
    if (D == 64) return launch_fa<TF16, 64>(Q, K, V, O, B, Hq, Hkv, Sq, Sk, q_strides, k_strides, v_strides, o_strides, c, sm_scale, stream);
    return launch_fa<TF16, 128>(Q, K, V, O, B, Hq, Hkv, Sq, Sk, q_strides, k_strides, v_strides, o_strides, c, sm_scale, stream);
  }
  if (D == 64) return launch_fa<TBF16, 64>(Q, K, V, O, B, Hq, Hkv, Sq, Sk, q_strides, k_strides, v_strides, o_strides, c, sm_scale, stream);
  return launch_fa<TBF16, 128>(Q, K, V, O, B, Hq, Hkv, Sq, Sk, q_strides, k_strides, v_strides, o_strides, c, sm_scale, stream);
}
