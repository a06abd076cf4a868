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
// Lazy rescale: the running max used as the exp2 base is only raised when a tile's max exceeds
// it by more than this (log2 units), so P stays <= 2^8 (exact in f16 / bf16 range) and the O
// accumulator is rescaled only a handful of times per row instead of on most tiles.
constexpr float kFaRescaleSlack = 8.0f;

#ifndef AK_FA_WAVES
#define AK_FA_WAVES 4
#endif
constexpr int kFaWaves = AK_FA_WAVES;        // waves per block, 32 query rows each
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
      // raise the base only when the tile's max passes it by more than the slack (or it is
      // still -inf / the tile holds +inf / NaN, which must propagate exactly)
      const float m_new = (m_tile > m_run + kFaRescaleSlack || m_run == -INFINITY || !(m_tile == m_tile) ||
                           m_tile == INFINITY) ? fmaxf(m_run, m_tile) : m_run;
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
  const float inv = 1.0f / l_tot;
  if (my_q < Sq) {
    uint16_t* orow = Ob + (int64_t)my_q * oss;
#pragma unroll
    for (int db = 0; db < NDB; ++db)
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int d = db * 32 + g * 8 + hh * 4;
        u32x2 pk;
        pk[0] = (uint32_t)T::from_f(o[db][g * 4 + 0] * inv) | ((uint32_t)T::from_f(o[db][g * 4 + 1] * inv) << 16);
        pk[1] = (uint32_t)T::from_f(o[db][g * 4 + 2] * inv) | ((uint32_t)T::from_f(o[db][g * 4 + 3] * inv) << 16);
        *reinterpret_cast<u32x2*>(orow + d) = pk;
      }
  }
}

template <typename T, int D>
static int launch_fa(const void* Q, const void* K, const void* V, void* O, int64_t B, int64_t Hq,
                     int64_t Hkv, int64_t Sq, int64_t Sk, const int64_t* qs, const int64_t* ks,
                     const int64_t* vs, const int64_t* os, int causal, float sm_scale, hipStream_t st) {
  const int64_t nblocks = cdiv(Sq, kFaBQ) * Hq * B;
  if (nblocks > INT_MAX) return AK_EINVAL;
  const dim3 grid((unsigned)nblocks);
  // Scores whose f16 rounding (or f16 scaling by sm_scale) overflows become +-inf.
  const float thr = 65520.0f / fmaxf(1.0f, fabsf(sm_scale));
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
  if (B < 0 || Hq < 0 || Hkv <= 0 || Sq < 0 || Sk < 0) return AK_EINVAL;
  if (Hq % Hkv != 0) return AK_EINVAL;
  if (!q_strides || !k_strides || !v_strides || !o_strides) return AK_EINVAL;
  if (B == 0 || Hq == 0 || Sq == 0) return AK_OK;
  if (!Q || !K || !V || !O) return AK_EINVAL;
  if (B * Hq > INT_MAX || Sq > INT_MAX || Sk > INT_MAX) return AK_EINVAL;
  if (dtype != AK_F16 && dtype != AK_BF16) return AK_EUNSUPPORTED;
  if (D != 64 && D != 128) return AK_EUNSUPPORTED;
  // 16-byte aligned rows: every stride a multiple of 8 elements, 16-byte aligned bases
  const int64_t* all[4] = {q_strides, k_strides, v_strides, o_strides};
  for (int i = 0; i < 4; ++i)
    for (int j = 0; j < 3; ++j)
      if (all[i][j] % 8 != 0) return AK_EUNSUPPORTED;
  if (!host_aligned16(Q) || !host_aligned16(K) || !host_aligned16(V) || !host_aligned16(O)) return AK_EUNSUPPORTED;
  if (Sk == 0) return AK_EUNSUPPORTED;  // softmax over an empty key set
  const bool c = causal != 0;
  if (dtype == AK_F16) {
    if (D == 64) return launch_fa<TF16, 64>(Q, K, V, O, B, Hq, Hkv, Sq, Sk, q_strides, k_strides, v_strides, o_strides, c, sm_scale, stream);
    return launch_fa<TF16, 128>(Q, K, V, O, B, Hq, Hkv, Sq, Sk, q_strides, k_strides, v_strides, o_strides, c, sm_scale, stream);
  }
  if (D == 64) return launch_fa<TBF16, 64>(Q, K, V, O, B, Hq, Hkv, Sq, Sk, q_strides, k_strides, v_strides, o_strides, c, sm_scale, stream);
  return launch_fa<TBF16, 128>(Q, K, V, O, B, Hq, Hkv, Sq, Sk, q_strides, k_strides, v_strides, o_strides, c, sm_scale, stream);
}
