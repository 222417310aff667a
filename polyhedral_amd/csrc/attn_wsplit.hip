// Attention forward for grids too small to fill the chip (gfx950, float32).
//
// The per-block kernels give a query block of BQ rows to one work-group that walks the
// block's KV list alone.  With few blocks (4 heads x 8 blocks of a 1024-token sequence)
// that leaves most CUs idle and every work-group runs its list serially on fp32 MFMAs.
// Here the work is cut finer and the list is split between waves instead:
//
//  * one work-group of 8 waves per (batch-head, 16 query rows): every wave owns the same
//    16 rows and takes every 8th live 16x16 sub-tile of their list (a listed tile is
//    A / 16 sub-tiles; the index's codes per 32-row x 32-column group say which are dead,
//    full or partial, so dead groups cost nothing and full ones are not masked);
//  * a wave computes S^T = K Q^T for its sub-tile on 16x16x4 f32 MFMAs straight from
//    global memory (lane quarter k holds dimensions [k D/4, (k+1) D/4) of its key and
//    query rows, the same split on both sides, so the contraction covers every
//    dimension), masks a partial sub-tile from the index's element bitmaps (or, without
//    them, by evaluating the predicate), and keeps a running max, sum and O^T = V^T P^T
//    of its own: in the 16x16 accumulator layout lane l holds row l % 16 and keys
//    4 (l / 16) + 0..3, which are exactly the P^T values the P.V MFMAs take from it;
//  * the 8 partial states are merged through LDS (max, rescaled sums, weighted output
//    rows), and the work-group writes the 16 output rows and their log-sum-exp.
//
// Same contract as the general kernel without permutations, class-B emulation or a
// merge input: o rows in float32, lse = natural-log sum-exp, rows with no live key
// give 0 and -inf.
#include "attn_kernel.hpp"

namespace pa {
namespace {

constexpr int kWsWaves = 8;
constexpr int kWsPitch = 17;  // LDS floats per (wave, dimension) row of 16 query rows

template <int D>
constexpr int wsplit_smem_bytes() {
  return (kWsWaves * D * kWsPitch + 2 * kWsWaves * 16) * 4;
}

__device__ __forceinline__ f32x4 mma16(float a, float b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}

// max / sum over the four lanes l % 16 + 16 k that hold one query row
__device__ __forceinline__ float quad_max(float x) {
  x = fmaxf(x, __shfl_xor(x, 16));
  return fmaxf(x, __shfl_xor(x, 32));
}
__device__ __forceinline__ float quad_sum(float x) {
  x += __shfl_xor(x, 16);
  return x + __shfl_xor(x, 32);
}

template <int D>
__global__ __launch_bounds__(kWsWaves * 64) void attn_wsplit_kernel(const AttnK a) {
  constexpr int D4 = D / 4;    // dimensions per lane quarter
  constexpr int NDB = D / 16;  // 16-wide output blocks
  extern __shared__ __attribute__((aligned(16))) float red[];
  __shared__ pa_term terms_s[PA_MAX_TERMS];
  float* red_m = red + kWsWaves * D * kWsPitch;
  float* red_l = red_m + kWsWaves * 16;

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int w = tid >> 6;
  const int kq = lane >> 4;  // lane quarter
  const int m = lane & 15;
  // (32-bit index arithmetic: the grid is below 2^31 work-groups, checked on the host)
  const uint32_t groups = (uint32_t)a.N >> 4;  // 16-row groups per head
  const uint32_t wg = blockIdx.x;
  const int row0 = (int)(wg % groups) * 16;
  const int64_t bh = wg / groups;
  const int qb = row0 / a.BQ;
  const int rt = row0 - qb * a.BQ;  // first row inside the query block
  const int g32 = rt >> 5;          // its 32-row group (index codes)
  const int row = row0 + m;         // this lane's query row (column m of S^T)

  // this lane's quarter of its query row
  float qf[D4];
  {
    const float* qp = reinterpret_cast<const float*>(a.q) + bh * a.q_sb + (int64_t)row * a.q_sn + kq * D4;
#pragma unroll
    for (int c = 0; c < D4; c += 4) {
      const f32x4 x = *reinterpret_cast<const f32x4*>(qp + c);
      qf[c] = x[0];
      qf[c + 1] = x[1];
      qf[c + 2] = x[2];
      qf[c + 3] = x[3];
    }
  }
  const float* kbase = reinterpret_cast<const float*>(a.k) + bh * a.k_sb;
  const float* vbase = reinterpret_cast<const float*>(a.v) + bh * a.v_sb;

  f32x4 acc[NDB];
#pragma unroll
  for (int i = 0; i < NDB; ++i) acc[i] = f32x4{0.f, 0.f, 0.f, 0.f};
  float m_run = -1e30f, l_part = 0.f;

  const int ncg = a.A >> 5;  // 32-column groups per tile
  const int32_t* idx = a.kv_idx + (int64_t)qb * a.pitch;
  const uint32_t* codes = a.kv_wave_bits + (int64_t)qb * a.pitch;
  // the list's first 64 entries, one per lane, loaded together with its length and the
  // query rows rather than one dependent load after another
  const int32_t lane_idx = lane < a.pitch ? idx[lane] : 0;
  const uint32_t lane_code = lane < a.pitch ? codes[lane] : 0u;
  const int32_t* boffs = a.kv_bits_off ? a.kv_bits_off + (int64_t)qb * a.pitch : nullptr;
  const int32_t lane_boff = (boffs && lane < a.pitch) ? boffs[lane] : -1;
  const int n = a.kv_num[qb];
  // without bitmaps, the predicate's terms, for the rolled evaluation of partial
  // sub-tiles (constant indices into the argument block: uniform loads, issued together)
  if (!boffs) {
    if (tid == 0) {
#pragma unroll
      for (int i = 0; i < PA_MAX_TERMS; ++i) terms_s[i] = a.pred.terms[i];
    }
    __syncthreads();
  }
  int live_seen = 0;  // live sub-tiles met so far (uniform)
  for (int t = 0; t < n; ++t) {
    const bool near = t < 64;
    const uint32_t tcode =
        (near ? (uint32_t)__builtin_amdgcn_readlane((int)lane_code, t) : codes[t]) >> (2 * g32 * ncg);
    const int tile = near ? __builtin_amdgcn_readlane(lane_idx, t) : idx[t];
    const int32_t boff = !boffs ? -1 : near ? __builtin_amdgcn_readlane(lane_boff, t) : boffs[t];
    for (int c16 = 0; c16 < 2 * ncg; ++c16) {
      const int cg = c16 >> 1;
      const uint32_t code = (tcode >> (2 * cg)) & 3u;
      if (!code) continue;
      if ((live_seen++ & (kWsWaves - 1)) != w) continue;
      const int col0 = tile * a.A + 16 * c16;
      // K quarter-row of key col0 + m; V column 16 db + m of keys 4 kq + 0..3, the keys
      // this lane's P^T values belong to; this lane's row word of a partial sub-tile's
      // bitmap (bit 16 (c16 % 2) + c = key col0 + c).  All issued before the first MFMA.
      const float* kp = kbase + (int64_t)(col0 + m) * a.k_sn + kq * D4;
      f32x4 kx[D4 / 4];
#pragma unroll
      for (int c = 0; c < D4 / 4; ++c) kx[c] = *reinterpret_cast<const f32x4*>(kp + 4 * c);
      float vx[4][NDB];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float* vp = vbase + (int64_t)(col0 + 4 * kq + i) * a.v_sn + m;
#pragma unroll
        for (int db = 0; db < NDB; ++db) vx[i][db] = vp[16 * db];
      }
      const uint32_t bword =
          (code != 3u && boff >= 0) ? a.kv_bits[(int64_t)boff + (rt + m) * ncg + cg] >> (16 * (c16 & 1)) : 0u;
      f32x4 s = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int c = 0; c < D4 / 4; ++c) {
        s = mma16(kx[c][0], qf[4 * c], s);
        s = mma16(kx[c][1], qf[4 * c + 1], s);
        s = mma16(kx[c][2], qf[4 * c + 2], s);
        s = mma16(kx[c][3], qf[4 * c + 3], s);
      }
      // s[i]: key col0 + 4 kq + i, query row `row`
      if (code != 3u) {
        uint32_t live = 0u;
        if (boff >= 0) {
          live = (bword >> (4 * kq)) & 0xfu;
        } else {
          // a rolled loop keeps one copy of the predicate's term switch in the code
#pragma unroll 1
          for (int i = 0; i < 4; ++i)
            live |= (pred_live_rolled(terms_s, a.pred.n_include, a.pred.n_exclude, row, col0 + 4 * kq + i,
                                      a.pred.dense_bits, a.pred.dense_words)
                         ? 1u
                         : 0u)
                    << i;
        }
#pragma unroll
        for (int i = 0; i < 4; ++i)
          if (!((live >> i) & 1u)) s[i] = -INFINITY;
      }
      const float mx = quad_max(fmaxf(fmaxf(s[0], s[1]), fmaxf(s[2], s[3])));
      const float m_new = fmaxf(m_run, mx * a.c);
      if (m_new > m_run) {
        const float alpha = exp2f(m_run - m_new);
        m_run = m_new;
        l_part *= alpha;
#pragma unroll
        for (int i = 0; i < NDB; ++i) acc[i] *= alpha;
      }
      const float neg_m = -m_run;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float p = __builtin_amdgcn_exp2f(__builtin_fmaf(s[i], a.c, neg_m));
        l_part += p;
        // O^T[d, q] += V^T[d, kv] P^T[kv, q]: MFMA i takes keys 4 k + i (k = lane quarter),
        // whose scores lane quarter k holds in s[i]
#pragma unroll
        for (int db = 0; db < NDB; ++db) acc[db] = mma16(vx[i][db], p, acc[db]);
      }
    }
  }

  // ---- merge of the waves' states ----------------------------------------------------
  const float l_tot = quad_sum(l_part);
  if (kq == 0) {
    red_m[w * 16 + m] = m_run;
    red_l[w * 16 + m] = l_tot;
  }
  __syncthreads();
  float M = -INFINITY;
#pragma unroll
  for (int u = 0; u < kWsWaves; ++u) M = fmaxf(M, red_m[u * 16 + m]);
  float L = 0.f;
#pragma unroll
  for (int u = 0; u < kWsWaves; ++u) L += red_l[u * 16 + m] * exp2f(red_m[u * 16 + m] - M);
  const float f = (l_tot > 0.f && L > 0.f) ? exp2f(m_run - M) / L : 0.f;
  // acc[db][i]: dimension 16 db + 4 kq + i of row m
#pragma unroll
  for (int db = 0; db < NDB; ++db)
#pragma unroll
    for (int i = 0; i < 4; ++i) red[(w * D + 16 * db + 4 * kq + i) * kWsPitch + m] = acc[db][i] * f;
  if (w == 0 && kq == 0 && a.lse) a.lse[bh * a.lse_sb + row] = L > 0.f ? (M + log2f(L)) * kLn2 : -INFINITY;
  __syncthreads();
  // 16 rows x D/4 float4 outputs, summed over the waves
  for (int e = tid; e < 16 * (D / 4); e += kWsWaves * 64) {
    const int r = e / (D / 4);
    const int d0 = 4 * (e % (D / 4));
    f32x4 x = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int u = 0; u < kWsWaves; ++u)
#pragma unroll
      for (int k = 0; k < 4; ++k) x[k] += red[(u * D + d0 + k) * kWsPitch + r];
    float* op = reinterpret_cast<float*>(a.o) + bh * a.o_sb + (int64_t)(row0 + r) * a.o_sn + d0;
    *reinterpret_cast<f32x4*>(op) = x;
  }
}

template <int D>
int launch_wsplit_d(const AttnK& a, hipStream_t s) {
  constexpr int smem = wsplit_smem_bytes<D>();
  static unsigned long long configured = 0ull;  // one bit per device
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return hip_fail(e, "hipGetDevice");
  if (dev >= 64 || !((configured >> dev) & 1ull)) {
    e = hipFuncSetAttribute(reinterpret_cast<const void*>(&attn_wsplit_kernel<D>),
                            hipFuncAttributeMaxDynamicSharedMemorySize, smem);
    if (e != hipSuccess) return hip_fail(e, "hipFuncSetAttribute(attn_wsplit_kernel)");
    if (dev < 64) configured |= 1ull << dev;
  }
  const int64_t grid = a.BH * (a.N / 16);
  hipLaunchKernelGGL((attn_wsplit_kernel<D>), dim3((unsigned)grid), dim3(kWsWaves * 64), smem, s, a);
  PA_LAUNCH_CHECK("attn_wsplit_kernel");
  return PA_OK;
}

}  // namespace

int launch_attn_wsplit(const AttnK& a, int D, hipStream_t s) {
  if (D == 64) return launch_wsplit_d<64>(a, s);
  if (D == 128) return launch_wsplit_d<128>(a, s);
  set_error("attention: no wave-split kernel for D=%d", D);
  return PA_E_UNSUPPORTED;
}

}  // namespace pa
