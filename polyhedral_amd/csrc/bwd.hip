// Backward of the block-sparse masked attention (gfx950, f16 / bf16, D = 64 or 128).
//
// The reference has no backward (gpu/triton_attn.py:9-10, README.md:118); this is the
// textbook gradient of o = softmax(scale q k^T, masked) v with the forward's row
// log-sum-exp saved: with P = exp(scale q k^T - lse) on live pairs (0 elsewhere),
//   dV = P^T dO,  dP = dO V^T,  dS = P * (dP - rowsum(dO * O)),
//   dQ = scale dS K,  dK = scale dS^T Q.
// Rows with no live key have P = 0 and get no gradient.
//
// Tiles are 64 x 64 (query block x key block), from the block index built at
// BQ = A = 64 and its transpose (pa_index_transpose).  Two kernels, no atomics:
//  * bwd_dkdv_kernel: one work-group of 2 waves per (key block, head), wave w owning 32
//    keys.  Its K and V rows stay in registers; per listed query block the Q and dO
//    rows (plus lse and rowsum(dO * O)) are staged in LDS, S = Q K^T and dP = dO V^T come
//    out with the wave's keys along the lanes, and dV^T += dO^T P, dK^T += Q^T dS use
//    transposed LDS reads of dO and Q.
//  * bwd_dq_kernel: one work-group of 2 waves per (query block, head), the same with the
//    roles of queries and keys exchanged (the forward's layout): S^T = K Q^T,
//    dP^T = V dO^T, dQ^T += K^T dS^T.
// Both evaluate the mask on partial tiles only, in original coordinates (perm_q /
// perm_kv map index-space rows to them, as in the forward).
#include <math.h>

#include "attn_kernel.hpp"

namespace pa {
namespace {

constexpr int kBT = 64;  // tile side (query rows = key rows)

struct BwdK {
  const char* q;
  const char* k;
  const char* v;
  const char* o;
  const char* dout;
  char* dq;
  char* dk;
  char* dv;
  int64_t sb, sn;          // element strides shared by every [BH, N, D] tensor
  const float* lse;        // [BH, N], natural log
  float* dvec;             // [BH, N]: rowsum(dO * O)
  int64_t lse_sb;
  int32_t N, nb;           // nb = N / 64
  float c;                 // scale * log2(e)
  float scale;
  const int32_t* kv_idx;   // [nb, pitch] key blocks of each query block
  const int32_t* kv_num;
  const int8_t* kv_partial;
  int64_t pitch;
  const int32_t* q_idx;    // [nb, tpitch] query blocks of each key block
  const int32_t* q_num;
  const int8_t* q_partial;
  int64_t tpitch;
  Pred pred;
};

// rowsum(dO * O) of one row per thread, in fp32.
template <typename T, int D>
__global__ __launch_bounds__(256) void bwd_pre_kernel(const BwdK a, int64_t rows) {
  const int64_t r = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (r >= rows) return;
  const int64_t bh = r / a.N, i = r - bh * a.N;
  const char* op = a.o + (bh * a.sb + i * a.sn) * (int64_t)sizeof(T);
  const char* dp = a.dout + (bh * a.sb + i * a.sn) * (int64_t)sizeof(T);
  constexpr int DT = __is_same(T, __bf16) ? PA_BF16 : PA_F16;
  float acc = 0.f;
#pragma unroll
  for (int d = 0; d < D; d += 4) {
    const f32x4 x = load4_any(op + d * sizeof(T), DT);
    const f32x4 y = load4_any(dp + d * sizeof(T), DT);
    acc += x[0] * y[0] + x[1] * y[1] + x[2] * y[2] + x[3] * y[3];
  }
  a.dvec[bh * a.lse_sb + i] = acc;
}

// LDS pitches of a staged 64-row tile: the K-style pitch (+16 B) serves the 16-byte row
// reads, the V-style pitch (+64 B) the transposed reads; a tile read both ways is
// staged twice.
template <typename T, int D>
constexpr int npitch() { return D * (int)sizeof(T) + 16; }
template <typename T, int D>
constexpr int tpitch() { return D * (int)sizeof(T) + 64; }

// Stage rows r0 .. r0 + 63 of a [BH, N, D] tensor into LDS at the row-read pitch and,
// with TR, also at the transposed-read pitch.  128 threads; a fixed unit count per
// thread, so every load is issued before any store.
template <typename T, int D, bool TR>
__device__ __forceinline__ void stage_tile(const char* base, int64_t sn, int r0, char* dst_n, char* dst_t, int tid) {
  constexpr int UPR = D * (int)sizeof(T) / 16;
  constexpr int PER = kBT * UPR / 128;
  uint4 x[PER];
#pragma unroll
  for (int i = 0; i < PER; ++i) {
    const int u = tid + 128 * i, r = u / UPR, c = u % UPR;
    x[i] = *reinterpret_cast<const uint4*>(base + ((int64_t)(r0 + r) * sn) * (int64_t)sizeof(T) + 16 * c);
  }
#pragma unroll
  for (int i = 0; i < PER; ++i) {
    const int u = tid + 128 * i, r = u / UPR, c = u % UPR;
    *reinterpret_cast<uint4*>(dst_n + r * npitch<T, D>() + 16 * c) = x[i];
    if constexpr (TR) *reinterpret_cast<uint4*>(dst_t + r * tpitch<T, D>() + 16 * c) = x[i];
  }
}

// Fragments of 16-byte row reads: lane (m, G) holds row m, bytes (16 kc + 8 G) * esz.
template <typename T, int D>
__device__ __forceinline__ void row_frags(const char* row, typename Mma<T>::frag* f) {
#pragma unroll
  for (int kc = 0; kc < D / 16; ++kc) f[kc] = __builtin_bit_cast(typename Mma<T>::frag, *reinterpret_cast<const uint4*>(row + kc * 32));
}

// A operand X^T[d][r] of a transposed product for rows 16 c + 4 G + 0..3 and
// 16 c + 8 + 4 G + 0..3 of a tile staged at the V-style pitch (the rows whose values
// this lane holds in elements 8 c .. 8 c + 7 of an accumulator): block db of D.
template <typename T, int D>
__device__ __forceinline__ typename Mma<T>::frag tr_frag(const char* tile_t, int lane, int G, int rbase, int db) {
  constexpr int TP = tpitch<T, D>();
  const int j16 = lane & 15;
  const char* p = tile_t + (rbase + 4 * G + (j16 >> 2)) * TP + (((lane >> 4) & 1) * 16 + 4 * (j16 & 3)) * 2 + db * 64;
  const s16x4 x1 = lds_read_tr(p);
  const s16x4 x2 = lds_read_tr(p + 8 * TP);
  const uint4 vx = {__builtin_bit_cast(uint2, x1).x, __builtin_bit_cast(uint2, x1).y, __builtin_bit_cast(uint2, x2).x,
                    __builtin_bit_cast(uint2, x2).y};
  return __builtin_bit_cast(typename Mma<T>::frag, vx);
}

__device__ __forceinline__ int32_t orig_of(const int32_t* perm, int32_t r) { return perm ? perm[r] : r; }

// ---------------------------------------------------------------------------------
template <typename T, int D>
__global__ __launch_bounds__(128) __attribute__((amdgpu_waves_per_eu(1))) void bwd_dkdv_kernel(const BwdK a) {
  using Frag = typename Mma<T>::frag;
  constexpr int ESZ = sizeof(T);
  constexpr int NKC = D / 16;
  constexpr int NDB = D / 32;
  constexpr int NP = npitch<T, D>();
  constexpr int TP = tpitch<T, D>();
  __shared__ __attribute__((aligned(16))) char q_n[kBT * NP];
  __shared__ __attribute__((aligned(16))) char q_t[kBT * TP];
  __shared__ __attribute__((aligned(16))) char do_n[kBT * NP];
  __shared__ __attribute__((aligned(16))) char do_t[kBT * TP];
  __shared__ float lse_s[kBT], dvec_s[kBT];
  __shared__ int32_t qo_s[kBT];
  __shared__ pa_term terms_s[PA_MAX_TERMS];
#pragma unroll
  for (int i = 0; i < PA_MAX_TERMS; ++i)  // (constant indices into the argument block)
    if (threadIdx.x == i) terms_s[i] = a.pred.terms[i];

  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, G = lane >> 5, m = lane & 31;
  const int kb = blockIdx.x;
  const int64_t bh = blockIdx.y;
  const int key = kb * kBT + w * 32 + m;  // this lane's key (index space)
  const int key_o = orig_of(a.pred.perm_kv, key);
  const char* hq = a.q + bh * a.sb * ESZ;
  const char* hdo = a.dout + bh * a.sb * ESZ;

  Frag kf[NKC], vf[NKC];
  row_frags<T, D>(a.k + (bh * a.sb + (int64_t)key * a.sn) * ESZ + 16 * G, kf);
  row_frags<T, D>(a.v + (bh * a.sb + (int64_t)key * a.sn) * ESZ + 16 * G, vf);
  f32x16 dkt[NDB], dvt[NDB];
#pragma unroll
  for (int i = 0; i < NDB; ++i) dkt[i] = dvt[i] = f32x16{0};

  const int nl = a.q_num[kb];
  for (int t = 0; t < nl; ++t) {
    const int qb = a.q_idx[(int64_t)kb * a.tpitch + t];
    const bool partial = a.q_partial[(int64_t)kb * a.tpitch + t] != 0;
    __syncthreads();  // the previous block's tiles are consumed
    stage_tile<T, D, true>(hq, a.sn, qb * kBT, q_n, q_t, tid);
    stage_tile<T, D, true>(hdo, a.sn, qb * kBT, do_n, do_t, tid);
    if (tid < kBT) {
      const float l = a.lse[bh * a.lse_sb + qb * kBT + tid];
      lse_s[tid] = l * 1.4426950408889634f;
      dvec_s[tid] = a.dvec[bh * a.lse_sb + qb * kBT + tid];
      qo_s[tid] = orig_of(a.pred.perm_q, qb * kBT + tid);
    }
    __syncthreads();
#pragma unroll
    for (int lb = 0; lb < 2; ++lb) {
      // S = Q K^T and dP = dO V^T for query rows 32 lb .. +31: element i of the lane is
      // query row 32 lb + 8 (i / 4) + 4 G + i % 4, key `key`
      f32x16 s = f32x16{0}, dp = f32x16{0};
      const char* qrow = q_n + (32 * lb + m) * NP + 16 * G;
      const char* drow = do_n + (32 * lb + m) * NP + 16 * G;
#pragma unroll
      for (int kc = 0; kc < NKC; ++kc) {
        s = Mma<T>::mma(__builtin_bit_cast(Frag, *reinterpret_cast<const uint4*>(qrow + kc * 32)), kf[kc], s);
        dp = Mma<T>::mma(__builtin_bit_cast(Frag, *reinterpret_cast<const uint4*>(drow + kc * 32)), vf[kc], dp);
      }
      // live bit i of the lane's elements: all set on a full tile, one rolled copy of the
      // predicate (terms from LDS) on a partial one
      uint32_t live = 0xffffu;
      if (partial) {
        live = 0u;
#pragma unroll 1
        for (int i = 0; i < 16; ++i) {
          const int qr = 32 * lb + 8 * (i >> 2) + 4 * G + (i & 3);
          if (pred_live_rolled(terms_s, a.pred.n_include, a.pred.n_exclude, qo_s[qr], key_o, a.pred.dense_bits,
                               a.pred.dense_words))
            live |= 1u << i;
        }
      }
      float p[16], ds[16];
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const int qr = 32 * lb + 8 * (i >> 2) + 4 * G + (i & 3);
        const float l2 = lse_s[qr];
        p[i] = (((live >> i) & 1u) && l2 != -INFINITY) ? __builtin_amdgcn_exp2f(__builtin_fmaf(s[i], a.c, -l2)) : 0.f;
        ds[i] = p[i] * (dp[i] - dvec_s[qr]);
      }
#pragma unroll
      for (int c = 0; c < 2; ++c) {
        f32x8 pv, sv;
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          pv[e] = p[8 * c + e];
          sv[e] = ds[8 * c + e];
        }
        const Frag pf = Mma<T>::cvt(pv), sf = Mma<T>::cvt(sv);
#pragma unroll
        for (int db = 0; db < NDB; ++db) {
          dvt[db] = Mma<T>::mma(tr_frag<T, D>(do_t, lane, G, 32 * lb + 16 * c, db), pf, dvt[db]);
          dkt[db] = Mma<T>::mma(tr_frag<T, D>(q_t, lane, G, 32 * lb + 16 * c, db), sf, dkt[db]);
        }
      }
    }
  }
  // dK^T / dV^T blocks [32 d x 32 keys]: lane (key m, G) holds d = 32 db + 8 i4 + 4 G + 0..3
  char* dkrow = a.dk + (bh * a.sb + (int64_t)key * a.sn) * ESZ;
  char* dvrow = a.dv + (bh * a.sb + (int64_t)key * a.sn) * ESZ;
#pragma unroll
  for (int db = 0; db < NDB; ++db) {
#pragma unroll
    for (int i4 = 0; i4 < 4; ++i4) {
      const int d0 = 32 * db + 8 * i4 + 4 * G;
      f32x4 xk = {dkt[db][4 * i4], dkt[db][4 * i4 + 1], dkt[db][4 * i4 + 2], dkt[db][4 * i4 + 3]};
      const f32x4 xv = {dvt[db][4 * i4], dvt[db][4 * i4 + 1], dvt[db][4 * i4 + 2], dvt[db][4 * i4 + 3]};
      xk *= a.scale;
      Mma<T>::store4(dkrow + d0 * ESZ, xk);
      Mma<T>::store4(dvrow + d0 * ESZ, xv);
    }
  }
}

// ---------------------------------------------------------------------------------
template <typename T, int D>
__global__ __launch_bounds__(128) __attribute__((amdgpu_waves_per_eu(2))) void bwd_dq_kernel(const BwdK a) {
  using Frag = typename Mma<T>::frag;
  constexpr int ESZ = sizeof(T);
  constexpr int NKC = D / 16;
  constexpr int NDB = D / 32;
  constexpr int NP = npitch<T, D>();
  constexpr int TP = tpitch<T, D>();
  __shared__ __attribute__((aligned(16))) char k_n[kBT * NP];
  __shared__ __attribute__((aligned(16))) char k_t[kBT * TP];
  __shared__ __attribute__((aligned(16))) char v_n[kBT * NP];
  __shared__ int32_t ko_s[kBT];
  __shared__ pa_term terms_s[PA_MAX_TERMS];
#pragma unroll
  for (int i = 0; i < PA_MAX_TERMS; ++i)
    if (threadIdx.x == i) terms_s[i] = a.pred.terms[i];

  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, G = lane >> 5, m = lane & 31;
  const int qb = blockIdx.x;
  const int64_t bh = blockIdx.y;
  const int row = qb * kBT + w * 32 + m;  // this lane's query row (index space)
  const int q_o = orig_of(a.pred.perm_q, row);
  const char* hk = a.k + bh * a.sb * ESZ;
  const char* hv = a.v + bh * a.sb * ESZ;

  Frag qf[NKC], df[NKC];
  row_frags<T, D>(a.q + (bh * a.sb + (int64_t)row * a.sn) * ESZ + 16 * G, qf);
  row_frags<T, D>(a.dout + (bh * a.sb + (int64_t)row * a.sn) * ESZ + 16 * G, df);
  const float l2 = a.lse[bh * a.lse_sb + row] * 1.4426950408889634f;
  const float dr = a.dvec[bh * a.lse_sb + row];
  f32x16 dqt[NDB];
#pragma unroll
  for (int i = 0; i < NDB; ++i) dqt[i] = f32x16{0};

  const int nl = a.kv_num[qb];
  for (int t = 0; t < nl; ++t) {
    const int kb = a.kv_idx[(int64_t)qb * a.pitch + t];
    const bool partial = a.kv_partial[(int64_t)qb * a.pitch + t] != 0;
    __syncthreads();
    stage_tile<T, D, true>(hk, a.sn, kb * kBT, k_n, k_t, tid);
    stage_tile<T, D, false>(hv, a.sn, kb * kBT, v_n, nullptr, tid);
    if (tid < kBT) ko_s[tid] = orig_of(a.pred.perm_kv, kb * kBT + tid);
    __syncthreads();
#pragma unroll
    for (int lb = 0; lb < 2; ++lb) {
      // S^T = K Q^T and dP^T = V dO^T for keys 32 lb .. +31: element i is key
      // 32 lb + 8 (i / 4) + 4 G + i % 4, query `row`
      f32x16 s = f32x16{0}, dp = f32x16{0};
      const char* krow = k_n + (32 * lb + m) * NP + 16 * G;
      const char* vrow = v_n + (32 * lb + m) * NP + 16 * G;
#pragma unroll
      for (int kc = 0; kc < NKC; ++kc) {
        s = Mma<T>::mma(__builtin_bit_cast(Frag, *reinterpret_cast<const uint4*>(krow + kc * 32)), qf[kc], s);
        dp = Mma<T>::mma(__builtin_bit_cast(Frag, *reinterpret_cast<const uint4*>(vrow + kc * 32)), df[kc], dp);
      }
      uint32_t live = 0xffffu;
      if (partial) {
        live = 0u;
#pragma unroll 1
        for (int i = 0; i < 16; ++i) {
          const int kr = 32 * lb + 8 * (i >> 2) + 4 * G + (i & 3);
          if (pred_live_rolled(terms_s, a.pred.n_include, a.pred.n_exclude, q_o, ko_s[kr], a.pred.dense_bits,
                               a.pred.dense_words))
            live |= 1u << i;
        }
      }
      float ds[16];
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const float p =
            (((live >> i) & 1u) && l2 != -INFINITY) ? __builtin_amdgcn_exp2f(__builtin_fmaf(s[i], a.c, -l2)) : 0.f;
        ds[i] = p * (dp[i] - dr);
      }
#pragma unroll
      for (int c = 0; c < 2; ++c) {
        f32x8 sv;
#pragma unroll
        for (int e = 0; e < 8; ++e) sv[e] = ds[8 * c + e];
        const Frag sf = Mma<T>::cvt(sv);
#pragma unroll
        for (int db = 0; db < NDB; ++db)
          dqt[db] = Mma<T>::mma(tr_frag<T, D>(k_t, lane, G, 32 * lb + 16 * c, db), sf, dqt[db]);
      }
    }
  }
  char* dqrow = a.dq + (bh * a.sb + (int64_t)row * a.sn) * ESZ;
#pragma unroll
  for (int db = 0; db < NDB; ++db) {
#pragma unroll
    for (int i4 = 0; i4 < 4; ++i4) {
      const int d0 = 32 * db + 8 * i4 + 4 * G;
      f32x4 x = {dqt[db][4 * i4], dqt[db][4 * i4 + 1], dqt[db][4 * i4 + 2], dqt[db][4 * i4 + 3]};
      x *= a.scale;
      Mma<T>::store4(dqrow + d0 * ESZ, x);
    }
  }
}

// Transposed block lists: for key block kb, the query blocks whose list holds kb, in
// ascending order, with the partial flag.  One thread per key block; each query block's
// list is sorted, so membership is a binary search.  q_idx == nullptr: counts only.
__global__ __launch_bounds__(256) void transpose_kernel(const int32_t* kv_idx, const int32_t* kv_num,
                                                        const int8_t* kv_partial, int32_t nq, int64_t pitch,
                                                        int32_t nk, int32_t* q_num, int32_t* q_idx, int8_t* q_partial,
                                                        int64_t tp) {
  const int kb = blockIdx.x * 256 + threadIdx.x;
  if (kb >= nk) return;
  int n = 0;
  for (int qb = 0; qb < nq; ++qb) {
    const int32_t* row = kv_idx + (int64_t)qb * pitch;
    int lo = 0, hi = kv_num[qb];
    while (lo < hi) {
      const int mid = (lo + hi) >> 1;
      if (row[mid] < kb)
        lo = mid + 1;
      else
        hi = mid;
    }
    if (lo < kv_num[qb] && row[lo] == kb) {
      if (q_idx && n < tp) {
        q_idx[(int64_t)kb * tp + n] = qb;
        q_partial[(int64_t)kb * tp + n] = kv_partial[(int64_t)qb * pitch + lo];
      }
      ++n;
    }
  }
  q_num[kb] = n;
}

template <typename T, int D>
int launch_bwd(const BwdK& k, int64_t BH, hipStream_t s) {
  const int64_t rows = BH * k.N;
  hipLaunchKernelGGL((bwd_pre_kernel<T, D>), dim3((unsigned)((rows + 255) / 256)), dim3(256), 0, s, k, rows);
  PA_LAUNCH_CHECK("bwd_pre_kernel");
  hipLaunchKernelGGL((bwd_dkdv_kernel<T, D>), dim3((unsigned)k.nb, (unsigned)BH), dim3(128), 0, s, k);
  PA_LAUNCH_CHECK("bwd_dkdv_kernel");
  hipLaunchKernelGGL((bwd_dq_kernel<T, D>), dim3((unsigned)k.nb, (unsigned)BH), dim3(128), 0, s, k);
  PA_LAUNCH_CHECK("bwd_dq_kernel");
  return PA_OK;
}

}  // namespace
}  // namespace pa

extern "C" int pa_index_transpose(const int32_t* kv_idx, const int32_t* kv_num, const int8_t* kv_partial, int32_t nq,
                                  int64_t pitch, int32_t nk, int32_t* q_num, int32_t* q_idx, int8_t* q_partial,
                                  int64_t tpitch, void* stream) {
  PA_CHECK_ARG(kv_num && q_num && nq >= 1 && nk >= 1 && pitch >= 0 && tpitch >= 0, "pa_index_transpose: bad arguments");
  PA_CHECK_ARG(pitch == 0 || kv_idx, "pa_index_transpose: null kv_idx");
  PA_CHECK_ARG(!q_idx || q_partial, "pa_index_transpose: q_idx needs q_partial");
  hipStream_t s = static_cast<hipStream_t>(stream);
  hipLaunchKernelGGL(pa::transpose_kernel, dim3((unsigned)((nk + 255) / 256)), dim3(256), 0, s, kv_idx, kv_num,
                     kv_partial, nq, pitch, nk, q_num, q_idx, q_partial, tpitch);
  PA_LAUNCH_CHECK("transpose_kernel");
  return PA_OK;
}

extern "C" int pa_attn_bwd(const pa_attn_bwd_args* x, void* stream) {
  PA_CHECK_ARG(x, "pa_attn_bwd: null arguments");
  PA_CHECK_ARG(x->dtype == PA_BF16 || x->dtype == PA_F16, "pa_attn_bwd: dtype must be f16 or bf16");
  PA_CHECK_ARG(x->D == 64 || x->D == 128, "pa_attn_bwd: D=%d (64 or 128)", x->D);
  PA_CHECK_ARG(x->BH >= 1 && x->BH <= 65535, "pa_attn_bwd: BH=%lld", (long long)x->BH);
  PA_CHECK_ARG(x->N >= 64 && x->N % 64 == 0 && x->N < (1ll << 31), "pa_attn_bwd: N=%lld must be a multiple of 64",
               (long long)x->N);
  PA_CHECK_ARG(x->q && x->k && x->v && x->o && x->dout && x->dq && x->dk && x->dv && x->lse && x->dvec,
               "pa_attn_bwd: null tensor");
  PA_CHECK_ARG(x->kv_num && x->q_num && (x->pitch == 0 || (x->kv_idx && x->kv_partial)) &&
                   (x->tpitch == 0 || (x->q_idx && x->q_partial)),
               "pa_attn_bwd: null index array");
  PA_CHECK_ARG(x->sn >= x->D && x->sb >= x->sn, "pa_attn_bwd: strides sb=%lld sn=%lld", (long long)x->sb,
               (long long)x->sn);
  auto al = [&](const void* p) { return (reinterpret_cast<uintptr_t>(p) % 16) == 0; };
  PA_CHECK_ARG(al(x->q) && al(x->k) && al(x->v) && al(x->o) && al(x->dout) && al(x->dq) && al(x->dk) && al(x->dv) &&
                   (x->sn * 2) % 16 == 0 && (x->sb * 2) % 16 == 0,
               "pa_attn_bwd: rows must be 16-byte aligned");
  const int rc = pa::check_mask(&x->mask, x->N);
  if (rc) return rc;
  pa::BwdK k;
  k.q = static_cast<const char*>(x->q);
  k.k = static_cast<const char*>(x->k);
  k.v = static_cast<const char*>(x->v);
  k.o = static_cast<const char*>(x->o);
  k.dout = static_cast<const char*>(x->dout);
  k.dq = static_cast<char*>(x->dq);
  k.dk = static_cast<char*>(x->dk);
  k.dv = static_cast<char*>(x->dv);
  k.sb = x->sb;
  k.sn = x->sn;
  k.lse = x->lse;
  k.dvec = x->dvec;
  k.lse_sb = x->lse_sb > 0 ? x->lse_sb : x->N;
  k.N = (int32_t)x->N;
  k.nb = (int32_t)(x->N / 64);
  k.scale = x->scale > 0.f ? x->scale : 1.f / sqrtf((float)x->D);
  k.c = k.scale * 1.4426950408889634f;
  k.kv_idx = x->kv_idx;
  k.kv_num = x->kv_num;
  k.kv_partial = x->kv_partial;
  k.pitch = x->pitch;
  k.q_idx = x->q_idx;
  k.q_num = x->q_num;
  k.q_partial = x->q_partial;
  k.tpitch = x->tpitch;
  k.pred = pa::make_pred(x->mask);
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (x->dtype == PA_BF16) return x->D == 128 ? pa::launch_bwd<__bf16, 128>(k, x->BH, s) : pa::launch_bwd<__bf16, 64>(k, x->BH, s);
  return x->D == 128 ? pa::launch_bwd<_Float16, 128>(k, x->BH, s) : pa::launch_bwd<_Float16, 64>(k, x->BH, s);
}
