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
// BQ = A = 64 and its transpose (pa_index_transpose).  Two passes, no atomics:
//  * dK / dV, per (key block, head): S = Q K^T and dP = dO V^T come out with the keys
//    along the lanes, and dV^T += dO^T P, dK^T += Q^T dS use transposed LDS reads of dO
//    and Q.  D = 64: bwd_dkdv_kernel, 2 waves of 32 keys, tiles staged through registers.
//    D = 128: bwd_dkdv_pair_kernel, 4 waves, a pair per 32 keys with the two products
//    split between the pair's waves, tiles by LDS DMA.
//  * dQ, per (query block, head), the same with the roles of queries and keys exchanged
//    (the forward's layout): S^T = K Q^T, dP^T = V dO^T, dQ^T += K^T dS^T.  D = 64:
//    bwd_dq_kernel; D = 128: bwd_dq_stream_kernel (tiles by LDS DMA).
// Partial tiles are masked from element bitmaps when given (D = 128), else by evaluating
// the mask in original coordinates (perm_q / perm_kv map index-space rows to them, as in
// the forward).
#include <math.h>

#include <type_traits>

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
  const int32_t* kv_bits_off;  // [nb, pitch] bitmap word offsets (-1: full), or NULL
  const uint32_t* kv_bits;     // 64 rows x 2 words per partial tile, row-major
  const int32_t* q_bits_off;   // [nb, tpitch], same offsets in the transposed lists
  const uint32_t* q_bits;      // the same bitmaps transposed (64 columns x 2 words)
  int32_t accumulate;          // add into dq / dk / dv
  // > 0 (D = 128 only): the tensors (and lse, dvec) are in ORIGINAL order and index-space
  // row r lives at row (r mod 2^qlog2) s + r div 2^qlog2 (the residue-s permutation in
  // closed form); a 64-row tile is then 64 rows s apart
  int32_t residue_s, residue_qlog2;
  const int32_t* kv_order;     // issue order of the key blocks in the dK / dV pass, or NULL
  Pred pred;
};

// Memory row of index-space row r.
__device__ __forceinline__ int64_t mem_row(const BwdK& a, int r) {
  return a.residue_s ? (int64_t)(r & ((1 << a.residue_qlog2) - 1)) * a.residue_s + (r >> a.residue_qlog2) : r;
}

// 4 gradient elements stored (or added to the stored ones) in the tensor's type.
template <typename T>
__device__ __forceinline__ void store_grad4(char* p, f32x4 x, bool acc) {
  if (acc) x += load4_any(p, __is_same(T, __bf16) ? PA_BF16 : PA_F16);
  Mma<T>::store4(p, x);
}

// rowsum(dO * O) in fp32: a row per D / 8 lanes, 16 bytes of each tensor per lane (the
// loads of a wave cover whole rows), summed across the row's lanes.
template <typename T, int D>
__global__ __launch_bounds__(256) void bwd_pre_kernel(const BwdK a, int64_t rows) {
  constexpr int LPR = D / 8;  // lanes per row
  const int64_t g = (int64_t)blockIdx.x * 256 + threadIdx.x;
  const int64_t r = g / LPR;
  const int u = (int)(g % LPR);
  float acc = 0.f;
  if (r < rows) {
    const int64_t bh = r / a.N, i = r - bh * a.N;
    const int64_t off = (bh * a.sb + i * a.sn) * (int64_t)sizeof(T) + 16 * u;
    typedef T t8 __attribute__((ext_vector_type(8)));
    const f32x8 x = __builtin_convertvector(*reinterpret_cast<const t8*>(a.o + off), f32x8);
    const f32x8 y = __builtin_convertvector(*reinterpret_cast<const t8*>(a.dout + off), f32x8);
#pragma unroll
    for (int e = 0; e < 8; ++e) acc = __builtin_fmaf(x[e], y[e], acc);
  }
#pragma unroll
  for (int o = LPR / 2; o >= 1; o >>= 1) acc += __shfl_xor(acc, o);
  if (r < rows && u == 0) {
    const int64_t bh = r / a.N, i = r - bh * a.N;
    a.dvec[bh * a.lse_sb + i] = acc;
  }
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
      store_grad4<T>(dkrow + d0 * ESZ, xk, a.accumulate);
      store_grad4<T>(dvrow + d0 * ESZ, xv, a.accumulate);
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
      store_grad4<T>(dqrow + d0 * ESZ, x, a.accumulate);
    }
  }
}

// ---------------------------------------------------------------------------------
// D = 128 (f16 / bf16): the same two products per tile, with the staged tiles brought
// into LDS by LDS DMA (no staging registers, no LDS stores), two stages deep: the next
// listed tile moves while the current one is consumed, behind one wait and one barrier
// per tile.  A DMA instruction writes 64 consecutive 16-byte units, so the rows are
// stored unpadded (256 B) and one XOR swizzle of the 16-byte units serves both ways a
// tile is read: unit u of row r sits at u ^ bswz(r), bswz(r) = 4 (r % 4) + (r / 4) % 4.
// The 16 rows of a 16-byte row read land on 16 different units of the 256-byte bank
// window, and the 4 rows of a transposed read on 4 different 64-byte groups.
// LDS: two stages of two tiles, then per stage 2 KB of row vectors (lse, rowsum(dO O),
// original row numbers; the partial tile's bitmap at +1 KB), then the mask terms.
constexpr int kTB = kBT * 256;
constexpr int kStage = 2 * kTB;
constexpr int kVecOff = 2 * kStage;
constexpr int kVec = 2048;
constexpr int kBitsAt = 1024;
constexpr int kTermsOff = kVecOff + 2 * kVec;
constexpr int kBwdSmem = kTermsOff + PA_MAX_TERMS * (int)sizeof(pa_term);

typedef const __attribute__((address_space(3))) f32x4 lds_f4;
typedef const __attribute__((address_space(3))) int32_t lds_i32;
typedef const __attribute__((address_space(3))) u32x2 lds_u2;
typedef const __attribute__((address_space(4))) int32_t cint;
typedef const __attribute__((address_space(4))) int8_t cbyte;

__device__ __forceinline__ int bswz(int r) { return 4 * (r & 3) + ((r >> 2) & 3); }

// Live bits of a score block's 16 elements (element i = row or column 8 (i / 4) + 4 G +
// i % 4 of the 32 the bitmap word covers).
__device__ __forceinline__ uint32_t live16(uint32_t word, int G) {
  const uint32_t x = word >> (4 * G);
  return (x & 0xfu) | ((x >> 4) & 0xf0u) | ((x >> 8) & 0xf00u) | ((x >> 12) & 0xf000u);
}

// Per-lane LDS geometry of a staged tile (offsets of stage, tile, block and chunk are
// immediates on top of these).
struct TileReads {
  lds_cptr row[8];     // 16-byte row reads: row m, unit 2 kc + G
  lds_cptr tr[4][2];   // transposed reads of block db: rows 4 G + j16 / 4 (+8)
};

__device__ __forceinline__ TileReads tile_reads(lds_cptr lds, int lane) {
  TileReads t;
  const int m = lane & 31, G = lane >> 5, j16 = lane & 15, h16 = (lane >> 4) & 1;
#pragma unroll
  for (int kc = 0; kc < 8; ++kc) {
    t.row[kc] = lds + m * 256 + 16 * ((2 * kc + G) ^ bswz(m));
    // (opaque, so each address stays whole in one register)
    asm volatile("" : "+v"(t.row[kc]));
  }
#pragma unroll
  for (int db = 0; db < 4; ++db)
#pragma unroll
    for (int s = 0; s < 2; ++s) {
      const int R = 4 * G + (j16 >> 2) + 8 * s;
      const int u = 4 * db + 2 * h16 + ((j16 & 3) >> 1);
      t.tr[db][s] = lds + R * 256 + 16 * (u ^ bswz(R)) + 8 * (j16 & 1);
      asm volatile("" : "+v"(t.tr[db][s]));
    }
  return t;
}

// A operand X^T of rows r0 .. r0 + 15 (r0 a multiple of 16) of a staged tile at byte
// offset `off` (stage + tile + r0 * 256): the transposed product's fragment for block db.
template <typename T>
__device__ __forceinline__ typename Mma<T>::frag tr_frag_sw(const TileReads& t, int db, int off) {
  const s16x4 x1 = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(t.tr[db][0] + off));
  const s16x4 x2 = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(t.tr[db][1] + off));
  const uint4 vx = {__builtin_bit_cast(uint2, x1).x, __builtin_bit_cast(uint2, x1).y, __builtin_bit_cast(uint2, x2).x,
                    __builtin_bit_cast(uint2, x2).y};
  return __builtin_bit_cast(typename Mma<T>::frag, vx);
}

// DMA of the 64 rows of a tile of two [N, 128] tensors (heads applied; the tile's first
// row at byte r0b, its rows `pitch` bytes apart: the row pitch, or s times it when the
// tile is gathered through the residue-s basis) into stage tiles at LDS m0 and m0 + kTB,
// in four parts (instructions 2 part, 2 part + 1 of each tensor: with 4 waves each moves
// two parts).  Wave w moves rows 32 w .. 32 w + 31; its instruction i writes rows
// 32 w + 4 i + l / 16, lane l unit l % 16, fetching the unit the swizzle stores there:
// (l % 16) ^ (4 (l / 16) + i % 4) (dvoff[i % 4]).
__device__ __forceinline__ void dma_tile_part(uint32_t m0, const char* g0, const char* g1, int64_t pitch, int64_t r0b,
                                              int w, const uint32_t* dvoff, int part) {
  const char* a0 = g0 + r0b + 32 * w * pitch;
  const char* a1 = g1 + r0b + 32 * w * pitch;
  const uint32_t mw = m0 + (uint32_t)(32 * w * 256);
#pragma unroll
  for (int ii = 0; ii < 2; ++ii) {
    const int i = 2 * part + ii;
    dma_x4(mw + i * 1024, a0 + 4 * i * pitch, dvoff[i & 3]);
    dma_x4(mw + kTB + i * 1024, a1 + 4 * i * pitch, dvoff[i & 3]);
  }
}

// ---------------------------------------------------------------------------------
// dK / dV (D = 128) with a key group's two products split over a pair of waves, so that
// a wave holds half the state (one of K / V, one of dK / dV: about 200 registers) and
// two waves share each SIMD.  Work-group: 4 waves, 64 keys; pair p owns keys
// 32 p .. 32 p + 31.  Per tile (one listed query block, staged as in the kernels above):
//   role 0: S = Q K^T, P = exp(scale S - lse) (masked), P to LDS; dV^T += dO^T P;
//   role 1: dP = dO V^T; with P from LDS, dS = P (dP - rowsum(dO O)); dK^T += Q^T dS.
// P goes through LDS in the MFMA operand layout (both roles map key m to lane m), as
// 2-byte values: dS is formed from the rounded P that the MFMAs also use.
constexpr int kPairP = kVecOff + 2 * kVec;          // P of both pairs: 2 x 4 KB
constexpr int kPairTerms = kPairP + 2 * 4096;
constexpr int kPairSmem = kPairTerms + PA_MAX_TERMS * (int)sizeof(pa_term);

template <typename T>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2, 2))) void bwd_dkdv_pair_kernel(const BwdK a) {
  using Frag = typename Mma<T>::frag;
  constexpr int ESZ = 2, NKC = 8, NDB = 4;
  extern __shared__ __attribute__((aligned(16))) char smem[];
  const uint32_t lds0 = (uint32_t)(uintptr_t)(lds_char_t*)smem;
  lds_cptr lds = (lds_cptr)smem;
  pa_term* terms_s = reinterpret_cast<pa_term*>(smem + kPairTerms);
#pragma unroll
  for (int i = 0; i < PA_MAX_TERMS; ++i)  // (constant indices into the argument block)
    if (threadIdx.x == i) terms_s[i] = a.pred.terms[i];

  const int tid = threadIdx.x, lane = tid & 63, G = lane >> 5, m = lane & 31;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int pair = w >> 1, role = w & 1;
  const int64_t id = xcd_remap(blockIdx.x, (int64_t)gridDim.x);
  const int kr = (int)(id % a.nb);
  const int kb = a.kv_order ? ((cint*)a.kv_order)[kr] : kr;
  const int64_t bh = id / a.nb;
  const int key = kb * kBT + pair * 32 + m;
  const int key_o = orig_of(a.pred.perm_kv, key);
  const int64_t key_m = mem_row(a, key);
  const int64_t rowb = a.sn * ESZ;
  const int rs = a.residue_s ? a.residue_s : 1;
  const int64_t pitch = rs * rowb;
  const char* hq = a.q + bh * a.sb * ESZ;
  const char* hdo = a.dout + bh * a.sb * ESZ;
  const char* hlse = reinterpret_cast<const char*>(a.lse + bh * a.lse_sb);
  const char* hdvec = reinterpret_cast<const char*>(a.dvec + bh * a.lse_sb);
  const char* hperm = reinterpret_cast<const char*>(a.pred.perm_q);
  const bool use_bits = a.q_bits != nullptr;

  uint32_t dvoff[4];
#pragma unroll
  for (int j = 0; j < 4; ++j)
    dvoff[j] = (uint32_t)((lane >> 4) * pitch) + 16u * (uint32_t)((lane & 15) ^ (4 * (lane >> 4) + j));
  // query block qb into stage S: wave w moves rows 16 w .. 16 w + 15 of Q and dO; lse
  // (and, without bitmaps, the original row numbers) by wave 0, rowsum(dO O) by wave 1,
  // a partial tile's bitmap (bo >= 0) columns 32 (w - 2) .. +31 by waves 2 and 3
  auto dma = [&](int qb, int bo, int S) __attribute__((always_inline)) {
    const int64_t r0 = mem_row(a, qb * kBT);
    dma_tile_part(lds0 + S * kStage, hq, hdo, pitch, r0 * rowb, pair, dvoff, 2 * role);
    dma_tile_part(lds0 + S * kStage, hq, hdo, pitch, r0 * rowb, pair, dvoff, 2 * role + 1);
    const uint32_t mv = lds0 + kVecOff + S * kVec;
    if (w == 0) {
      dma_x1(mv, hlse + r0 * 4, 4u * rs * lane);
      if (hperm && !use_bits) dma_x1(mv + 512, hperm + (int64_t)qb * 256, 4u * lane);
    } else if (w == 1) {
      dma_x1(mv + 256, hdvec + r0 * 4, 4u * rs * lane);
    } else if (use_bits && bo >= 0) {
      dma_x1(mv + kBitsAt + 256 * (w - 2), reinterpret_cast<const char*>(a.q_bits + bo) + 256 * (w - 2), 4u * lane);
    }
  };

  const TileReads rd = tile_reads(lds, lane);
  lds_cptr vrow = lds + kVecOff + 16 * G;  // row vector entries 8 j + 4 G + 0..3 (+ 32 lb)
  char* pbuf = smem + kPairP + pair * 4096 + lane * 16;  // this lane's P fragments (+ 1 KB per (lb, c))

  // role 0 keeps K and dV, role 1 V and dK
  Frag kv[NKC];
  row_frags<T, 128>((role == 0 ? a.k : a.v) + (bh * a.sb + key_m * a.sn) * ESZ + 16 * G, kv);
  f32x16 acc[NDB];
#pragma unroll
  for (int i = 0; i < NDB; ++i) acc[i] = f32x16{0};

  // this lane's 16 x 2 score elements: element i of block lb is query row
  // 32 lb + 8 (i / 4) + 4 G + i % 4, key `key`
  auto scores = [&](int SO, int tile_off, f32x16* s) __attribute__((always_inline)) {
#pragma unroll
    for (int lb = 0; lb < 2; ++lb) {
      u32x4 xa[NKC];
#pragma unroll
      for (int kc = 0; kc < NKC; ++kc) xa[kc] = *(lds_u4*)(rd.row[kc] + SO + tile_off + lb * 8192);
      s[lb] = Mma<T>::mma(__builtin_bit_cast(Frag, xa[0]), kv[0], f32x16{0});
#pragma unroll
      for (int kc = 1; kc < NKC; ++kc) s[lb] = Mma<T>::mma(__builtin_bit_cast(Frag, xa[kc]), kv[kc], s[lb]);
    }
  };
  // acc^T += X^T Y for the tile at tile_off (dO for dV, Q for dK), Y = the 4 fragments
  auto accum = [&](int SO, int tile_off, const Frag* y) __attribute__((always_inline)) {
#pragma unroll
    for (int lb = 0; lb < 2; ++lb) {
      Frag fx[8];
#pragma unroll
      for (int c = 0; c < 2; ++c)
#pragma unroll
        for (int db = 0; db < NDB; ++db) fx[4 * c + db] = tr_frag_sw<T>(rd, db, SO + tile_off + (32 * lb + 16 * c) * 256);
#pragma unroll
      for (int c = 0; c < 2; ++c)
#pragma unroll
        for (int db = 0; db < NDB; ++db) acc[db] = Mma<T>::mma(fx[4 * c + db], y[2 * lb + c], acc[db]);
    }
  };

  auto tile = [&](auto SC, bool partial, int qb) __attribute__((always_inline)) {
    constexpr int S = decltype(SC)::value;
    constexpr int SO = S * kStage;
    if (role == 0) {
      uint32_t live[2] = {0xffffu, 0xffffu};
      if (partial && use_bits) {
        const u32x2 bw = *(lds_u2*)(lds + kVecOff + S * kVec + kBitsAt + (32 * pair + m) * 8);
        const uint32_t b0 = bw.x, b1 = bw.y;
        live[0] = live16(b0, G);
        live[1] = live16(b1, G);
      } else if (partial) {
        lds_i32* qo = (lds_i32*)(lds + kVecOff + S * kVec + 512);
#pragma unroll
        for (int lb = 0; lb < 2; ++lb) {
          live[lb] = 0u;
#pragma unroll 1
          for (int i = 0; i < 16; ++i) {
            const int qr = 32 * lb + 8 * (i >> 2) + 4 * G + (i & 3);
            const int q_o = hperm ? qo[qr] : qb * kBT + qr;
            if (pred_live_rolled(terms_s, a.pred.n_include, a.pred.n_exclude, q_o, key_o, a.pred.dense_bits,
                                 a.pred.dense_words))
              live[lb] |= 1u << i;
          }
        }
      }
      f32x4 l4[2][4];
#pragma unroll
      for (int lb = 0; lb < 2; ++lb)
#pragma unroll
        for (int j = 0; j < 4; ++j) l4[lb][j] = *(lds_f4*)(vrow + S * kVec + (32 * lb + 8 * j) * 4);
      f32x16 s[2];
      scores(SO, 0, s);
      Frag pf[4];
#pragma unroll
      for (int lb = 0; lb < 2; ++lb)
#pragma unroll
        for (int c = 0; c < 2; ++c) {
          f32x8 pv;
#pragma unroll
          for (int e = 0; e < 8; ++e) {
            const int i = 8 * c + e;
            const float lse = l4[lb][i >> 2][i & 3];
            const float pe = __builtin_amdgcn_exp2f(__builtin_fmaf(s[lb][i], a.c, -lse * 1.4426950408889634f));
            pv[e] = (((live[lb] >> i) & 1u) && lse != -INFINITY) ? pe : 0.f;
          }
          pf[2 * lb + c] = Mma<T>::cvt(pv);
          *reinterpret_cast<__attribute__((address_space(3))) u32x4*>((lds_char_t*)pbuf + (2 * lb + c) * 1024) =
              __builtin_bit_cast(u32x4, pf[2 * lb + c]);
        }
      __syncthreads();  // P is in LDS
      accum(SO, kTB, pf);  // dV^T += dO^T P
    } else {
      f32x4 d4[2][4];
#pragma unroll
      for (int lb = 0; lb < 2; ++lb)
#pragma unroll
        for (int j = 0; j < 4; ++j) d4[lb][j] = *(lds_f4*)(vrow + S * kVec + 256 + (32 * lb + 8 * j) * 4);
      f32x16 dp[2];
      scores(SO, kTB, dp);
      __syncthreads();  // P is in LDS
      Frag sf[4];
#pragma unroll
      for (int lb = 0; lb < 2; ++lb)
#pragma unroll
        for (int c = 0; c < 2; ++c) {
          const Frag pf = __builtin_bit_cast(Frag, *(lds_u4*)(lds + kPairP + pair * 4096 + lane * 16 + (2 * lb + c) * 1024));
          const f32x8 pfl = __builtin_convertvector(pf, f32x8);
          f32x8 sv;
#pragma unroll
          for (int e = 0; e < 8; ++e) {
            const int i = 8 * c + e;
            sv[e] = pfl[e] * (dp[lb][i] - d4[lb][i >> 2][i & 3]);
          }
          sf[2 * lb + c] = Mma<T>::cvt(sv);
        }
      accum(SO, 0, sf);  // dK^T += Q^T dS
    }
  };

  const int nl = ((cint*)a.q_num)[kb];
  cint* qlist = (cint*)(a.q_idx + (int64_t)kb * a.tpitch);
  cbyte* plist = (cbyte*)(a.q_partial + (int64_t)kb * a.tpitch);
  cint* olist = (cint*)(use_bits ? a.q_bits_off + (int64_t)kb * a.tpitch : a.q_idx);
  auto tile_of = [&](int t, int& qb, int& bo) __attribute__((always_inline)) {
    qb = qlist[t];
    bo = use_bits ? olist[t] : (plist[t] != 0 ? 0 : -1);
  };
  int qb_c = 0, bo_c = -1, qb_n = 0, bo_n = -1;
  if (nl > 0) {
    tile_of(0, qb_c, bo_c);
    dma(qb_c, bo_c, 0);
  }
  if (nl > 1) tile_of(1, qb_n, bo_n);
  auto step = [&](auto SC, int t) __attribute__((always_inline)) {
    constexpr int S = decltype(SC)::value;
    dma_wait_all();
    __syncthreads();  // stage S is in; every wave is past stage S ^ 1 and the last P
    if (t + 1 < nl) dma(qb_n, bo_n, S ^ 1);
    const int qb = qb_c;
    const bool partial = bo_c >= 0;
    qb_c = qb_n;
    bo_c = bo_n;
    if (t + 2 < nl) tile_of(t + 2, qb_n, bo_n);
    tile(SC, partial, qb);
  };
  int t = 0;
  for (; t + 1 < nl; t += 2) {
    step(std::integral_constant<int, 0>{}, t);
    step(std::integral_constant<int, 1>{}, t + 1);
  }
  if (t < nl) step(std::integral_constant<int, 0>{}, t);

  // role 0: dV^T, role 1: dK^T blocks [32 d x 32 keys]: lane (key m, G) holds
  // d = 32 db + 8 i4 + 4 G + 0..3
  char* grow = (role == 0 ? a.dv : a.dk) + (bh * a.sb + key_m * a.sn) * ESZ;
  const float gs = role == 0 ? 1.f : a.scale;
#pragma unroll
  for (int db = 0; db < NDB; ++db) {
#pragma unroll
    for (int i4 = 0; i4 < 4; ++i4) {
      const int d0 = 32 * db + 8 * i4 + 4 * G;
      f32x4 x = {acc[db][4 * i4], acc[db][4 * i4 + 1], acc[db][4 * i4 + 2], acc[db][4 * i4 + 3]};
      x *= gs;
      store_grad4<T>(grow + d0 * ESZ, x, a.accumulate);
    }
  }
}

template <typename T>
__global__ __launch_bounds__(128) __attribute__((amdgpu_waves_per_eu(1, 1))) void bwd_dq_stream_kernel(const BwdK a) {
  using Frag = typename Mma<T>::frag;
  constexpr int ESZ = 2, NKC = 8, NDB = 4;
  extern __shared__ __attribute__((aligned(16))) char smem[];
  const uint32_t lds0 = (uint32_t)(uintptr_t)(lds_char_t*)smem;
  lds_cptr lds = (lds_cptr)smem;
  pa_term* terms_s = reinterpret_cast<pa_term*>(smem + kTermsOff);
#pragma unroll
  for (int i = 0; i < PA_MAX_TERMS; ++i)
    if (threadIdx.x == i) terms_s[i] = a.pred.terms[i];

  const int tid = threadIdx.x, lane = tid & 63, G = lane >> 5, m = lane & 31;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int64_t id = xcd_remap(blockIdx.x, (int64_t)gridDim.x);
  const int qb = (int)(id % a.nb);
  const int64_t bh = id / a.nb;
  const int row = qb * kBT + w * 32 + m;  // this lane's query row (index space)
  const int q_o = orig_of(a.pred.perm_q, row);
  const int64_t row_m = mem_row(a, row);
  const int64_t rowb = a.sn * ESZ;
  const int rs = a.residue_s ? a.residue_s : 1;
  const int64_t pitch = rs * rowb;
  const char* hk = a.k + bh * a.sb * ESZ;
  const char* hv = a.v + bh * a.sb * ESZ;
  const char* hperm = reinterpret_cast<const char*>(a.pred.perm_kv);

  uint32_t dvoff[4];
#pragma unroll
  for (int j = 0; j < 4; ++j)
    dvoff[j] = (uint32_t)((lane >> 4) * pitch) + 16u * (uint32_t)((lane & 15) ^ (4 * (lane >> 4) + j));
  const bool use_bits = a.kv_bits != nullptr;
  // key block kb into stage S: K and V tiles; without bitmaps the original key numbers by
  // wave 0; a partial tile's bitmap (bo >= 0), rows 32 w .. 32 w + 31 by wave w
  auto dma = [&](int kb, int bo, int S, int part) __attribute__((always_inline)) {
    dma_tile_part(lds0 + S * kStage, hk, hv, pitch, mem_row(a, kb * kBT) * rowb, w, dvoff, part);
    if (part) return;
    const uint32_t mv = lds0 + kVecOff + S * kVec;
    if (hperm && !use_bits && w == 0) dma_x1(mv + 512, hperm + (int64_t)kb * 256, 4u * lane);
    if (use_bits && bo >= 0)
      dma_x1(mv + kBitsAt + 256 * w, reinterpret_cast<const char*>(a.kv_bits + bo) + 256 * w, 4u * lane);
  };

  const TileReads rd = tile_reads(lds, lane);

  Frag qf[NKC], df[NKC];
  row_frags<T, 128>(a.q + (bh * a.sb + row_m * a.sn) * ESZ + 16 * G, qf);
  row_frags<T, 128>(a.dout + (bh * a.sb + row_m * a.sn) * ESZ + 16 * G, df);
  const float lse = a.lse[bh * a.lse_sb + row_m];
  const float nl2 = -lse * 1.4426950408889634f;
  const bool dead = lse == -INFINITY;
  const float dr = a.dvec[bh * a.lse_sb + row_m];
  f32x16 dqt[NDB];
#pragma unroll
  for (int i = 0; i < NDB; ++i) dqt[i] = f32x16{0};

  // One tile (stage S), phases as in the dK/dV kernel: A scores of keys 0..31; B scores of
  // keys 32..63 beside the gradient of keys 0..31; C dQ^T += K^T dS^T of keys 0..31 beside
  // the gradient of 32..63; D dQ^T of keys 32..63.  Element i of a score block is key
  // 32 lb + 8 (i / 4) + 4 G + i % 4, query `row`.
  auto compute = [&](auto SC, bool partial, int kb, auto&& pre) __attribute__((always_inline)) {
    constexpr int S = decltype(SC)::value;
    constexpr int SO = S * kStage;
    uint32_t live[2] = {dead ? 0u : 0xffffu, dead ? 0u : 0xffffu};
    if (partial && !dead && use_bits) {
      // this lane's row of the tile: columns 0..31, 32..63
      const u32x2 bw = *(lds_u2*)(lds + kVecOff + S * kVec + kBitsAt + (32 * w + m) * 8);
      const uint32_t b0 = bw.x, b1 = bw.y;
      live[0] = live16(b0, G);
      live[1] = live16(b1, G);
    } else if (partial && !dead) {
      lds_i32* ko = (lds_i32*)(lds + kVecOff + S * kVec + 512);
#pragma unroll
      for (int lb = 0; lb < 2; ++lb) {
        live[lb] = 0u;
#pragma unroll 1
        for (int i = 0; i < 16; ++i) {
          const int kr = 32 * lb + 8 * (i >> 2) + 4 * G + (i & 3);
          const int k_o = hperm ? ko[kr] : kb * kBT + kr;
          if (pred_live_rolled(terms_s, a.pred.n_include, a.pred.n_exclude, q_o, k_o, a.pred.dense_bits,
                               a.pred.dense_words))
            live[lb] |= 1u << i;
        }
      }
    }
    auto scores = [&](int lb, f32x16& s, f32x16& dp) __attribute__((always_inline)) {
      u32x4 ka[NKC], va[NKC];
#pragma unroll
      for (int kc = 0; kc < NKC; ++kc) {
        ka[kc] = *(lds_u4*)(rd.row[kc] + SO + lb * 8192);
        va[kc] = *(lds_u4*)(rd.row[kc] + SO + kTB + lb * 8192);
      }
      s = Mma<T>::mma(__builtin_bit_cast(Frag, ka[0]), qf[0], f32x16{0});
      dp = Mma<T>::mma(__builtin_bit_cast(Frag, va[0]), df[0], f32x16{0});
#pragma unroll
      for (int kc = 1; kc < NKC; ++kc) {
        s = Mma<T>::mma(__builtin_bit_cast(Frag, ka[kc]), qf[kc], s);
        dp = Mma<T>::mma(__builtin_bit_cast(Frag, va[kc]), df[kc], dp);
      }
    };
    auto grads = [&](int lb, const f32x16& s, const f32x16& dp, Frag* sf) __attribute__((always_inline)) {
#pragma unroll
      for (int c = 0; c < 2; ++c) {
        f32x8 sv;
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const int i = 8 * c + e;
          const float pe = __builtin_amdgcn_exp2f(__builtin_fmaf(s[i], a.c, nl2));
          const float p = ((live[lb] >> i) & 1u) ? pe : 0.f;
          sv[e] = p * (dp[i] - dr);
        }
        sf[c] = Mma<T>::cvt(sv);
      }
    };
    // dQ^T += K^T dS^T for keys 32 lb .. +31: the transposed K fragments (chunk c, block db
    // at 4 c + db) are read first, into registers
    auto tr_reads = [&](int lb, Frag* fk) __attribute__((always_inline)) {
#pragma unroll
      for (int c = 0; c < 2; ++c) {
        const int off = SO + (32 * lb + 16 * c) * 256;
#pragma unroll
        for (int db = 0; db < NDB; ++db) fk[4 * c + db] = tr_frag_sw<T>(rd, db, off);
      }
    };
    auto accum = [&](const Frag* fk, const Frag* sf) __attribute__((always_inline)) {
#pragma unroll
      for (int c = 0; c < 2; ++c)
#pragma unroll
        for (int db = 0; db < NDB; ++db) dqt[db] = Mma<T>::mma(fk[4 * c + db], sf[c], dqt[db]);
    };
    f32x16 s0, dp0, s1, dp1;
    Frag sf0[2], sf1[2], fk[8];
    pre(0);
    pre(1);
    pre(2);
    pre(3);
    scores(0, s0, dp0);
    __builtin_amdgcn_sched_group_barrier(0x100, 4, 0);
#pragma unroll
    for (int q_ = 0; q_ < 12; ++q_) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
      __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
    }
    __builtin_amdgcn_sched_group_barrier(0x008, 4, 0);
    __builtin_amdgcn_sched_barrier(0);
    scores(1, s1, dp1);
    grads(0, s0, dp0, sf0);
    __builtin_amdgcn_sched_group_barrier(0x100, 4, 0);
#pragma unroll
    for (int q_ = 0; q_ < 12; ++q_) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
      __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
      __builtin_amdgcn_sched_group_barrier(0x002, 6, 0);
    }
#pragma unroll
    for (int q_ = 0; q_ < 4; ++q_) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
      __builtin_amdgcn_sched_group_barrier(0x002, 6, 0);
    }
    __builtin_amdgcn_sched_barrier(0);
    tr_reads(0, fk);
    grads(1, s1, dp1, sf1);
    accum(fk, sf0);
    __builtin_amdgcn_sched_group_barrier(0x100, 16, 0);
#pragma unroll
    for (int q_ = 0; q_ < 8; ++q_) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
      __builtin_amdgcn_sched_group_barrier(0x002, 12, 0);
    }
    __builtin_amdgcn_sched_barrier(0);
    tr_reads(1, fk);
    accum(fk, sf1);
    __builtin_amdgcn_sched_group_barrier(0x100, 16, 0);
    __builtin_amdgcn_sched_group_barrier(0x008, 8, 0);
  };

  const int nl = ((cint*)a.kv_num)[qb];
  cint* klist = (cint*)(a.kv_idx + (int64_t)qb * a.pitch);
  cbyte* plist = (cbyte*)(a.kv_partial + (int64_t)qb * a.pitch);
  cint* olist = (cint*)(use_bits ? a.kv_bits_off + (int64_t)qb * a.pitch : a.kv_idx);
  auto tile_of = [&](int t, int& kb, int& bo) __attribute__((always_inline)) {
    kb = klist[t];
    bo = use_bits ? olist[t] : (plist[t] != 0 ? 0 : -1);
  };
  int kb_c = 0, bo_c = -1, kb_n = 0, bo_n = -1;
  if (nl > 0) {
    tile_of(0, kb_c, bo_c);
#pragma unroll
    for (int part = 0; part < 4; ++part) dma(kb_c, bo_c, 0, part);
  }
  if (nl > 1) tile_of(1, kb_n, bo_n);
  auto step = [&](auto SC, int t) __attribute__((always_inline)) {
    constexpr int S = decltype(SC)::value;
    dma_wait_all();
    __syncthreads();
    const bool more = t + 1 < nl;
    const int kb = kb_c, kb_d = kb_n, bo_d = bo_n;
    const bool partial = bo_c >= 0;
    kb_c = kb_n;
    bo_c = bo_n;
    if (t + 2 < nl) tile_of(t + 2, kb_n, bo_n);
    compute(SC, partial, kb, [&](int part) __attribute__((always_inline)) {
      if (more) dma(kb_d, bo_d, S ^ 1, part);
    });
  };
  int t = 0;
  for (; t + 1 < nl; t += 2) {
    step(std::integral_constant<int, 0>{}, t);
    step(std::integral_constant<int, 1>{}, t + 1);
  }
  if (t < nl) step(std::integral_constant<int, 0>{}, t);

  char* dqrow = a.dq + (bh * a.sb + row_m * a.sn) * ESZ;
#pragma unroll
  for (int db = 0; db < NDB; ++db) {
#pragma unroll
    for (int i4 = 0; i4 < 4; ++i4) {
      const int d0 = 32 * db + 8 * i4 + 4 * G;
      f32x4 x = {dqt[db][4 * i4], dqt[db][4 * i4 + 1], dqt[db][4 * i4 + 2], dqt[db][4 * i4 + 3]};
      x *= a.scale;
      store_grad4<T>(dqrow + d0 * ESZ, x, a.accumulate);
    }
  }
}

// Transposed block lists: for key block kb, the query blocks whose list holds kb, in
// ascending order, with the partial flag.  One thread per key block; each query block's
// list is sorted, so membership is a binary search.  q_idx == nullptr: counts only.
__global__ __launch_bounds__(256) void transpose_kernel(const int32_t* kv_idx, const int32_t* kv_num,
                                                        const int8_t* kv_partial, const int32_t* kv_bits_off,
                                                        int32_t nq, int64_t pitch, int32_t nk, int32_t* q_num,
                                                        int32_t* q_idx, int8_t* q_partial, int32_t* q_bits_off,
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
        if (q_bits_off) q_bits_off[(int64_t)kb * tp + n] = kv_bits_off[(int64_t)qb * pitch + lo];
      }
      ++n;
    }
  }
  q_num[kb] = n;
}

// One 64 x 64 bitmap per work-group of 64 threads (listed tile j of query block i, when
// kv_bits_off[i, j] >= 0): thread k assembles column k from the 64 row words.
__global__ __launch_bounds__(64) void bits_transpose_kernel(const int32_t* kv_bits_off, int64_t pitch,
                                                             const uint32_t* kv_bits, uint32_t* q_bits) {
  const int64_t off = kv_bits_off[(int64_t)blockIdx.y * pitch + blockIdx.x];
  if (off < 0) return;
  const int k = threadIdx.x;
  uint32_t col[2] = {0u, 0u};
#pragma unroll 8
  for (int r = 0; r < 64; ++r) col[r >> 5] |= ((kv_bits[off + 2 * r + (k >> 5)] >> (k & 31)) & 1u) << (r & 31);
  q_bits[off + 2 * k] = col[0];
  q_bits[off + 2 * k + 1] = col[1];
}

template <typename T, int D>
int launch_bwd(const BwdK& k, int64_t BH, bool dvec_given, hipStream_t s) {
  const int64_t rows = BH * k.N;
  if (!dvec_given) {
    hipLaunchKernelGGL((bwd_pre_kernel<T, D>), dim3((unsigned)((rows * (D / 8) + 255) / 256)), dim3(256), 0, s, k,
                       rows);
    PA_LAUNCH_CHECK("bwd_pre_kernel");
  }
  if constexpr (D == 128) {
    // the dynamic LDS limit is raised once per device
    static unsigned long long configured = 0ull;
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return hip_fail(e, "hipGetDevice");
    if (dev >= 64 || !((configured >> dev) & 1ull)) {
      e = hipFuncSetAttribute(reinterpret_cast<const void*>(&bwd_dkdv_pair_kernel<T>),
                              hipFuncAttributeMaxDynamicSharedMemorySize, kPairSmem);
      if (e == hipSuccess)
        e = hipFuncSetAttribute(reinterpret_cast<const void*>(&bwd_dq_stream_kernel<T>),
                                hipFuncAttributeMaxDynamicSharedMemorySize, kBwdSmem);
      if (e != hipSuccess) return hip_fail(e, "hipFuncSetAttribute(bwd stream kernels)");
      if (dev < 64) configured |= 1ull << dev;
    }
    const unsigned grid = (unsigned)(k.nb * BH);
    hipLaunchKernelGGL(bwd_dkdv_pair_kernel<T>, dim3(grid), dim3(256), kPairSmem, s, k);
    PA_LAUNCH_CHECK("bwd_dkdv_pair_kernel");
    hipLaunchKernelGGL(bwd_dq_stream_kernel<T>, dim3(grid), dim3(128), kBwdSmem, s, k);
    PA_LAUNCH_CHECK("bwd_dq_stream_kernel");
  } else {
    hipLaunchKernelGGL((bwd_dkdv_kernel<T, D>), dim3((unsigned)k.nb, (unsigned)BH), dim3(128), 0, s, k);
    PA_LAUNCH_CHECK("bwd_dkdv_kernel");
    hipLaunchKernelGGL((bwd_dq_kernel<T, D>), dim3((unsigned)k.nb, (unsigned)BH), dim3(128), 0, s, k);
    PA_LAUNCH_CHECK("bwd_dq_kernel");
  }
  return PA_OK;
}

}  // namespace
}  // namespace pa

extern "C" int pa_index_transpose(const int32_t* kv_idx, const int32_t* kv_num, const int8_t* kv_partial,
                                  const int32_t* kv_bits_off, int32_t nq, int64_t pitch, int32_t nk, int32_t* q_num,
                                  int32_t* q_idx, int8_t* q_partial, int32_t* q_bits_off, int64_t tpitch,
                                  void* stream) {
  PA_CHECK_ARG(kv_num && q_num && nq >= 1 && nk >= 1 && pitch >= 0 && tpitch >= 0, "pa_index_transpose: bad arguments");
  PA_CHECK_ARG(pitch == 0 || (kv_idx && kv_partial), "pa_index_transpose: null kv_idx / kv_partial");
  PA_CHECK_ARG(!q_idx || q_partial, "pa_index_transpose: q_idx needs q_partial");
  PA_CHECK_ARG(!q_bits_off || (kv_bits_off && q_idx), "pa_index_transpose: q_bits_off needs kv_bits_off and q_idx");
  hipStream_t s = static_cast<hipStream_t>(stream);
  hipLaunchKernelGGL(pa::transpose_kernel, dim3((unsigned)((nk + 255) / 256)), dim3(256), 0, s, kv_idx, kv_num,
                     kv_partial, kv_bits_off, nq, pitch, nk, q_num, q_idx, q_partial, q_bits_off, tpitch);
  PA_LAUNCH_CHECK("transpose_kernel");
  return PA_OK;
}

extern "C" int pa_index_bits_transpose(const int32_t* kv_bits_off, int32_t nq, int64_t pitch, const uint32_t* kv_bits,
                                       uint32_t* q_bits, void* stream) {
  PA_CHECK_ARG(nq >= 1 && nq <= 65535 && pitch >= 0 && pitch < (1ll << 31), "pa_index_bits_transpose: nq=%d pitch=%lld",
               nq, (long long)pitch);
  if (pitch == 0) return PA_OK;
  PA_CHECK_ARG(kv_bits_off && kv_bits && q_bits, "pa_index_bits_transpose: null array");
  hipStream_t s = static_cast<hipStream_t>(stream);
  hipLaunchKernelGGL(pa::bits_transpose_kernel, dim3((unsigned)pitch, (unsigned)nq), dim3(64), 0, s, kv_bits_off,
                     pitch, kv_bits, q_bits);
  PA_LAUNCH_CHECK("bits_transpose_kernel");
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
  PA_CHECK_ARG(x->lse_sb >= x->N, "pa_attn_bwd: lse_sb=%lld < N=%lld (lse and dvec rows must not overlap)",
               (long long)x->lse_sb, (long long)x->N);
  PA_CHECK_ARG(x->sn >= x->D && x->sb >= x->sn && x->sn < (1ll << 28), "pa_attn_bwd: strides sb=%lld sn=%lld",
               (long long)x->sb, (long long)x->sn);
  PA_CHECK_ARG((x->N / 64) * x->BH < (1ll << 31), "pa_attn_bwd: %lld blocks x %lld heads exceed one launch",
               (long long)(x->N / 64), (long long)x->BH);
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
  k.lse_sb = x->lse_sb;
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
  const bool nb_ = !x->kv_bits_off, nk_ = !x->kv_bits, qo_ = !x->q_bits_off, qk_ = !x->q_bits;
  PA_CHECK_ARG(nb_ == nk_ && nb_ == qo_ && nb_ == qk_, "pa_attn_bwd: the four bitmap arrays are all NULL or all given");
  k.kv_bits_off = x->kv_bits_off;
  k.kv_bits = x->kv_bits;
  k.q_bits_off = x->q_bits_off;
  k.q_bits = x->q_bits;
  PA_CHECK_ARG((x->flags & ~(PA_BWD_ACCUMULATE | PA_BWD_DVEC_GIVEN)) == 0, "pa_attn_bwd: unknown flags %d", x->flags);
  k.accumulate = (x->flags & PA_BWD_ACCUMULATE) != 0;
  k.residue_s = 0;
  k.residue_qlog2 = 0;
  k.kv_order = x->kv_order;
  if (x->residue_s > 1) {
    const int64_t per = x->N / x->residue_s;
    PA_CHECK_ARG(x->D == 128 && x->N % x->residue_s == 0 && (per & (per - 1)) == 0 && per % 64 == 0,
                 "pa_attn_bwd: residue_s=%d needs D = 128 and N / s a power of two and a multiple of 64 (N=%lld)",
                 x->residue_s, (long long)x->N);
    PA_CHECK_ARG((int64_t)x->residue_s * x->sn * 2 * 4 < (1ll << 32), "pa_attn_bwd: residue_s=%d rows too far apart",
                 x->residue_s);
    k.residue_s = x->residue_s;
    while ((1ll << k.residue_qlog2) < per) ++k.residue_qlog2;
  }
  const bool dg = (x->flags & PA_BWD_DVEC_GIVEN) != 0;
  k.pred = pa::make_pred(x->mask);
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (x->dtype == PA_BF16)
    return x->D == 128 ? pa::launch_bwd<__bf16, 128>(k, x->BH, dg, s) : pa::launch_bwd<__bf16, 64>(k, x->BH, dg, s);
  return x->D == 128 ? pa::launch_bwd<_Float16, 128>(k, x->BH, dg, s) : pa::launch_bwd<_Float16, 64>(k, x->BH, dg, s);
}
