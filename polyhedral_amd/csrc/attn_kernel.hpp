// Block-sparse masked attention forward for gfx950 (CDNA4).
//
// Replaces the Triton kernel _attn_fwd (gpu/triton_attn.py:62-182).  Same
// contract: one work-group per (query block of BQ rows, batch-head), iterate the
// live KV tiles listed for that block (kv_idx / kv_num), online softmax with the
// finite -1e30 sentinel and the l > 0 guard, output in the input dtype.  The
// MI355X design differs from the reference's in how it gets there:
//
//  * Scores are computed transposed, S^T = K Q^T, on 32x32 MFMAs
//    (32x32x16 bf16/f16, 32x32x2 f32).  In the 32x32 accumulator layout lane l
//    then owns query row l % 32 and 16 of the 32 KV columns, so a row max is 15
//    in-lane max ops plus one exchange with lane l ^ 32, and P^T is already in
//    the register layout the P.V MFMA wants as its B operand: no shuffles.
//  * Each wave owns 32 query rows; a work-group is BQ/32 waves (one wave with 16
//    live rows for BQ = 16).  K and V of 64 KV rows (4 segments of 16 rows, each
//    segment taken from any listed tile) are staged per step into LDS, double
//    buffered, the next step's global loads in flight while this one computes.
//    K rows are stored with a 16-B XOR swizzle; V is stored transposed (V^T) for
//    the bf16/f16 MFMA A operand, in the KV-slot order that matches P^T's.
//  * Everything a step needs to know about its segments (tile row, wave codes,
//    bitmap offset) is read with uniform (scalar) loads two steps ahead, and a
//    residue-class permutation is evaluated in closed form, so no global load
//    depends on another inside the loop.
//  * Per-wave skip: the tile codes (2 bits per 32-row x 32-column wave group)
//    let a wave skip MFMA work on a 32x32 block that is dead for its rows and
//    mask only blocks that are not full for its rows.  Partial segments are
//    masked from element bitmaps staged into LDS with K and V, or, without
//    bitmaps, by evaluating the predicate in a compact loop.
//  * Lazy rescaling: the running max m is raised only when a row's new max
//    exceeds it by more than 8 (log2 units); the result is identical in exact
//    arithmetic and the wave skips the O rescale on most steps.
//  * exp2 with scale*log2(e) folded into one FMA; LSE = (m + log2 l) ln 2.
#pragma once

#include "common.hpp"

namespace pa {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

struct AttnK {
  const char* q;
  const char* k;
  const char* v;
  char* o;
  int64_t q_sb, q_sn, k_sb, k_sn, v_sb, v_sn, o_sb, o_sn;  // element strides
  int32_t N, BQ, A, nq;
  int32_t spt_log2;  // log2(A / 16): 16-row segments per tile
  int64_t total_wg;
  float c;  // scale * log2(e)
  const int32_t* kv_idx;
  const int32_t* kv_num;
  const int8_t* kv_partial;
  const uint32_t* kv_wave_bits;
  int64_t pitch;
  const int32_t* kv_bits_off;
  const uint32_t* kv_bits;
  Pred pred;
  int32_t gather_q, gather_kv, scatter_o;
  int32_t residue_s, residue_qlog2;
  float* lse;
  int64_t lse_sb;
  const char* prev_o;
  int32_t prev_dtype;
  int64_t prev_sb, prev_sn;
  const float* prev_lse;
  const int32_t* qblock_order;
};

constexpr int kStep = 64;          // KV rows per staged step
constexpr float kSentinel = -1e30f;
constexpr float kLazy = 8.0f;      // rescale threshold, log2 units
constexpr float kLn2 = 0.69314718055994530942f;

template <typename T>
struct Mma;

template <>
struct Mma<__bf16> {
  using frag = bf16x8;
  __device__ static f32x16 mma(frag a, frag b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
  }
  __device__ static frag cvt(f32x8 x) { return __builtin_convertvector(x, bf16x8); }
  __device__ static void store4(char* p, f32x4 x) {
    *reinterpret_cast<bf16x4*>(p) = __builtin_convertvector(x, bf16x4);
  }
};

template <>
struct Mma<_Float16> {
  using frag = f16x8;
  __device__ static f32x16 mma(frag a, frag b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
  }
  __device__ static frag cvt(f32x8 x) { return __builtin_convertvector(x, f16x8); }
  __device__ static void store4(char* p, f32x4 x) {
    *reinterpret_cast<f16x4*>(p) = __builtin_convertvector(x, f16x4);
  }
};

template <>
struct Mma<float> {
  using frag = float;
  __device__ static f32x16 mma(float a, float b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x2f32(a, b, c, 0, 0, 0);
  }
  __device__ static void store4(char* p, f32x4 x) { *reinterpret_cast<f32x4*>(p) = x; }
};

// 4 consecutive elements of a partial result in dtype dt, as floats.
__device__ __forceinline__ f32x4 load4_any(const char* p, int32_t dt) {
  if (dt == PA_F32) return *reinterpret_cast<const f32x4*>(p);
  if (dt == PA_F16) return __builtin_convertvector(*reinterpret_cast<const f16x4*>(p), f32x4);
  return __builtin_convertvector(*reinterpret_cast<const bf16x4*>(p), f32x4);
}

__device__ __forceinline__ float other_half(float x) { return __shfl_xor(x, 32, 64); }

// Uniform description of the 4 segments of one step.
struct StepMeta {
  int32_t base[4];   // index-space KV row of the segment's first row; -1 past the list
  uint32_t code[4];  // tile code shifted to the segment's column group (0 past the list)
  int32_t boff[4];   // bitmap word offset of the segment's tile (-1: none)
};

// Two waves per SIMD where the registers allow it (4-wave work-groups, except fp32 with
// D = 128): two work-groups then share a CU, one computing while the other waits on its
// K/V loads.  The 1- and 2-wave shapes (BQ <= 64) stage more rows per thread and keep one.
template <typename T, int D, int NW>
constexpr int occupancy_target() {
  return (NW == 4 && (sizeof(T) == 2 || D == 64)) ? 2 : 1;
}

template <typename T, int D, int NW>
__global__ __launch_bounds__(NW * 64) __attribute__((amdgpu_waves_per_eu(occupancy_target<T, D, NW>())))
void attn_fwd_kernel(const AttnK a) {
  constexpr bool kF32 = sizeof(T) == 4;
  constexpr int ESZ = sizeof(T);
  constexpr int UPR = D * ESZ / 16;                 // 16-B units per row
  constexpr int NT = NW * 64;
  constexpr int K_BYTES = kStep * D * ESZ;          // K tile (and V tile) bytes per buffer
  constexpr int BUF_BYTES = 2 * K_BYTES;
  constexpr int KU = (kStep * UPR + NT - 1) / NT;   // K units per thread
  constexpr int VTASKS = kF32 ? 0 : 16 * UPR;       // V^T tasks (4 rows x 16 B each)
  constexpr int VT = kF32 ? 0 : (VTASKS + NT - 1) / NT;
  constexpr int VU = kF32 ? KU : 1;                 // f32: V staged like K
  constexpr int NDB = D / 32;                       // 32-wide output blocks
  constexpr int ROWS = NW * 32;                     // query rows held by the work-group
  constexpr int BW = (4 * ROWS + NT - 1) / NT;      // bitmap words staged per thread

  extern __shared__ __attribute__((aligned(16))) char smem[];
  __shared__ int32_t kvo_s[2][kStep];
  __shared__ uint32_t bits_s[2][4][ROWS];
  __shared__ pa_term terms_s[PA_MAX_TERMS];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int w = tid >> 6;
  const int G = lane >> 5;  // half-wave
  const int m = lane & 31;  // query row within the wave

  const int64_t lid = xcd_remap(blockIdx.x, a.total_wg);
  const int64_t bh = lid / a.nq;
  const int qb_lin = (int)(lid % a.nq);
  const int qb = a.qblock_order ? a.qblock_order[qb_lin] : qb_lin;

  const int A = a.A;
  const int spt_log2 = a.spt_log2;
  const int spt_mask = (1 << spt_log2) - 1;
  const int ncg = A >= 32 ? (A >> 5) : 1;  // wave column groups per tile
  const int64_t row0 = (int64_t)qb * a.pitch;
  const int n_seg = a.kv_num[qb] << spt_log2;
  const int n_steps = (n_seg + 3) >> 2;
  const bool use_bits = a.kv_bits != nullptr;

  // index-space position -> original position
  const int32_t rmask = (1 << a.residue_qlog2) - 1;
  auto orig_q = [&](int p) -> int {
    if (a.residue_s) return (p & rmask) * a.residue_s + (p >> a.residue_qlog2);
    return a.pred.perm_q ? a.pred.perm_q[p] : p;
  };
  auto orig_kv = [&](int p) -> int {
    if (a.residue_s) return (p & rmask) * a.residue_s + (p >> a.residue_qlog2);
    return a.pred.perm_kv ? a.pred.perm_kv[p] : p;
  };
  const bool has_pq = a.residue_s || a.pred.perm_q;
  const bool gather_kv = a.gather_kv && (a.residue_s || a.pred.perm_kv);

  const int rows_valid = a.BQ < 32 ? a.BQ : 32;
  const bool q_ok = m < rows_valid;
  const int r_idx = qb * a.BQ + w * 32 + m;  // index-space query row of this lane
  int q_orig = 0, r_load = r_idx;
  if (q_ok) {
    q_orig = has_pq ? orig_q(r_idx) : r_idx;
    if (a.gather_q && has_pq) r_load = q_orig;
  }

  // ---- Q fragment (B operand of S^T = K Q^T) -------------------------------
  using QFrag = typename Mma<T>::frag;
  constexpr int NQF = kF32 ? D / 2 : D / 16;
  QFrag qf[NQF];
  {
    const char* qrow = a.q + (bh * a.q_sb + (int64_t)r_load * a.q_sn) * ESZ;
    if constexpr (kF32) {
      // lane half G holds d in [G*D/2, G*D/2 + D/2)
#pragma unroll
      for (int c = 0; c < D / 2; c += 4) {
        f32x4 x = q_ok ? *reinterpret_cast<const f32x4*>(qrow + (G * (D / 2) + c) * 4) : f32x4{0, 0, 0, 0};
        qf[c] = x[0];
        qf[c + 1] = x[1];
        qf[c + 2] = x[2];
        qf[c + 3] = x[3];
      }
    } else {
#pragma unroll
      for (int kc = 0; kc < D / 16; ++kc) {
        uint4 x = q_ok ? *reinterpret_cast<const uint4*>(qrow + (16 * kc + 8 * G) * ESZ) : uint4{0, 0, 0, 0};
        qf[kc] = __builtin_bit_cast(QFrag, x);
      }
    }
  }

  f32x16 acc[NDB];
#pragma unroll
  for (int i = 0; i < NDB; ++i) acc[i] = f32x16{0};
  float m_run = kSentinel;
  float l_part = 0.f;

  const char* kbase = a.k + bh * a.k_sb * ESZ;
  const char* vbase = a.v + bh * a.v_sb * ESZ;

  // ---- per-step metadata (uniform, scalar loads) -----------------------------
  auto step_meta = [&](int j) -> StepMeta {
    StepMeta mt;
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      const int seg = 4 * j + t;
      mt.base[t] = -1;
      mt.code[t] = 0u;
      mt.boff[t] = -1;
      if (seg < n_seg) {
        const int64_t ti = row0 + (seg >> spt_log2);
        const int within = seg & spt_mask;
        mt.base[t] = a.kv_idx[ti] * A + within * 16;
        if (a.kv_wave_bits) {
          const int cg = A >= 32 ? (within >> 1) : 0;
          mt.code[t] = a.kv_wave_bits[ti] >> (2 * cg);
        } else {
          mt.code[t] = a.kv_partial[ti] ? 0x55555555u : 0xffffffffu;
        }
        if (use_bits) mt.boff[t] = a.kv_bits_off[ti];
      }
    }
    return mt;
  };
  auto seg_base = [](const StepMeta& mt, int r) -> int {
    const int t = r >> 4;
    return t == 0 ? mt.base[0] : t == 1 ? mt.base[1] : t == 2 ? mt.base[2] : mt.base[3];
  };

  // ---- staging ------------------------------------------------------------
  uint4 kreg[KU];
  uint4 vreg[kF32 ? VU : VT][kF32 ? 1 : 4];
  uint32_t breg[BW];

  auto load_row = [&](const StepMeta& mt, int r) -> int {  // global row, or -1
    const int b0 = seg_base(mt, r);
    if (b0 < 0) return -1;
    const int kvr = b0 + (r & 15);
    return gather_kv ? orig_kv(kvr) : kvr;
  };

  auto load_step = [&](const StepMeta& mt) {
#pragma unroll
    for (int i = 0; i < KU; ++i) {
      const int u = tid + i * NT;
      kreg[i] = uint4{0, 0, 0, 0};
      if (u < kStep * UPR) {
        const int r = u / UPR, un = u % UPR;
        const int lr = load_row(mt, r);
        if (lr >= 0) kreg[i] = *reinterpret_cast<const uint4*>(kbase + ((int64_t)lr * a.k_sn) * ESZ + un * 16);
      }
    }
    if constexpr (kF32) {
#pragma unroll
      for (int i = 0; i < VU; ++i) {
        const int u = tid + i * NT;
        vreg[i][0] = uint4{0, 0, 0, 0};
        if (u < kStep * UPR) {
          const int r = u / UPR, un = u % UPR;
          const int lr = load_row(mt, r);
          if (lr >= 0)
            vreg[i][0] = *reinterpret_cast<const uint4*>(vbase + ((int64_t)lr * a.v_sn) * ESZ + un * 16);
        }
      }
    } else {
#pragma unroll
      for (int i = 0; i < VT; ++i) {
        const int t = tid + i * NT;
#pragma unroll
        for (int e = 0; e < 4; ++e) vreg[i][e] = uint4{0, 0, 0, 0};
        if (t < VTASKS) {
          const int g = t / UPR, un = t % UPR;
          // slot group g holds rows 16*(g/4) + 4*swap(g%4) + 0..3, swap = {0, 2, 1, 3}
          const int gg = g & 3;
          const int rbase = 16 * (g >> 2) + 4 * (((gg & 1) << 1) | (gg >> 1));
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const int lr = load_row(mt, rbase + e);
            if (lr >= 0)
              vreg[i][e] = *reinterpret_cast<const uint4*>(vbase + ((int64_t)lr * a.v_sn) * ESZ + un * 16);
          }
        }
      }
    }
    if (use_bits) {
      const int wpr = (A + 31) >> 5;
#pragma unroll
      for (int i = 0; i < BW; ++i) {
        const int x = tid + i * NT;
        breg[i] = 0u;
        if (x < 4 * ROWS) {
          const int t = x / ROWS, rr = x % ROWS;
          const int off = t == 0 ? mt.boff[0] : t == 1 ? mt.boff[1] : t == 2 ? mt.boff[2] : mt.boff[3];
          const int sb = t == 0 ? mt.base[0] : t == 1 ? mt.base[1] : t == 2 ? mt.base[2] : mt.base[3];
          const int col = sb & (A - 1);  // first column of the segment inside its tile
          if (off >= 0 && rr < a.BQ) breg[i] = a.kv_bits[(int64_t)off + rr * wpr + (col >> 5)] >> (col & 31);
        }
      }
    }
  };

  auto ksw = [](int r) -> int { return UPR >= 16 ? (r & 15) : ((r >> 1) & 7); };

  auto store_step = [&](const StepMeta& mt, int b) {
    char* Ks = smem + b * BUF_BYTES;
    char* Vs = Ks + K_BYTES;
#pragma unroll
    for (int i = 0; i < KU; ++i) {
      const int u = tid + i * NT;
      if (u < kStep * UPR) {
        const int r = u / UPR, un = u % UPR;
        *reinterpret_cast<uint4*>(Ks + (r * UPR + (un ^ ksw(r))) * 16) = kreg[i];
      }
    }
    if constexpr (kF32) {
#pragma unroll
      for (int i = 0; i < VU; ++i) {
        const int u = tid + i * NT;
        if (u < kStep * UPR) {
          const int r = u / UPR, un = u % UPR;
          *reinterpret_cast<uint4*>(Vs + (r * UPR + (un ^ ksw(r))) * 16) = vreg[i][0];
        }
      }
    } else {
      // V^T[d][slot]: 64 slots of 2 B = 128 B per d row, 16-B unit swizzle unit ^ ((d >> 1) & 7)
#pragma unroll
      for (int i = 0; i < VT; ++i) {
        const int t = tid + i * NT;
        if (t < VTASKS) {
          const int g = t / UPR, un = t % UPR;
          // 16-bit element e of a 16-B unit: word e / 2, half e % 2 (no address taken,
          // so the staging registers never go to scratch)
          auto half = [](const uint4& u, int e) -> uint32_t {
            const uint32_t wv = e < 2 ? u.x : e < 4 ? u.y : e < 6 ? u.z : u.w;
            return (e & 1) ? (wv >> 16) : (wv & 0xffffu);
          };
#pragma unroll
          for (int e = 0; e < 8; ++e) {
            const int d = 8 * un + e;
            uint2 val;
            val.x = half(vreg[i][0], e) | (half(vreg[i][1], e) << 16);
            val.y = half(vreg[i][2], e) | (half(vreg[i][3], e) << 16);
            const int unit = (g >> 1) ^ ((d >> 1) & 7);
            *reinterpret_cast<uint2*>(Vs + d * 128 + unit * 16 + (g & 1) * 8) = val;
          }
        }
      }
    }
    if (use_bits) {
#pragma unroll
      for (int i = 0; i < BW; ++i) {
        const int x = tid + i * NT;
        if (x < 4 * ROWS) bits_s[b][x / ROWS][x % ROWS] = breg[i];
      }
    } else if (tid < kStep) {
      // predicate path: original KV coordinate of every staged row
      const int b0 = seg_base(mt, tid);
      kvo_s[b][tid] = b0 < 0 ? -1 : orig_kv(b0 + (tid & 15));
    }
  };

  // 8 live bits for elements 8h..8h+7 of block lb (segment t = 2 lb + h), a segment
  // that is partial for this wave.  Element e sits at segment row 8 * (e / 4) + 4 * G + e % 4.
  auto seg_live8 = [&](int b, int lb, int h) -> uint32_t {
    if (use_bits) {
      const uint32_t field = q_ok ? bits_s[b][2 * lb + h][w * 32 + m] : 0u;
      return ((field >> (4 * G)) & 0xfu) | (((field >> (8 + 4 * G)) & 0xfu) << 4);
    }
    uint32_t bits = 0u;
#pragma unroll 1
    for (int e = 0; e < 8; ++e) {
      const int ko = kvo_s[b][32 * lb + 16 * h + 8 * (e >> 2) + 4 * G + (e & 3)];
      if (ko >= 0 && pred_live_rolled(terms_s, a.pred.n_include, a.pred.n_exclude, q_orig, ko,
                                      a.pred.dense_bits, a.pred.dense_words))
        bits |= 1u << e;
    }
    return bits;
  };

  // ---- main loop ------------------------------------------------------------
#pragma unroll
  for (int i = 0; i < PA_MAX_TERMS; ++i)  // constant indices into the argument block
    if (tid == i) terms_s[i] = a.pred.terms[i];
  StepMeta m_cur = step_meta(0);
  StepMeta m_nxt = step_meta(1);
  if (n_steps > 0) {
    load_step(m_cur);
    store_step(m_cur, 0);
  }
  __syncthreads();

  const int gshift = 2 * w * ncg;  // this wave's group inside a (shifted) tile code
  for (int j = 0; j < n_steps; ++j) {
    const int b = j & 1;
    const bool more = j + 1 < n_steps;
    const StepMeta m_after = step_meta(j + 2);  // scalar loads, in flight during this step
    if (more) load_step(m_nxt);

    const char* Ks = smem + b * BUF_BYTES;
    const char* Vs = Ks + K_BYTES;

    f32x16 s[2];
    bool blive[2];
#pragma unroll
    for (int lb = 0; lb < 2; ++lb) {
      const uint32_t c0 = m_cur.code[2 * lb] >> gshift, c1 = m_cur.code[2 * lb + 1] >> gshift;
      const bool any0 = c0 & 1u, all0 = (c0 >> 1) & 1u, any1 = c1 & 1u, all1 = (c1 >> 1) & 1u;
      blive[lb] = any0 || any1;
      s[lb] = f32x16{0};
      if (!blive[lb]) continue;
      // S^T block: rows = 32 KV rows of this block, cols = the wave's 32 query rows
      const int kr = 32 * lb + m;
      const char* krow = Ks + kr * UPR * 16;
      if constexpr (kF32) {
#pragma unroll
        for (int c = 0; c < D / 2; c += 4) {
          const int un = (G * (D / 2) + c) >> 2;
          const f32x4 kx = *reinterpret_cast<const f32x4*>(krow + (un ^ ksw(kr)) * 16);
          s[lb] = Mma<float>::mma(kx[0], qf[c], s[lb]);
          s[lb] = Mma<float>::mma(kx[1], qf[c + 1], s[lb]);
          s[lb] = Mma<float>::mma(kx[2], qf[c + 2], s[lb]);
          s[lb] = Mma<float>::mma(kx[3], qf[c + 3], s[lb]);
        }
      } else {
#pragma unroll
        for (int kc = 0; kc < D / 16; ++kc) {
          const int un = 2 * kc + G;
          const uint4 kx = *reinterpret_cast<const uint4*>(krow + (un ^ ksw(kr)) * 16);
          s[lb] = Mma<T>::mma(__builtin_bit_cast(typename Mma<T>::frag, kx), qf[kc], s[lb]);
        }
      }
      if (!(all0 && all1)) {
        // live bit i <-> s[lb][i]; a segment is full, dead, or looked up / evaluated
        const uint32_t lo = all0 ? 0xffu : (any0 ? seg_live8(b, lb, 0) : 0u);
        const uint32_t hi = all1 ? 0xffu : (any1 ? seg_live8(b, lb, 1) : 0u);
        const uint32_t live = lo | (hi << 8);
#pragma unroll
        for (int i = 0; i < 16; ++i)
          if (!((live >> i) & 1u)) s[lb][i] = -INFINITY;
      }
    }

    if (blive[0] || blive[1]) {
      float mx = -INFINITY;
#pragma unroll
      for (int lb = 0; lb < 2; ++lb)
        if (blive[lb]) {
#pragma unroll
          for (int i = 0; i < 16; ++i) mx = fmaxf(mx, s[lb][i]);
        }
      mx = fmaxf(mx, other_half(mx));
      const float m_new = fmaxf(m_run, mx * a.c);
      if (__ballot(m_new > m_run + kLazy) != 0ull) {
        const float alpha = exp2f(m_run - m_new);
        m_run = m_new;
        l_part *= alpha;
#pragma unroll
        for (int i = 0; i < NDB; ++i) acc[i] *= alpha;
      }
      const float neg_m = -m_run;
#pragma unroll
      for (int lb = 0; lb < 2; ++lb) {
        if (!blive[lb]) continue;
        float p[16];
#pragma unroll
        for (int i = 0; i < 16; ++i) {
          p[i] = __builtin_amdgcn_exp2f(__builtin_fmaf(s[lb][i], a.c, neg_m));
          l_part += p[i];
        }
        if constexpr (kF32) {
          // PV: O^T[d, q] += V^T[d, kv] P^T[kv, q]; MFMA j pairs KV rows R0(j) (half 0)
          // and R0(j)+4 (half 1) -- exactly the rows whose scores this lane holds in p[j].
#pragma unroll
          for (int jj = 0; jj < 16; ++jj) {
            const int vr = 32 * lb + 8 * (jj >> 2) + 4 * G + (jj & 3);
            const char* vrow = Vs + vr * UPR * 16;
#pragma unroll
            for (int db = 0; db < NDB; ++db) {
              const int d = 32 * db + m;
              const float vx = *reinterpret_cast<const float*>(vrow + (((d >> 2) ^ ksw(vr)) * 16) + (d & 3) * 4);
              acc[db] = Mma<float>::mma(vx, p[jj], acc[db]);
            }
          }
        } else {
#pragma unroll
          for (int c = 0; c < 2; ++c) {
            f32x8 pv;
#pragma unroll
            for (int e = 0; e < 8; ++e) pv[e] = p[8 * c + e];
            const typename Mma<T>::frag pf = Mma<T>::cvt(pv);
            const int unit0 = 4 * lb + 2 * c + G;
#pragma unroll
            for (int db = 0; db < NDB; ++db) {
              const int d = 32 * db + m;
              const uint4 vx = *reinterpret_cast<const uint4*>(Vs + d * 128 + ((unit0 ^ ((d >> 1) & 7)) * 16));
              acc[db] = Mma<T>::mma(__builtin_bit_cast(typename Mma<T>::frag, vx), pf, acc[db]);
            }
          }
        }
      }
    }

    if (more) store_step(m_nxt, b ^ 1);
    m_cur = m_nxt;
    m_nxt = m_after;
    __syncthreads();
  }

  // ---- epilogue -------------------------------------------------------------
  const float l_tot = l_part + other_half(l_part);
  const bool has = l_tot > 0.f;
  float lse_v = has ? (m_run + log2f(l_tot)) * kLn2 : -INFINITY;
  float a_own = has ? 1.f / l_tot : 0.f;  // weight on acc
  float a_prev = 0.f;
  const int srow = (a.scatter_o && has_pq) ? q_orig : r_idx;
  if (a.prev_o && q_ok) {
    const float lp = a.prev_lse[bh * a.lse_sb + srow];
    const float M = fmaxf(lse_v, lp);
    if (M == -INFINITY) {
      a_own = 0.f;
      a_prev = 0.f;
      lse_v = -INFINITY;
    } else {
      const float w1 = has ? expf(lse_v - M) : 0.f;
      const float w2 = lp == -INFINITY ? 0.f : expf(lp - M);
      const float den = w1 + w2;
      a_own = has ? (w1 / den) / l_tot : 0.f;
      a_prev = w2 / den;
      lse_v = M + logf(den);
    }
  }
  if (q_ok) {
    char* orow = a.o + (bh * a.o_sb + (int64_t)srow * a.o_sn) * ESZ;
    const int psz = a.prev_dtype == PA_F32 ? 4 : 2;
    const char* prow = a.prev_o ? a.prev_o + (bh * a.prev_sb + (int64_t)srow * a.prev_sn) * psz : nullptr;
#pragma unroll
    for (int db = 0; db < NDB; ++db) {
#pragma unroll
      for (int i4 = 0; i4 < 4; ++i4) {
        const int d0 = 32 * db + 8 * i4 + 4 * G;
        f32x4 x = {acc[db][4 * i4], acc[db][4 * i4 + 1], acc[db][4 * i4 + 2], acc[db][4 * i4 + 3]};
        x *= a_own;
        if (prow && a_prev != 0.f) x += a_prev * load4_any(prow + d0 * psz, a.prev_dtype);
        Mma<T>::store4(orow + d0 * ESZ, x);
      }
    }
    if (a.lse && G == 0) a.lse[bh * a.lse_sb + srow] = lse_v;
  }
}

template <typename T, int D, int NW>
constexpr int attn_smem_bytes() {
  return 2 * 2 * kStep * D * (int)sizeof(T);
}

}  // namespace pa
