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
//    K and V rows are stored with padded pitches (bank-conflict free for their
//    reads, all addresses affine); the bf16/f16 V^T operand of P.V comes from
//    gfx950's transposed LDS read (ds_read_b64_tr_b16), in the KV-row order that
//    matches P^T's registers.  Each thread's staging offsets are loop invariant;
//    per step only a uniform segment base pointer changes.
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
  const int32_t* steps;  // step descriptors (streaming kernel only)
  int64_t steps_pitch;
  int64_t BH;
  int32_t heads_desc;  // heads issued last to first
  int32_t gather_mult, gather_scatter;  // class-B traffic emulation (K only)
  const char* wsel;
  int64_t wsel_sb;
  const int32_t* run_steps;  // persistent schedule (attn_run_kernel only): run rows
  const int32_t* run_start;  //   and each work-group's first row, [groups + 1]
  // attn_run_kernel: the pieces a run's rows may name (word 9 bit 2), each with its own
  // basis and role, and the counters of a two-piece split in one launch
  int32_t run_res[2], run_qlog2[2];  // closed-form residue basis of piece p (0: none)
  int32_t run_flags[2];              // piece p: gather_q 1, gather_kv 2, scatter_o 4, merge 8
  int32_t* run_sync;                 // [2 * run_sync_groups]: items finished, merges done
  int32_t run_sync_groups, run_sync_signal, run_sync_wait;
  int32_t* run_status;               // set to 1 when a merge gives up waiting
  // attn_stream_kernel<T, true>: a two-piece split in one grid, one work-group per item
  const int32_t* split_items;        // [total_wg][4]: piece, batch-head, query block, sync group
  const int32_t* steps1;             // piece 1's step descriptors (index order), its pitch and
  int64_t steps_pitch1;              //   bitmap pool (piece 0's are steps / steps_pitch / kv_bits)
  const uint32_t* kv_bits1;
};

// flags of a piece of a persistent run (AttnK::run_flags)
constexpr int kPieceGatherQ = 1, kPieceGatherKV = 2, kPieceScatterO = 4, kPieceMerge = 8;

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
  __device__ static bf16x4 cvt4(f32x4 x) { return __builtin_convertvector(x, bf16x4); }
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
  __device__ static f16x4 cvt4(f32x4 x) { return __builtin_convertvector(x, f16x4); }
};

template <>
struct Mma<float> {
  using frag = float;
  __device__ static f32x16 mma(float a, float b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x2f32(a, b, c, 0, 0, 0);
  }
  __device__ static void store4(char* p, f32x4 x) { *reinterpret_cast<f32x4*>(p) = x; }
};

// Class-B traffic emulation (gpu/triton_attn.py:108-128): one 16-byte unit of K rows
// (row krow, kv column col) becomes sum_r wsel[r] * K[row_r] over r < gather_mult, the
// extra rows read contiguously ((krow + r A) mod N) or through the kv permutation
// (perm_kv((col + r A) mod N)).  Accumulated in fp32, rounded once.
template <typename T>
__device__ __forceinline__ uint4 gather_mult_unit(const AttnK& a, const char* kbase, int64_t krow_b, int64_t bh,
                                                  uint4 kx, int krow, int col, int un16) {
  constexpr int E = sizeof(T) == 4 ? 4 : 8;
  typedef float fv __attribute__((ext_vector_type(E)));
  typedef T tv __attribute__((ext_vector_type(E)));
  const T* ws = reinterpret_cast<const T*>(a.wsel) + bh * a.wsel_sb;
  const int32_t rmask = (1 << a.residue_qlog2) - 1;
  fv acc = __builtin_convertvector(__builtin_bit_cast(tv, kx), fv) * (float)ws[0];
  for (int r = 1; r < a.gather_mult; ++r) {
    int er;
    if (a.gather_scatter) {
      const int c = (int)(((int64_t)col + (int64_t)r * a.A) % a.N);
      er = a.residue_s ? (c & rmask) * a.residue_s + (c >> a.residue_qlog2) : (a.pred.perm_kv ? a.pred.perm_kv[c] : c);
    } else {
      er = (int)(((int64_t)krow + (int64_t)r * a.A) % a.N);
    }
    const uint4 x = *reinterpret_cast<const uint4*>(kbase + (int64_t)er * krow_b + un16);
    acc += __builtin_convertvector(__builtin_bit_cast(tv, x), fv) * (float)ws[r];
  }
  return __builtin_bit_cast(uint4, __builtin_convertvector(acc, tv));
}

// 4 consecutive elements of a partial result in dtype dt, as floats.
__device__ __forceinline__ f32x4 load4_any(const char* p, int32_t dt) {
  if (dt == PA_F32) return *reinterpret_cast<const f32x4*>(p);
  if (dt == PA_F16) return __builtin_convertvector(*reinterpret_cast<const f16x4*>(p), f32x4);
  return __builtin_convertvector(*reinterpret_cast<const bf16x4*>(p), f32x4);
}

// Lanes l and l ^ 32 hold the two halves of one query row's KV columns.
// permlane32_swap(x, x) returns {x[l % 32], x[l % 32 + 32]} in every lane.
__device__ __forceinline__ float row_max(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__builtin_bit_cast(int, x), __builtin_bit_cast(int, x), false, false);
  return fmaxf(__builtin_bit_cast(float, (int)r[0]), __builtin_bit_cast(float, (int)r[1]));
}
__device__ __forceinline__ float row_sum(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__builtin_bit_cast(int, x), __builtin_bit_cast(int, x), false, false);
  return __builtin_bit_cast(float, (int)r[0]) + __builtin_bit_cast(float, (int)r[1]);
}

typedef short s16x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) s16x4 lds_s16x4;

// ds_read_b64_tr_b16: in each group of 16 lanes, lane i receives element i % 4 of the
// 8-byte reads of lanes 4e + i / 4 (e = 0..3).  If lane j of the group reads 4
// consecutive columns c0 + 4 (j % 4) of row r0 + j / 4, lane i gets column c0 + i of
// rows r0..r0+3: a transposed 4 x 16 tile.
__device__ __forceinline__ s16x4 lds_read_tr(const char* p) {
  return __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(p));
}

typedef __attribute__((address_space(3))) char lds_char_t;
typedef const __attribute__((address_space(3))) char* lds_cptr;
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef const __attribute__((address_space(3))) u32x4 lds_u4;
typedef const __attribute__((address_space(3))) uint32_t lds_u32;

// LDS DMA (global_load_lds_dwordx4 / _dword): lane l writes LDS[m0 + 16 l] / LDS[m0 + 4 l]
// from gbase + voff.  Issued from inline assembly, so the compiler, which cannot tell
// which LDS bytes a DMA writes, does not wait for it before unrelated LDS reads; the
// caller waits itself (dma_wait_all, then a work-group barrier).  An LDS DMA that reads
// M0 right after a scalar write of M0 needs one wait state, which the compiler's hazard
// pass does not insert inside inline assembly: hence the s_nop 0.
__device__ __forceinline__ void dma_x4(uint32_t m0, const char* gbase, uint32_t voff) {
  asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %1, %2" ::"s"(m0), "v"(voff), "s"(gbase)
               : "m0");
}
__device__ __forceinline__ void dma_x1(uint32_t m0, const char* gbase, uint32_t voff) {
  asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tglobal_load_lds_dword %1, %2" ::"s"(m0), "v"(voff), "s"(gbase)
               : "m0");
}
__device__ __forceinline__ void dma_wait_all() { asm volatile("s_waitcnt vmcnt(0)"); }
// The same DMA with agent-scope coherence (sc1): reads data another work-group published
// with agent-scope stores, whichever XCD's L2 it went through.
__device__ __forceinline__ void dma_x4_sc1(uint32_t m0, const char* gbase, uint32_t voff) {
  asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %1, %2 sc1" ::"s"(m0), "v"(voff),
               "s"(gbase) : "m0");
}
// A 16-byte agent-scope store (sc1: written through to memory, visible to every XCD once
// complete); the caller waits for it (s_waitcnt vmcnt) before publishing.  On gfx950 a VALU
// write to the data registers of a store wider than 8 bytes needs two wait states after
// the store; the compiler's hazard pass does not look inside inline assembly, so the
// s_nop 1 is part of it (without it the next instruction may overwrite the data before
// the store has read it).
__device__ __forceinline__ void store_x4_sc1(char* p, uint32_t x, uint32_t y, uint32_t z, uint32_t w) {
  typedef uint32_t v4 __attribute__((ext_vector_type(4)));
  const v4 v = {x, y, z, w};
  asm volatile("global_store_dwordx4 %0, %1, off sc1\n\ts_nop 1" ::"v"(p), "v"(v) : "memory");
}

// Uniform description of the 4 segments (16 index-space KV rows each) of one step.
struct StepMeta {
  int32_t base[4];   // index-space KV row of the segment's first row; -1 past the list
  int32_t grow[4];   // global row of the segment's first row (after the basis change)
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

// LDS row pitches.  K: one extra 16-B unit, so the 16 rows a 128-bit read touches at
// one column fall in 16 different bank groups.  V (bf16/f16): 64 extra bytes, so the
// 4 consecutive rows of a transposed read fall in 4 disjoint 16-bank ranges.  Padding
// instead of an XOR swizzle keeps every address affine: one base register per lane
// plus immediate offsets.
template <typename T, int D>
constexpr int k_pitch() { return D * (int)sizeof(T) + 16; }
template <typename T, int D>
constexpr int v_pitch() { return D * (int)sizeof(T) + (sizeof(T) == 2 ? 64 : 16); }
template <typename T, int D>
constexpr int buf_bytes() { return kStep * (k_pitch<T, D>() + v_pitch<T, D>()); }

template <typename T, int D, int NW>
__global__ __launch_bounds__(NW * 64) __attribute__((amdgpu_waves_per_eu(occupancy_target<T, D, NW>())))
void attn_fwd_kernel(const AttnK a) {
  constexpr bool kF32 = sizeof(T) == 4;
  constexpr int ESZ = sizeof(T);
  constexpr int UPR = D * ESZ / 16;                 // 16-B units per row
  constexpr int NT = NW * 64;
  constexpr int KP = k_pitch<T, D>();
  constexpr int VP = v_pitch<T, D>();
  constexpr int K_BYTES = kStep * KP;
  constexpr int BUF = buf_bytes<T, D>();
  constexpr int KU = kStep * UPR / NT;              // K (and V) 16-B units per thread
  static_assert(kStep * UPR % NT == 0, "staging units must divide evenly over the threads");
  constexpr int SEGU = 16 * UPR;                    // units per 16-row segment
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
  const int64_t bh = a.heads_desc ? a.BH - 1 - lid / a.nq : lid / a.nq;
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
  const bool closed = a.residue_s != 0;
  const int32_t rmask = (1 << a.residue_qlog2) - 1;
  auto orig_q = [&](int p) __attribute__((always_inline)) -> int {
    if (closed) return (p & rmask) * a.residue_s + (p >> a.residue_qlog2);
    return a.pred.perm_q ? a.pred.perm_q[p] : p;
  };
  auto orig_kv = [&](int p) __attribute__((always_inline)) -> int {
    if (closed) return (p & rmask) * a.residue_s + (p >> a.residue_qlog2);
    return a.pred.perm_kv ? a.pred.perm_kv[p] : p;
  };
  const bool has_pq = closed || a.pred.perm_q;
  const bool gather_kv = a.gather_kv && (closed || a.pred.perm_kv);
  // rows of a segment are an arithmetic progression of global rows unless a permutation
  // table is gathered through (then every row is looked up)
  const bool table = gather_kv && !closed;
  const int rstride = (gather_kv && closed) ? a.residue_s : 1;

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
  const int64_t krow_b = a.k_sn * ESZ, vrow_b = a.v_sn * ESZ;  // bytes per global row

  // ---- per-thread staging geometry -------------------------------------------
  // unit i of this thread: u = i * NT + tid -> row r = i * (NT / UPR) + tid / UPR (0..63),
  // 16-B unit tid % UPR, segment r / 16, row within the segment r % 16.
  constexpr int RPI = NT / UPR;         // rows advanced per unit index
  const int t_row = tid / UPR;          // row of unit 0
  const int t_un16 = (tid % UPR) * 16;  // byte offset of this thread's unit inside a row
  const int64_t kstep_b = (int64_t)rstride * krow_b, vstep_b = (int64_t)rstride * vrow_b;
  // segment of unit i: compile-time when a block of NT units sits inside one segment,
  // else one of two (NT = 2 * SEGU), picked by a fixed per-thread flag
  const bool hi_half = NT > SEGU && (tid >= SEGU);

  // ---- per-step metadata (uniform, scalar loads) -----------------------------
  auto step_meta = [&](int j) __attribute__((always_inline)) -> StepMeta {
    StepMeta mt;
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      const int seg = 4 * j + t;
      mt.base[t] = -1;
      mt.grow[t] = 0;
      mt.code[t] = 0u;
      mt.boff[t] = -1;
      if (seg < n_seg) {
        const int64_t ti = row0 + (seg >> spt_log2);
        const int within = seg & spt_mask;
        const int b0 = a.kv_idx[ti] * A + within * 16;
        mt.base[t] = b0;
        mt.grow[t] = (gather_kv && closed) ? orig_kv(b0) : b0;
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

  // ---- staging ------------------------------------------------------------
  // Prefetch (PA_LOAD_STEP) and LDS store (PA_STORE_STEP) are macros rather than
  // lambdas: a lambda capturing the staging arrays by reference made the compiler keep
  // them in scratch and wait on every prefetch load right after issuing it.
  // Unit i of a thread belongs to segment (i * NT) / SEGU (+1 in the upper half when
  // NT = 2 * SEGU); past-the-list rows read row 0 (valid memory) and V is zeroed there
  // so P = 0 never meets a non-finite value (their scores are masked).
  // The staging registers are single vector values (never memory): element 4 i + c is
  // dword c of unit i.
  typedef uint32_t stage_t __attribute__((ext_vector_type(4 * KU)));
  typedef uint32_t bstage_t __attribute__((ext_vector_type(BW < 2 ? 2 : BW)));
  stage_t kreg, vreg;
  bstage_t breg;

#define PA_LOAD_STEP(mt) \
  do { \
_Pragma("unroll") \
    for (int i = 0; i < KU; ++i) { \
      const int t0 = (i * NT) / SEGU; \
      const int t = (NT > SEGU) ? t0 + (hi_half ? 1 : 0) : t0; \
      const int grow = t == 0 ? (mt).grow[0] : t == 1 ? (mt).grow[1] : t == 2 ? (mt).grow[2] : (mt).grow[3]; \
      const int b0 = t == 0 ? (mt).base[0] : t == 1 ? (mt).base[1] : t == 2 ? (mt).base[2] : (mt).base[3]; \
      const bool valid = b0 >= 0; \
      const int rr = (i * RPI + t_row) & 15; \
      uint4 kx, vx; \
      if (!table) { \
        const char* kp = kbase + (int64_t)grow * krow_b; \
        const char* vp = vbase + (int64_t)grow * vrow_b; \
        kx = *reinterpret_cast<const uint4*>(kp + (int)(rr * kstep_b) + t_un16); \
        vx = *reinterpret_cast<const uint4*>(vp + (int)(rr * vstep_b) + t_un16); \
        if (a.gather_mult > 1 && valid) \
          kx = gather_mult_unit<T>(a, kbase, krow_b, bh, kx, grow + rr * rstride, b0 + rr, t_un16); \
      } else { \
        const int lr = valid ? a.pred.perm_kv[b0 + rr] : 0; \
        kx = *reinterpret_cast<const uint4*>(kbase + (int64_t)lr * krow_b + t_un16); \
        vx = *reinterpret_cast<const uint4*>(vbase + (int64_t)lr * vrow_b + t_un16); \
        if (a.gather_mult > 1 && valid) kx = gather_mult_unit<T>(a, kbase, krow_b, bh, kx, lr, b0 + rr, t_un16); \
      } \
      if (!valid) vx = uint4{0, 0, 0, 0}; \
      kreg[4 * i] = kx.x; kreg[4 * i + 1] = kx.y; kreg[4 * i + 2] = kx.z; kreg[4 * i + 3] = kx.w; \
      vreg[4 * i] = vx.x; vreg[4 * i + 1] = vx.y; vreg[4 * i + 2] = vx.z; vreg[4 * i + 3] = vx.w; \
    } \
    if (use_bits) { \
      const int wpr = (A + 31) >> 5; \
_Pragma("unroll") \
      for (int i = 0; i < BW; ++i) { \
        const int x = tid + i * NT; \
        breg[i] = 0u; \
        const int t = x / ROWS, rr = x % ROWS; \
        if (x < 4 * ROWS) { \
          const int off = t == 0 ? (mt).boff[0] : t == 1 ? (mt).boff[1] : t == 2 ? (mt).boff[2] : (mt).boff[3]; \
          const int sb = t == 0 ? (mt).base[0] : t == 1 ? (mt).base[1] : t == 2 ? (mt).base[2] : (mt).base[3]; \
          const int col = sb & (A - 1); \
          if (off >= 0 && rr < a.BQ) breg[i] = a.kv_bits[(int64_t)off + rr * wpr + (col >> 5)] >> (col & 31); \
        } \
      } \
    } \
  } while (0)

#define PA_STORE_STEP(mt, b) \
  do { \
    char* buf = smem + (b) * BUF; \
    char* kdst = buf + t_row * KP + t_un16; \
    char* vdst = buf + K_BYTES + t_row * VP + t_un16; \
_Pragma("unroll") \
    for (int i = 0; i < KU; ++i) { \
      *reinterpret_cast<uint4*>(kdst + i * RPI * KP) = uint4{kreg[4 * i], kreg[4 * i + 1], kreg[4 * i + 2], kreg[4 * i + 3]}; \
      *reinterpret_cast<uint4*>(vdst + i * RPI * VP) = uint4{vreg[4 * i], vreg[4 * i + 1], vreg[4 * i + 2], vreg[4 * i + 3]}; \
    } \
    if (use_bits) { \
_Pragma("unroll") \
      for (int i = 0; i < BW; ++i) { \
        const int x = tid + i * NT; \
        if (x < 4 * ROWS) bits_s[(b)][x / ROWS][x % ROWS] = breg[i]; \
      } \
    } else if (tid < kStep) { \
      int b0 = (mt).base[3]; \
      if (tid < 16) b0 = (mt).base[0]; \
      else if (tid < 32) b0 = (mt).base[1]; \
      else if (tid < 48) b0 = (mt).base[2]; \
      kvo_s[(b)][tid] = b0 < 0 ? -1 : orig_kv(b0 + (tid & 15)); \
    } \
  } while (0)

  // 8 live bits for elements 8h..8h+7 of block lb (segment t = 2 lb + h), a segment
  // that is partial for this wave.  Element e sits at segment row 8 * (e / 4) + 4 * G + e % 4.
  auto seg_live8 = [&](int b, int lb, int h) __attribute__((always_inline)) -> uint32_t {
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

  // ---- loop-invariant LDS read offsets ---------------------------------------
  // QK: lane reads K row 32 lb + m, 16-B units 2 kc + G (kc = 0..D/16-1), i.e.
  //     k_rd + lb * 32 * KP + kc * 32.
  const int k_rd = m * KP + G * 16;
  // PV (bf16/f16): transposed reads of V rows 32 lb + 16 c + 4 G + j / 4 (+8), columns
  //     32 db + 16 dgrp + 4 (j % 4) (j = lane % 16): v_rd + lb * 32 VP + c * 16 VP + db * 64.
  const int j16 = lane & 15;
  const int v_rd = K_BYTES + (4 * G + (j16 >> 2)) * VP + (((lane >> 4) & 1) * 16 + 4 * (j16 & 3)) * ESZ;

  // ---- main loop ------------------------------------------------------------
#pragma unroll
  for (int i = 0; i < PA_MAX_TERMS; ++i)  // constant indices into the argument block
    if (tid == i) terms_s[i] = a.pred.terms[i];
  StepMeta m_cur = step_meta(0);
  StepMeta m_nxt = step_meta(1);
  if (n_steps > 0) {
    PA_LOAD_STEP(m_cur);
    PA_STORE_STEP(m_cur, 0);
  }
  __syncthreads();

  const int gshift = 2 * w * ncg;  // this wave's group inside a (shifted) tile code
  for (int j = 0; j < n_steps; ++j) {
    const int b = j & 1;
    const bool more = j + 1 < n_steps;
    const StepMeta m_after = step_meta(j + 2);  // scalar loads, in flight during this step
    if (more) PA_LOAD_STEP(m_nxt);

    const char* buf = smem + b * BUF;

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
      const char* krow = buf + k_rd + lb * 32 * KP;
      if constexpr (kF32) {
        // f32: lane half G holds d in [G*D/2, +D/2): 16-B reads at columns G*D/2 + c
        const char* kr2 = buf + m * KP + lb * 32 * KP + G * (D / 2) * 4;
#pragma unroll
        for (int c = 0; c < D / 2; c += 4) {
          const f32x4 kx = *reinterpret_cast<const f32x4*>(kr2 + c * 4);
          s[lb] = Mma<float>::mma(kx[0], qf[c], s[lb]);
          s[lb] = Mma<float>::mma(kx[1], qf[c + 1], s[lb]);
          s[lb] = Mma<float>::mma(kx[2], qf[c + 2], s[lb]);
          s[lb] = Mma<float>::mma(kx[3], qf[c + 3], s[lb]);
        }
        (void)krow;
      } else {
#pragma unroll
        for (int kc = 0; kc < D / 16; ++kc) {
          const uint4 kx = *reinterpret_cast<const uint4*>(krow + kc * 32);
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
      mx = row_max(mx);
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
            const char* vrow = buf + K_BYTES + vr * VP;
#pragma unroll
            for (int db = 0; db < NDB; ++db) {
              const float vx = *reinterpret_cast<const float*>(vrow + (32 * db + m) * 4);
              acc[db] = Mma<float>::mma(vx, p[jj], acc[db]);
            }
          }
        } else {
          // A operand V^T[d][kv]: lane (d = l % 32, half G) needs rows 16 c + 4 G + 0..3 and
          // 16 c + 8 + 4 G + 0..3 (the rows of its P^T values) at column d: two transposed
          // reads, lane j of each 16-lane group reading row r0 + j / 4, columns 4 (j % 4)..+3.
#pragma unroll
          for (int c = 0; c < 2; ++c) {
            f32x8 pv;
#pragma unroll
            for (int e = 0; e < 8; ++e) pv[e] = p[8 * c + e];
            const typename Mma<T>::frag pf = Mma<T>::cvt(pv);
            const char* v1 = buf + v_rd + (32 * lb + 16 * c) * VP;
#pragma unroll
            for (int db = 0; db < NDB; ++db) {
              const s16x4 x1 = lds_read_tr(v1 + db * 32 * ESZ);
              const s16x4 x2 = lds_read_tr(v1 + 8 * VP + db * 32 * ESZ);
              const uint4 vx = {__builtin_bit_cast(uint2, x1).x, __builtin_bit_cast(uint2, x1).y,
                                __builtin_bit_cast(uint2, x2).x, __builtin_bit_cast(uint2, x2).y};
              acc[db] = Mma<T>::mma(__builtin_bit_cast(typename Mma<T>::frag, vx), pf, acc[db]);
            }
          }
        }
      }
    }

    if (more) PA_STORE_STEP(m_nxt, b ^ 1);
    m_cur = m_nxt;
    m_nxt = m_after;
    __syncthreads();
  }

  // ---- epilogue -------------------------------------------------------------
  const float l_tot = row_sum(l_part);
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
  return 2 * buf_bytes<T, D>();
}

}  // namespace pa

#undef PA_LOAD_STEP
#undef PA_STORE_STEP
