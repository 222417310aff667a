// Streaming block-sparse attention forward for gfx950: f16 / bf16, D = 128, BQ = 128.
//
// Same contract and numerics as attn_fwd_kernel (the replacement of the Triton
// kernel _attn_fwd, gpu/triton_attn.py:62-182): one work-group of 4 waves per
// (query block, batch-head), each wave owning 32 query rows, scores computed
// transposed (S^T = K Q^T) on 32x32x16 MFMAs, online softmax with the finite
// -1e30 sentinel, lazy rescale and the l > 0 guard.  What differs is how K and V
// reach the MFMAs and how little work a step costs outside them:
//
//  * K and V rows go from global memory straight into LDS with gfx950's LDS DMA
//    (global_load_lds_dwordx4): no staging registers, no LDS store instructions.
//    The DMA is issued from inline assembly so that the compiler, which cannot
//    tell which LDS stage a DMA writes, does not wait for all of them before every
//    LDS read; the kernel waits itself (vmcnt(0) at the top of a step, then the
//    work-group barrier), one step ahead, with two LDS stages.
//  * A DMA instruction writes 64 consecutive 16-byte units, so rows are stored
//    unpadded and the bank conflicts are removed by an XOR swizzle of the 16-byte
//    units inside a 256-byte row: K unit u of row r sits at u ^ (r & 15) (the 16
//    rows a 128-bit read touches hit 16 different bank groups), V unit u at
//    u ^ 4 (r & 3) (the 4 rows of a transposed read hit disjoint bank groups).
//    The lane of a DMA picks its source unit so that the LDS layout comes out
//    swizzled; every read address is loop invariant plus an immediate offset.
//  * What a step needs to know (segment columns, per-wave codes, bitmap offsets) is
//    one 64-byte descriptor built with the index (pa_index_steps), read with scalar
//    loads two steps ahead.
//  * Partial blocks are masked from element bitmaps that the DMA also brings into
//    LDS; row maxima use max3, row sums are dot2 products of the packed P values.
#pragma once

#include "attn_kernel.hpp"

namespace pa {

struct StepDesc {
  int32_t base[4];  // K / V row of each 16-column segment (gather basis applied), 0 past the list
  uint32_t code;    // byte t: segment t's 2-bit codes for the 4 row groups
  int32_t boff[4];  // pool word offset of the bitmap word of segment t, -1 when none
  int32_t pad[7];
};
static_assert(sizeof(StepDesc) == 64, "descriptor is 16 words");

// LDS layout: two bitmap slots (4 x 128 words each), a ring of two V slots and a ring of
// two K slots (64 rows x 256 B each).  K and V have separate rings because a step's
// K is consumed one iteration before its V (the QK of step j + 1 runs beside the P.V
// of step j).  Every read offset (slot, block, chunk) fits a DS instruction's 16-bit
// immediate on top of a per-lane base register.
constexpr int kBits = 0;
constexpr int kBitsSlot = 2048;
constexpr int kVring = 4096;
constexpr int kKring = 36864;
constexpr int kSlot = 16384;
constexpr int kStreamSmem = kKring + 2 * kSlot;
// polls of a split grid's sync count before a merge gives up (each ~0.5 us)
constexpr int kSplitMaxPolls = 1 << 20;

template <typename T>
__device__ __forceinline__ float dot2_sum(uint32_t packed, float acc);
template <>
__device__ __forceinline__ float dot2_sum<__bf16>(uint32_t packed, float acc) {
  typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
  const bf16x2 one = {(__bf16)1.0f, (__bf16)1.0f};
  return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, packed), one, acc, false);
}
template <>
__device__ __forceinline__ float dot2_sum<_Float16>(uint32_t packed, float acc) {
  typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
  const f16x2 one = {(_Float16)1.0f, (_Float16)1.0f};
  return __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2, packed), one, acc, false);
}

// SPLIT: the grid holds the items of both pieces of a disjoint split (AttnK::split_items,
// in the order the work-groups are dispatched).  A first-piece item publishes its output
// rows and log-sum-exp with agent-scope stores and counts itself in its sync group; a
// second-piece item waits for its group's count before it reads those rows to merge them.
// Work-groups are dispatched in id order and the items a second-piece item waits for have
// lower ids, so they are running or done when it waits; the wait is also bounded (a merge
// that gives up sets *run_status, which only the host clears, together with the counters;
// a status left set by an earlier launch does not shorten this launch's waits).  The last
// merge of a group zeroes the group's counters.
// MODE (one work-group per item only): 0 every option from the arguments; the others are
// compiled for 32-column tiles and one basis, with the merge known: 1 index space (no basis,
// no permutation tables), 2 closed-form residue basis with Q and K / V gathered and O
// scattered through it (N / s >= 128, so a query block lies in one class's segment), 3 and
// 4 the same two merging into a 2-byte previous partial.  The launcher picks the mode from
// the arguments; every mode gives the same results bit for bit.
template <typename T, bool SPLIT, int MODE = 0>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2)))
void attn_stream_kernel(const AttnK a) {
  constexpr int D = 128;
  constexpr int ESZ = 2;
  constexpr int NDB = D / 32;   // 32-wide output blocks
  constexpr int NQF = D / 16;   // Q fragments (16 dims each)
  using Frag = typename Mma<T>::frag;

  extern __shared__ __attribute__((aligned(16))) char smem[];
  const uint32_t lds0 = (uint32_t)(uintptr_t)(lds_char_t*)smem;

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int G = lane >> 5;
  const int m = lane & 31;

  // (32-bit index arithmetic: the grid is below 2^31 work-groups, checked on the host)
  const uint32_t lid = xcd_remap32(blockIdx.x, (uint32_t)a.total_wg);
  typedef const __attribute__((address_space(4))) int32_t cint;
  int64_t bh;
  int pc = 0, sg = -1;
  int qb_direct;  // the query block when it is known without reading the first descriptor
  const StepDesc* desc;
  if constexpr (SPLIT) {
    // the item of this work-group and its piece's descriptors (index order)
    cint* it = (cint*)a.split_items + 4 * (int64_t)lid;
    pc = it[0];
    bh = it[1];
    sg = it[3];
    desc = reinterpret_cast<const StepDesc*>(pc ? a.steps1 : a.steps) + (int64_t)it[2] * (pc ? a.steps_pitch1 : a.steps_pitch);
    qb_direct = it[2];
  } else {
    const uint32_t bh_l = lid / (uint32_t)a.nq;
    bh = a.heads_desc ? a.BH - 1 - bh_l : bh_l;
    const int qb_lin = (int)(lid - bh_l * (uint32_t)a.nq);
    // The lists are laid out in issue order; a list's first descriptor names its query
    // block and its length, so one scalar load starts the work-group.
    desc = reinterpret_cast<const StepDesc*>(a.steps) + (int64_t)qb_lin * a.steps_pitch;
    qb_direct = a.qblock_order ? -1 : qb_lin;
  }
  // Lists in index order (a split grid's, or a launch without an issue order) start on
  // their own query block, so the query rows' loads need not wait for the descriptor.
  const int qb = qb_direct >= 0 ? qb_direct : ((cint*)desc)[13];
  const int n_steps = ((cint*)desc)[14];
  // the basis of the specialised modes: 1 and 3 index space, 2 and 4 closed-form residue;
  // 3 and 4 merge into a 2-byte previous partial (its row layout that of the output)
  constexpr int BASIS = MODE == 0 ? 0 : (MODE == 1 || MODE == 3) ? 1 : 2;
  constexpr int MERGE = MODE == 0 ? -1 : MODE >= 3 ? 1 : 0;
  const int A = MODE ? 32 : a.A;

  // the piece's basis and role: the launch's arguments, or in a split grid those of the
  // item's piece (the second piece merges into the first piece's output and log-sum-exp)
  const int res_s = BASIS == 1 ? 0 : SPLIT ? a.run_res[pc] : a.residue_s;
  const int res_q = BASIS == 1 ? 0 : SPLIT ? a.run_qlog2[pc] : a.residue_qlog2;
  const int pflags = SPLIT ? a.run_flags[pc] : 0;
  const bool g_q = BASIS ? BASIS == 2 : SPLIT ? (pflags & kPieceGatherQ) != 0 : a.gather_q != 0;
  const bool g_kv = BASIS ? BASIS == 2 : SPLIT ? (pflags & kPieceGatherKV) != 0 : a.gather_kv != 0;
  const bool sc_o = BASIS ? BASIS == 2 : SPLIT ? (pflags & kPieceScatterO) != 0 : a.scatter_o != 0;
  const char* prev_o = MERGE == 0 ? nullptr : (!SPLIT || (pflags & kPieceMerge)) ? a.prev_o : nullptr;
  const bool signal = SPLIT && pc == 0;
  const bool waits = SPLIT && pc == 1;

  const bool closed = BASIS ? BASIS == 2 : res_s != 0;
  const int32_t rmask = (1 << res_q) - 1;
  const bool has_pq = BASIS ? BASIS == 2 : closed || (!SPLIT && a.pred.perm_q);
  const bool gather_kv = g_kv && closed;
  const int rstride = gather_kv ? res_s : 1;

  const int r_idx = qb * 128 + w * 32 + m;  // index-space query row of this lane
  int q_orig = r_idx;
  if (has_pq) q_orig = closed ? (r_idx & rmask) * res_s + (r_idx >> res_q) : a.pred.perm_q[r_idx];
  const int r_load = (g_q && has_pq) ? q_orig : r_idx;

  const char* kbase = a.k + bh * a.k_sb * ESZ;
  const char* vbase = a.v + bh * a.v_sb * ESZ;
  // row offsets inside a head fit in 32 bits (checked on the host)
  const uint32_t krow_b32 = (uint32_t)(a.k_sn * ESZ), vrow_b32 = (uint32_t)(a.v_sn * ESZ);
  const char* bits = reinterpret_cast<const char*>(SPLIT && pc ? a.kv_bits1 : a.kv_bits);
  const int wpr = (A + 31) >> 5;

  // ---- DMA geometry (loop invariant) ----------------------------------------
  // Wave w moves rows 4 w .. 4 w + 3 of every 16-row segment, one row per 16 lanes:
  // lane l writes LDS unit p = l % 16 of row rs = 4 w + l / 16 and fetches the global
  // unit that the swizzle stores there.
  const int rs = 4 * w + (lane >> 4);
  const int pu = lane & 15;
  const uint32_t k_goff = (uint32_t)(rs * rstride) * krow_b32 + 16u * (uint32_t)(pu ^ rs);
  const uint32_t v_goff = (uint32_t)(rs * rstride) * vrow_b32 + 16u * (uint32_t)(pu ^ (4 * (rs & 3)));
  // bitmaps: A >= 32 -> wave w moves rows 64 (w & 1) + lane of block (w >> 1)'s word
  // column; A = 16 -> wave w moves all 128 rows of segment w's word column
  const uint32_t b_goff = A >= 32 ? (uint32_t)((64 * (w & 1) + lane) * wpr * 4) : (uint32_t)(lane * 4);
  // The previous partial (2-byte types, rows in index order or through the closed-form
  // basis) is DMAed into the K ring at the end of the list: rows 0..63 of the block while
  // the last iteration runs, rows 64..127 at the last step; 16-row segments as for K.
  const bool prev16 = MERGE >= 0 ? MERGE == 1 : prev_o && a.prev_dtype != PA_F32;
  const bool prev_dma = prev16 && !(sc_o && has_pq && !closed);
  const bool prev_closed = sc_o && closed;
  const uint32_t p_goff =
      (uint32_t)(rs * (prev_closed ? res_s : 1)) * (uint32_t)(a.prev_sn * 2) + 16u * (uint32_t)(pu ^ rs);
  const char* pbase = prev_o + bh * a.prev_sb * 2;

  // ---- LDS read geometry (loop invariant; slot / block / chunk offsets are immediates)
  // QK: lane (m, G) reads K row 32 lb + m, unit 2 kc + G.
  lds_cptr lds = (lds_cptr)smem;
  lds_cptr kptr[NQF];
#pragma unroll
  for (int kc = 0; kc < NQF; ++kc) {
    kptr[kc] = lds + kKring + m * 256 + 16 * ((2 * kc + G) ^ (m & 15));
    // (opaque to the compiler, so each address stays whole in one register instead of
    // being rebuilt from shared parts at every read)
    asm volatile("" : "+v"(kptr[kc]));
  }
  // PV: transposed reads of V rows 32 lb + 16 c + 4 G + j16 / 4 (+8), columns
  // 32 db + 16 h16 + 4 (j16 % 4) .. +3; row % 4 = j16 / 4 fixes the swizzle.
  const int j16 = lane & 15;
  const int h16 = (lane >> 4) & 1;
  lds_cptr vptr[NDB];
#pragma unroll
  for (int db = 0; db < NDB; ++db) {
    vptr[db] = lds + kVring + (4 * G + (j16 >> 2)) * 256 +
               16 * ((4 * db + 2 * h16 + ((j16 & 3) >> 1)) ^ (4 * (j16 >> 2))) + 8 * (j16 & 1);
    asm volatile("" : "+v"(vptr[db]));
  }
  lds_cptr bptr = lds + kBits + (w * 32 + m) * 4;  // this lane's word in a bitmap slot
  asm volatile("" : "+v"(bptr));

  // ---- Q fragments (B operand of S^T = K Q^T) --------------------------------
  Frag qf[NQF];
  {
    const char* qrow = a.q + (bh * a.q_sb + (int64_t)r_load * a.q_sn) * ESZ;
#pragma unroll
    for (int kc = 0; kc < NQF; ++kc)
      qf[kc] = __builtin_bit_cast(Frag, *reinterpret_cast<const uint4*>(qrow + (16 * kc + 8 * G) * ESZ));
  }

  f32x16 acc[NDB];
#pragma unroll
  for (int i = 0; i < NDB; ++i) acc[i] = f32x16{0};
  float m_run = kSentinel;
  float l_part = 0.f;
  const float cexp = a.c;

  // The first descriptors of a list are read through the constant address space, as
  // scalar loads.  Inside the step loop a descriptor is instead one vector load (lane l
  // reads word l % 16), unpacked with v_readlane after the next iteration's vmcnt(0)
  // wait, which the DMA needs anyway: a scalar load there would share lgkmcnt with the
  // LDS reads, and since scalar loads return out of order, the first LDS wait of the
  // MFMA block would have to be lgkmcnt(0) and would stall on the scalar load.
  auto load_desc = [&](int jd) __attribute__((always_inline)) -> StepDesc {
    cint* c = (cint*)(reinterpret_cast<const int32_t*>(desc + jd));
    StepDesc r{};
    r.base[0] = c[0];
    r.base[1] = c[1];
    r.base[2] = c[2];
    r.base[3] = c[3];
    r.code = (uint32_t)c[4];
    r.boff[0] = c[5];
    r.boff[1] = c[6];
    r.boff[2] = c[7];
    r.boff[3] = c[8];
    return r;
  };
  auto load_desc_v = [&](int jd) __attribute__((always_inline)) -> int32_t {
    return reinterpret_cast<const int32_t*>(desc + jd)[lane & 15];
  };
  auto unpack_desc = [&](int32_t dv) __attribute__((always_inline)) -> StepDesc {
    StepDesc r{};
    r.base[0] = __builtin_amdgcn_readlane(dv, 0);
    r.base[1] = __builtin_amdgcn_readlane(dv, 1);
    r.base[2] = __builtin_amdgcn_readlane(dv, 2);
    r.base[3] = __builtin_amdgcn_readlane(dv, 3);
    r.code = (uint32_t)__builtin_amdgcn_readlane(dv, 4);
    r.boff[0] = __builtin_amdgcn_readlane(dv, 5);
    r.boff[1] = __builtin_amdgcn_readlane(dv, 6);
    r.boff[2] = __builtin_amdgcn_readlane(dv, 7);
    r.boff[3] = __builtin_amdgcn_readlane(dv, 8);
    return r;
  };
  // This wave's view of a step: bit t = segment t has a live pair / is all live.
  struct Flags {
    uint32_t live, full;
  };
  auto flags_of = [&](uint32_t code) __attribute__((always_inline)) -> Flags {
    const uint32_t cw = code >> (2 * w);
    return Flags{(cw & 1u) | ((cw >> 7) & 2u) | ((cw >> 14) & 4u) | ((cw >> 21) & 8u),
                 ((cw >> 1) & 1u) | ((cw >> 8) & 2u) | ((cw >> 15) & 4u) | ((cw >> 22) & 8u)};
  };

#include "attn_stream_ops.inc"

  // DMA of rows 64 h .. 64 h + 63 of the previous partial into K slot SL.
#define PA_DMA_PREV(h, SL)                                                                        \
  do {                                                                                            \
    _Pragma("unroll") for (int t = 0; t < 4; ++t) {                                               \
      const int r_ = qb * 128 + 64 * (h) + 16 * t;                                                \
      const int pr_ = prev_closed ? (r_ & rmask) * res_s + (r_ >> res_q) : r_;                    \
      if (waits)                                                                                  \
        dma_x4_sc1(lds0 + kKring + (SL) * kSlot + (16 * t + 4 * w) * 256, pbase + (int64_t)pr_ * a.prev_sn * 2, p_goff); \
      else                                                                                        \
        dma_x4(lds0 + kKring + (SL) * kSlot + (16 * t + 4 * w) * 256, pbase + (int64_t)pr_ * a.prev_sn * 2, p_goff); \
    }                                                                                             \
  } while (0)

  // One iteration jj (P = jj & 1), for jj + 1 < n_steps: QK of step jj + 1 (K slot P ^ 1)
  // beside the softmax of step jj, P.V of step jj (V slot P) beside the shaping and the
  // maximum of step jj + 1.  At entry, after the wait and the barrier, K / bitmaps of
  // step jj + 1 and V of step jj are in LDS; the slots the new DMA writes were last read
  // before the barrier.  A block dead for this wave holds -inf (set when its scores
  // were made), so its P is 0 and one straight-line body serves every step.
#define PA_ITER(jj, P)                                                                            \
  do {                                                                                            \
    dma_wait_all();                                                                               \
    __syncthreads();                                                                              \
    if ((jj) + 2 < n_steps) {                                                                     \
      d_j2 = unpack_desc(dv_j2);                                                                  \
      PA_DMA_K(d_j2, (P));                                                                        \
    } else if (prev_dma) {                                                                        \
      PA_SPLIT_WAIT();                                                                            \
      PA_DMA_PREV(0, (P));                                                                        \
    }                                                                                             \
    PA_DMA_V(d_j1, (P) ^ 1);                                                                      \
    if ((jj) + 3 < n_steps) dv_j2 = load_desc_v((jj) + 3);                                        \
    const Flags fn = flags_of(d_j1.code);                                                         \
    const float neg_m = -m_run;                                                                   \
    f32x16 sn0, sn1;                                                                              \
    if (fc.live | fn.live) {                                                                      \
      Frag pf00, pf01, pf10, pf11;                                                                \
      PA_EXP(pf00, sc0, 0);                                                                       \
      PA_EXP(pf01, sc0, 1);                                                                       \
      PA_EXP(pf10, sc1, 0);                                                                       \
      PA_EXP(pf11, sc1, 1);                                                                       \
      PA_QK(sn0, sn1, (P) ^ 1);                                                                   \
      PA_PV(pf00, (P), 0, 0);                                                                     \
      PA_PV(pf01, (P), 0, 1);                                                                     \
      PA_PV(pf10, (P), 1, 0);                                                                     \
      PA_PV(pf11, (P), 1, 1);                                                                     \
      PA_FAST_ORDER();                                                                            \
    }                                                                                             \
    PA_SHAPE(sn0, (P) ^ 1, 0, fn);                                                                \
    PA_SHAPE(sn1, (P) ^ 1, 1, fn);                                                                \
    if (fn.live) {                                                                                \
      float mx = -INFINITY;                                                                       \
      PA_BLOCK_MAX(mx, sn0);                                                                      \
      PA_BLOCK_MAX(mx, sn1);                                                                      \
      PA_RAISE(mx);                                                                               \
    }                                                                                             \
    sc0 = sn0;                                                                                    \
    sc1 = sn1;                                                                                    \
    fc = fn;                                                                                      \
    d_j1 = d_j2;                                                                                  \
  } while (0)

  // The last step: its V (slot P) arrives, then its softmax and P.V.  The previous
  // partial result the epilogue merges (2-byte types) is loaded here, after the last
  // wait for a DMA, so its latency hides behind this step.
#define PA_LAST(P)                                                                                \
  do {                                                                                            \
    dma_wait_all();                                                                               \
    __syncthreads();                                                                              \
    if (prev_dma) {                                                                               \
      PA_SPLIT_WAIT();                                                                            \
      if (n_steps == 1) PA_DMA_PREV(0, (P) ^ 1);                                                  \
      PA_DMA_PREV(1, (P));                                                                        \
      PA_PREV_LSE();                                                                              \
    } else {                                                                                      \
      PA_PREV_LOAD();                                                                             \
    }                                                                                             \
    if (fc.live) {                                                                                \
      const float neg_m = -m_run;                                                                 \
      Frag pf00, pf01, pf10, pf11;                                                                \
      PA_EXP(pf00, sc0, 0);                                                                       \
      PA_EXP(pf01, sc0, 1);                                                                       \
      PA_EXP(pf10, sc1, 0);                                                                       \
      PA_EXP(pf11, sc1, 1);                                                                       \
      PA_PV(pf00, (P), 0, 0);                                                                     \
      PA_PV(pf01, (P), 0, 1);                                                                     \
      PA_PV(pf10, (P), 1, 0);                                                                     \
      PA_PV(pf11, (P), 1, 1);                                                                     \
    }                                                                                             \
  } while (0)

  // Rows of the previous partial (prev_o, 2-byte types): 4 elements per (db, i4), the
  // columns this lane writes in the epilogue.
  const int srow = (sc_o && has_pq) ? q_orig : r_idx;
  uint2 prevw[NDB * 4];
  float prev_lse = -INFINITY;
  // A second-piece item of a split grid waits, before its first read of the merge
  // input, until every first-piece item of its sync group has published its rows
  // (thread 0 polls the group's count; the barrier releases the work-group).
  bool waited = false;
#define PA_SPLIT_WAIT()                                                                           \
  do {                                                                                            \
    if (waits && !waited) {                                                                       \
      if (tid == 0) {                                                                             \
        int polls_ = 0;                                                                           \
        while (__hip_atomic_load(a.run_sync + sg, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) <   \
               a.run_sync_signal) {                                                               \
          if (++polls_ >= kSplitMaxPolls) {                                                       \
            __hip_atomic_store(a.run_status, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);      \
            break;                                                                                \
          }                                                                                       \
          __builtin_amdgcn_s_sleep(16);                                                           \
        }                                                                                         \
      }                                                                                           \
      __syncthreads();                                                                            \
      waited = true;                                                                              \
    }                                                                                             \
  } while (0)
#define PA_PREV_LSE()                                                                             \
  do {                                                                                            \
    if (prev_o) {                                                                                 \
      const float* lp_ = a.prev_lse + bh * a.lse_sb + srow;                                       \
      prev_lse = waits ? __hip_atomic_load(lp_, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) : *lp_; \
    }                                                                                             \
  } while (0)
#define PA_PREV_LOAD()                                                                            \
  do {                                                                                            \
    PA_SPLIT_WAIT();                                                                              \
    PA_PREV_LSE();                                                                                \
    if (prev16) {                                                                                 \
      const char* prow_ = prev_o + (bh * a.prev_sb + (int64_t)srow * a.prev_sn) * 2;               \
      _Pragma("unroll") for (int q_ = 0; q_ < NDB * 4; ++q_) {                                    \
        const uint2* at_ = reinterpret_cast<const uint2*>(prow_ + (32 * (q_ >> 2) + 8 * (q_ & 3) + 4 * G) * 2); \
        prevw[q_] = waits ? __builtin_bit_cast(uint2, __hip_atomic_load(reinterpret_cast<const uint64_t*>(at_), \
                                                                        __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)) \
                          : *at_;                                                                 \
      }                                                                                           \
    }                                                                                             \
  } while (0)

  // Prologue: step 0's K, bitmaps and V; then step 1's K; QK, shaping and maximum of
  // step 0.
  // d_j1 / d_j2: descriptors of the steps one and two ahead; dv_j2: the raw descriptor
  // (one word per lane) that becomes d_j2 at the top of the next iteration
  StepDesc d_j1{}, d_j2{};
  int32_t dv_j2 = 0;
  Flags fc{0u, 0u};
  f32x16 sc0, sc1;
  if (n_steps > 0) {
    const StepDesc d0 = load_desc(0);
    if (n_steps > 1) d_j1 = load_desc(1);
    if (n_steps > 2) dv_j2 = load_desc_v(2);
    PA_DMA_K(d0, 0);
    PA_DMA_V(d0, 0);
    dma_wait_all();
    // The compiler counts its own vector loads in vmcnt and would place the waits for Q
    // at the first use, inside the loop, where they would also wait for the DMA of the
    // next step; using the fragments here makes it wait once, here, where the Q loads
    // and step 0's DMA have been in flight together.
#pragma unroll
    for (int kc = 0; kc < NQF; ++kc) asm volatile("" ::"v"(qf[kc]));
    __syncthreads();
    if (n_steps > 1) PA_DMA_K(d_j1, 1);
    fc = flags_of(d0.code);
    PA_QK(sc0, sc1, 0);
    PA_QK_ORDER();
    PA_SHAPE(sc0, 0, 0, fc);
    PA_SHAPE(sc1, 0, 1, fc);
    float mx = -INFINITY;
    PA_BLOCK_MAX(mx, sc0);
    PA_BLOCK_MAX(mx, sc1);
    m_run = fmaxf(m_run, row_max(mx) * cexp);
    // iterations 0 .. n_steps - 2 (two per trip, so every slot offset is a constant)
    int j = 0;
    for (; j + 1 < n_steps; j += 2) {
      PA_ITER(j, 0);
      if (j + 2 >= n_steps) {
        j += 1;
        break;
      }
      PA_ITER(j + 1, 1);
    }
    // j = n_steps - 1 now (the loop leaves with j + 1 == n_steps)
    if (j & 1)
      PA_LAST(1);
    else
      PA_LAST(0);
    if (prev_dma) {
      // rows 0..63 sit in K slot P ^ 1, rows 64..127 in slot P (P = parity of the last step)
      dma_wait_all();
      __syncthreads();
      const int rr = (w & 1) * 32 + m;
      lds_cptr prow_l = lds + kKring + ((j & 1) ^ ((w >> 1) ^ 1)) * kSlot + rr * 256 + 8 * G;
#pragma unroll
      for (int q_ = 0; q_ < NDB * 4; ++q_)
        prevw[q_] = __builtin_bit_cast(uint2, *(const __attribute__((address_space(3))) u32x2*)(prow_l + 16 * (q_ ^ (rr & 15))));
    }
  } else {
    PA_PREV_LOAD();
  }

#undef PA_ITER
#undef PA_LAST
#undef PA_PREV_LOAD
#undef PA_PREV_LSE
#undef PA_SPLIT_WAIT
#undef PA_FAST_ORDER
#undef PA_PV
#undef PA_EXP
#undef PA_RAISE
#undef PA_BLOCK_MAX
#undef PA_MASK
#undef PA_SHAPE
#undef PA_QK_ORDER
#undef PA_QK
#undef PA_DMA_V
#undef PA_DMA_K
#undef PA_DMA_PREV
#undef PA_SEG_ROW

  // ---- epilogue (as attn_fwd_kernel) -------------------------------------------
  const float l_tot = row_sum(l_part);
  const bool has = l_tot > 0.f;
  float lse_v = has ? (m_run + log2f(l_tot)) * kLn2 : -INFINITY;
  float a_own = has ? 1.f / l_tot : 0.f;
  float a_prev = 0.f;
  if (prev_o) {
    const float lp = prev_lse;
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
  // The output rows go through LDS (the V ring, 8 KB per wave, swizzled as K) and leave as
  // whole rows: 16 bytes per lane, four full rows per store instruction.
  __syncthreads();  // every wave is past its last read of the V ring
  lds_char_t* stage = (lds_char_t*)smem + kVring + w * 8192;
  typedef __attribute__((address_space(3))) u32x2 lds_w2;
  const int psz = a.prev_dtype == PA_F32 ? 4 : 2;
  const char* prow = prev_o ? prev_o + (bh * a.prev_sb + (int64_t)srow * a.prev_sn) * psz : nullptr;
#pragma unroll
  for (int db = 0; db < NDB; ++db) {
#pragma unroll
    for (int i4 = 0; i4 < 4; ++i4) {
      const int d0 = 32 * db + 8 * i4 + 4 * G;
      f32x4 x = {acc[db][4 * i4], acc[db][4 * i4 + 1], acc[db][4 * i4 + 2], acc[db][4 * i4 + 3]};
      x *= a_own;
      if (prow && a_prev != 0.f) {
        if (prev16) {
          const uint2 pw = prevw[4 * db + i4];
          const f32x4 pvv = a.prev_dtype == PA_BF16
                                ? __builtin_convertvector(__builtin_bit_cast(bf16x4, pw), f32x4)
                                : __builtin_convertvector(__builtin_bit_cast(f16x4, pw), f32x4);
          x += a_prev * pvv;
        } else {
          x += a_prev * load4_any(prow + d0 * psz, a.prev_dtype);
        }
      }
      *(lds_w2*)(stage + m * 256 + 16 * ((4 * db + i4) ^ (m & 15)) + 8 * G) =
          __builtin_bit_cast(u32x2, Mma<T>::cvt4(x));
    }
  }
  if (a.lse && G == 0) {
    float* lo_ = a.lse + bh * a.lse_sb + srow;
    if (signal)
      __hip_atomic_store(lo_, lse_v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    else
      *lo_ = lse_v;
  }
  // (each wave reads back only the rows it wrote: LDS keeps a wave's accesses in order)
  if constexpr (BASIS != 0) {
    const int r0 = qb * 128 + w * 32 + (lane >> 4);
    const int s0 = BASIS == 2 ? (r0 & rmask) * res_s + (r0 >> res_q) : r0;
    char* dst0 = a.o + (bh * a.o_sb + (int64_t)s0 * a.o_sn) * ESZ + 16 * (lane & 15);
    const int64_t step_b = (int64_t)4 * (BASIS == 2 ? res_s : 1) * a.o_sn * ESZ;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int rr = 4 * i + (lane >> 4);
      const u32x4 v = *(lds_u4*)(stage + rr * 256 + 16 * ((lane & 15) ^ (rr & 15)));
      *reinterpret_cast<u32x4*>(dst0 + i * step_b) = v;
    }
  } else {
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int rr = 4 * i + (lane >> 4);
      const u32x4 v = *(lds_u4*)(stage + rr * 256 + 16 * ((lane & 15) ^ (rr & 15)));
      const int r_ = qb * 128 + w * 32 + rr;
      const int s_ = (sc_o && has_pq) ? (closed ? (r_ & rmask) * res_s + (r_ >> res_q) : a.pred.perm_q[r_]) : r_;
      char* dst_ = a.o + (bh * a.o_sb + (int64_t)s_ * a.o_sn) * ESZ + 16 * (lane & 15);
      if (signal)
        store_x4_sc1(dst_, v.x, v.y, v.z, v.w);
      else
        *reinterpret_cast<u32x4*>(dst_) = v;
    }
  }
  if constexpr (SPLIT) {
    if (signal) {
      // the rows are complete in memory before the group counts them
      __builtin_amdgcn_s_waitcnt(0);
      __syncthreads();
      if (tid == 0) __hip_atomic_fetch_add(a.run_sync + sg, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    } else if (tid == 0) {
      // the last merge of the group zeroes both counters for the next launch
      const int done = __hip_atomic_fetch_add(a.run_sync + a.run_sync_groups + sg, 1, __ATOMIC_RELAXED,
                                              __HIP_MEMORY_SCOPE_AGENT);
      if (done == a.run_sync_wait - 1) {
        __hip_atomic_store(a.run_sync + sg, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __hip_atomic_store(a.run_sync + a.run_sync_groups + sg, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      }
    }
  }
}

}  // namespace pa
