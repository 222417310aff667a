// Persistent streaming attention forward for gfx950: f16 / bf16, D = 128, BQ = 128.
//
// The same per-step work as attn_stream_kernel (K / V by LDS DMA into two-slot rings,
// 32x32x16 MFMAs on S^T = K Q^T, masking from bitmaps, lazy rescale), but a work-group
// is not one (query block, head) item: it is one of a fixed number of work-groups (two
// per CU) and runs a precomputed list of items back to back as ONE stream of steps
// (pa_index_run).  Each run row is a step descriptor that also names its item (head,
// query block, piece) and whether it is the item's first or last step, with its K / V
// rows given as rows of the whole [BH, N] tensor.  So the software pipeline never
// drains between items:
//
//  * the DMA of the next item's first K / V tiles is issued while the current item's
//    last steps run, exactly as for any other step two iterations ahead;
//  * the next item's Q rows are loaded into the Q fragments right after the current
//    item's last QK has consumed them, one iteration before the next item's first QK;
//  * the current item's epilogue (row sum, log-sum-exp, merge with a previous partial,
//    output store) runs after its last P.V, beside the next item's first scores.
//
// A run may hold the items of two pieces of a disjoint split (a band in the identity
// basis and a lattice in a residue basis, say), so that one launch computes the whole
// forward and the second piece finds the first piece's output, its query rows and much
// of its K / V in the L2 / memory-side cache instead of re-reading them from HBM.  An
// item of the second piece merges into the rows the first piece wrote, so it waits for
// them: the rows of a query block of one piece are covered by `run_sync_signal` query
// blocks of the other (one sync group), the first piece's items publish their rows and
// count themselves in the group, and the second piece's items wait for the count before
// their epilogue reads those rows.  The published rows are written and read with
// agent-scope (sc1) accesses and the count with agent-scope atomics, so the handshake
// holds whichever XCD the two items run on.  The schedule orders every item after the
// items it waits for in each work-group's list, and the launch is cooperative (every
// work-group resident), so every wait ends; a wait is also bounded, and one that gives
// up sets *run_status for the host to report.  The last waiter of a group resets both
// of its counters, so they are zero again for the next launch.
#pragma once

#include "attn_stream.hpp"

namespace pa {

// word 9 of a run row: bit 0 = the item's first step, bit 1 = its last step, bit 2 = the
// piece, the item's query block in the bits above; word 10: the item's batch-head;
// word 11: the item's sync group (-1: none)
constexpr int kRunFirst = 1;
constexpr int kRunLast = 2;
constexpr int kRunPiece = 4;
constexpr int kRunQbShift = 3;
// polls of a sync counter before a merge gives up (each poll sleeps ~0.4 us); every wait is
// bounded on its own, so a *run_status left set by an earlier launch (cleared only by the
// host, with the counters) does not shorten this launch's waits
constexpr int kRunMaxPolls = 1 << 20;

template <typename T>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2)))
void attn_run_kernel(const AttnK a) {
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

  typedef const __attribute__((address_space(4))) int32_t cint;
  const int32_t s_begin = ((cint*)a.run_start)[blockIdx.x];
  const int n_steps = ((cint*)a.run_start)[blockIdx.x + 1] - s_begin;
  if (n_steps <= 0) return;
  const StepDesc* desc = reinterpret_cast<const StepDesc*>(a.run_steps) + s_begin;
  const int A = a.A;

  // run rows hold K / V rows of the whole tensor (head offset included; 32-bit byte
  // offsets, checked on the host)
  const char* kbase = a.k;
  const char* vbase = a.v;
  const uint32_t krow_b32 = (uint32_t)(a.k_sn * ESZ), vrow_b32 = (uint32_t)(a.v_sn * ESZ);
  const char* bits = reinterpret_cast<const char*>(a.kv_bits);
  const int wpr = (A + 31) >> 5;

  // ---- DMA geometry (loop invariant; as attn_stream_kernel, for each piece's basis:
  // a gathered piece's 16-row segment is 16 rows s apart in memory) -------------------
  const int rs = 4 * w + (lane >> 4);
  const int pu = lane & 15;
  const int rstr0 = (a.run_flags[0] & kPieceGatherKV) ? a.run_res[0] : 1;
  const int rstr1 = (a.run_flags[1] & kPieceGatherKV) ? a.run_res[1] : 1;
  const uint32_t k_goff0 = (uint32_t)(rs * rstr0) * krow_b32 + 16u * (uint32_t)(pu ^ rs);
  const uint32_t v_goff0 = (uint32_t)(rs * rstr0) * vrow_b32 + 16u * (uint32_t)(pu ^ (4 * (rs & 3)));
  const uint32_t k_goff1 = (uint32_t)(rs * rstr1) * krow_b32 + 16u * (uint32_t)(pu ^ rs);
  const uint32_t v_goff1 = (uint32_t)(rs * rstr1) * vrow_b32 + 16u * (uint32_t)(pu ^ (4 * (rs & 3)));
  const uint32_t b_goff = A >= 32 ? (uint32_t)((64 * (w & 1) + lane) * wpr * 4) : (uint32_t)(lane * 4);

  // ---- LDS read geometry ---------------------------------------------------------
  lds_cptr lds = (lds_cptr)smem;
  lds_cptr kptr[NQF];
#pragma unroll
  for (int kc = 0; kc < NQF; ++kc) {
    kptr[kc] = lds + kKring + m * 256 + 16 * ((2 * kc + G) ^ (m & 15));
    asm volatile("" : "+v"(kptr[kc]));
  }
  const int j16 = lane & 15;
  const int h16 = (lane >> 4) & 1;
  lds_cptr vptr[NDB];
#pragma unroll
  for (int db = 0; db < NDB; ++db) {
    vptr[db] = lds + kVring + (4 * G + (j16 >> 2)) * 256 +
               16 * ((4 * db + 2 * h16 + ((j16 & 3) >> 1)) ^ (4 * (j16 >> 2))) + 8 * (j16 & 1);
    asm volatile("" : "+v"(vptr[db]));
  }
  lds_cptr bptr = lds + kBits + (w * 32 + m) * 4;
  asm volatile("" : "+v"(bptr));

  // original row of index-space row r_idx in piece pc's basis
  auto q_orig_of = [&](int pc, int r_idx) __attribute__((always_inline)) -> int {
    const int s = a.run_res[pc];
    return s ? (r_idx & ((1 << a.run_qlog2[pc]) - 1)) * s + (r_idx >> a.run_qlog2[pc]) : r_idx;
  };

  // ---- Q fragments (B operand of S^T = K Q^T) of item (bh, qb) of piece pc ---------
  Frag qf[NQF];
  auto load_q = [&](int pc, int bh, int qb) __attribute__((always_inline)) {
    const int r_idx = qb * 128 + w * 32 + m;
    const int r_load = (a.run_flags[pc] & kPieceGatherQ) ? q_orig_of(pc, r_idx) : r_idx;
    const char* qrow = a.q + ((int64_t)bh * a.q_sb + (int64_t)r_load * a.q_sn) * ESZ;
#pragma unroll
    for (int kc = 0; kc < NQF; ++kc)
      qf[kc] = __builtin_bit_cast(Frag, *reinterpret_cast<const uint4*>(qrow + (16 * kc + 8 * G) * ESZ));
  };

  f32x16 acc[NDB];
#pragma unroll
  for (int i = 0; i < NDB; ++i) acc[i] = f32x16{0};
  float m_run = kSentinel;
  float l_part = 0.f;
  const float cexp = a.c;

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
    r.pad[0] = c[9];   // flags | piece | qb << 3
    r.pad[1] = c[10];  // bh
    r.pad[2] = c[11];  // sync group
    return r;
  };
  // Inside the step loop a run row is one vector load (lane l reads word l % 16), unpacked
  // with v_readlane after the next iteration's vmcnt(0) wait: a scalar load there would
  // share lgkmcnt with the LDS reads of the MFMA block and, returning out of order, make
  // its first LDS wait an lgkmcnt(0) that stalls on the row (a miss: each row is read once).
  const int lane16 = lane & 15;
  auto load_desc_v = [&](int jd) __attribute__((always_inline)) -> int32_t {
    return reinterpret_cast<const int32_t*>(desc + jd)[lane16];
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
    r.pad[0] = __builtin_amdgcn_readlane(dv, 9);
    r.pad[1] = __builtin_amdgcn_readlane(dv, 10);
    r.pad[2] = __builtin_amdgcn_readlane(dv, 11);
    return r;
  };
  struct Flags {
    uint32_t live, full;
  };
  auto flags_of = [&](uint32_t code) __attribute__((always_inline)) -> Flags {
    const uint32_t cw = code >> (2 * w);
    return Flags{(cw & 1u) | ((cw >> 7) & 2u) | ((cw >> 14) & 4u) | ((cw >> 21) & 8u),
                 ((cw >> 1) & 1u) | ((cw >> 8) & 2u) | ((cw >> 15) & 4u) | ((cw >> 22) & 8u)};
  };

#include "attn_stream_ops.inc"

  // ---- epilogue of item (bh, qb) of piece pc: normalise, merge with the previous
  // partial, store; in a split run, publish the rows (first piece) or wait for them
  // (second piece).  Every previous-partial element is loaded before the first store
  // (the output may be the previous partial itself: the merge is in place, each lane
  // rewriting what it read).  Row pointers include the lane's column offset 4 G, so every
  // column below is an immediate offset: no per-column address stays live across items.
  const bool prev16 = a.prev_o && a.prev_dtype != PA_F32;
  auto finish = [&](int pc, int bh, int qb, int sg, int SL) __attribute__((always_inline)) {
    const int flags = a.run_flags[pc];
    const bool merge = (flags & kPieceMerge) != 0;
    const bool signal = a.run_sync && sg >= 0 && !merge;   // publishes rows another piece merges into
    const bool waits = a.run_sync && sg >= 0 && merge;     // merges into rows another item publishes
    const int r_idx = qb * 128 + w * 32 + m;
    const int srow = (flags & kPieceScatterO) ? q_orig_of(pc, r_idx) : r_idx;
    const float l_tot = row_sum(l_part);
    const bool has = l_tot > 0.f;
    float lse_v = has ? (m_run + log2f(l_tot)) * kLn2 : -INFINITY;
    float a_own = has ? 1.f / l_tot : 0.f;
    float a_prev = 0.f;
    if (waits) {
      // every item of the other piece that covers these rows has published them
      if (tid == 0) {
        int polls = 0;
        while (__hip_atomic_load(a.run_sync + sg, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) < a.run_sync_signal) {
          if (++polls >= kRunMaxPolls) {
            __hip_atomic_store(a.run_status, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            break;
          }
          __builtin_amdgcn_s_sleep(16);
        }
      }
      __syncthreads();
    }
    uint2 prevw[NDB * 4];
    const int psz = prev16 ? 2 : 4;
    const char* prow = merge ? a.prev_o + ((int64_t)bh * a.prev_sb + (int64_t)srow * a.prev_sn + 4 * G) * psz : nullptr;
    if (merge) {
      const float* lp_at = a.prev_lse + (int64_t)bh * a.lse_sb + srow;
      const float lp = waits ? __hip_atomic_load(lp_at, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) : *lp_at;
      if (prev16) {
        if (waits) {
#pragma unroll
          for (int q_ = 0; q_ < NDB * 4; ++q_)
            prevw[q_] = __builtin_bit_cast(
                uint2, __hip_atomic_load(reinterpret_cast<const uint64_t*>(prow + (32 * (q_ >> 2) + 8 * (q_ & 3)) * 2),
                                         __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT));
        } else {
#pragma unroll
          for (int q_ = 0; q_ < NDB * 4; ++q_)
            prevw[q_] = *reinterpret_cast<const uint2*>(prow + (32 * (q_ >> 2) + 8 * (q_ & 3)) * 2);
        }
      }
      const float M = fmaxf(lse_v, lp);
      if (M == -INFINITY) {
        a_own = 0.f;
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
    // The output rows go through LDS and leave as whole rows, 16 bytes per lane and four
    // full rows per store instruction (no partial cache lines for the L2 to fill): wave w
    // stages its 32 rows (8 KB, 16-byte units swizzled as K) in the V slot this step's P.V
    // read (waves 0, 1) or the K slot its QK read (waves 2, 3), after every wave is past
    // those reads; the next DMA into them follows the next iteration's barrier.
    __syncthreads();
    lds_char_t* stage = (lds_char_t*)smem + (w < 2 ? kVring + SL * kSlot : kKring + (SL ^ 1) * kSlot) + (w & 1) * 8192;
    typedef __attribute__((address_space(3))) u32x2 lds_w2;
    // (lane terms made opaque here, so the staging addresses are computed per item
    // instead of being hoisted out of the step loop into registers)
    int mx16 = 16 * (m & 15), lx16 = 16 * (lane & 15), rq = lane >> 4;
    asm volatile("" : "+v"(mx16), "+v"(lx16), "+v"(rq));
#pragma unroll
    for (int db = 0; db < NDB; ++db) {
#pragma unroll
      for (int i4 = 0; i4 < 4; ++i4) {
        f32x4 x = {acc[db][4 * i4], acc[db][4 * i4 + 1], acc[db][4 * i4 + 2], acc[db][4 * i4 + 3]};
        x *= a_own;
        if (a_prev != 0.f) {
          if (prev16) {
            const uint2 pw = prevw[4 * db + i4];
            const f32x4 pvv = a.prev_dtype == PA_BF16
                                  ? __builtin_convertvector(__builtin_bit_cast(bf16x4, pw), f32x4)
                                  : __builtin_convertvector(__builtin_bit_cast(f16x4, pw), f32x4);
            x += a_prev * pvv;
          } else {
            x += a_prev * load4_any(prow + (32 * db + 8 * i4) * 4, PA_F32);
          }
        }
        *(lds_w2*)(stage + m * 256 + ((16 * (4 * db + i4)) ^ mx16) + 8 * G) =
            __builtin_bit_cast(u32x2, Mma<T>::cvt4(x));
      }
    }
    // (each wave reads back only the rows it wrote: LDS keeps a wave's accesses in order)
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int rr = 4 * i + rq;
      const u32x4 v = *(lds_u4*)(stage + rr * 256 + (lx16 ^ (16 * (rr & 15))));
      const int r_ = qb * 128 + w * 32 + rr;
      const int s_ = (flags & kPieceScatterO) ? q_orig_of(pc, r_) : r_;
      char* dst = a.o + ((int64_t)bh * a.o_sb + (int64_t)s_ * a.o_sn) * ESZ + lx16;
      if (signal) {
        __hip_atomic_store(reinterpret_cast<uint64_t*>(dst), (uint64_t)v.x | ((uint64_t)v.y << 32), __ATOMIC_RELAXED,
                           __HIP_MEMORY_SCOPE_AGENT);
        __hip_atomic_store(reinterpret_cast<uint64_t*>(dst + 8), (uint64_t)v.z | ((uint64_t)v.w << 32),
                           __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      } else {
        *reinterpret_cast<u32x4*>(dst) = v;
      }
    }
    if (a.lse && G == 0) {
      float* lo = a.lse + (int64_t)bh * a.lse_sb + srow;
      if (signal)
        __hip_atomic_store(lo, lse_v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      else
        *lo = lse_v;
    }
    if (signal) {
      // the rows are complete in memory before the group counts them
      __builtin_amdgcn_s_waitcnt(0);
      __syncthreads();
      if (tid == 0) __hip_atomic_fetch_add(a.run_sync + sg, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    } else if (waits && tid == 0) {
      // the last of the group's merges resets both counters for the next launch
      const int done = __hip_atomic_fetch_add(a.run_sync + a.run_sync_groups + sg, 1, __ATOMIC_RELAXED,
                                              __HIP_MEMORY_SCOPE_AGENT);
      if (done == a.run_sync_wait - 1) {
        __hip_atomic_store(a.run_sync + sg, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __hip_atomic_store(a.run_sync + a.run_sync_groups + sg, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      }
    }
#pragma unroll
    for (int i = 0; i < NDB; ++i) acc[i] = f32x16{0};
    m_run = kSentinel;
    l_part = 0.f;
  };

  // One iteration jj (P = jj & 1), for jj + 1 < n_steps: as attn_stream_kernel's, plus
  // the item boundaries: after the MFMA block, the epilogue of the item whose last step
  // is jj, and the Q rows of the item that starts at jj + 2 when jj + 1 ends an item
  // (QK of jj + 1 was the last use of the fragments).  The uses of the Q fragments right
  // after the wait make the compiler place its own wait for Q there, before this
  // iteration's DMA is issued (a wait at the QK would also wait for that DMA).  Each
  // step's DMA takes the row offsets of its piece's basis.
#define PA_RITER(jj, P)                                                                           \
  do {                                                                                            \
    dma_wait_all();                                                                               \
    _Pragma("unroll") for (int kc = 0; kc < NQF; ++kc) asm volatile("" ::"v"(qf[kc]));             \
    __syncthreads();                                                                              \
    if ((jj) + 2 < n_steps) {                                                                     \
      d_j2 = unpack_desc(dv_j2);                                                                  \
      const uint32_t k_goff = (d_j2.pad[0] & kRunPiece) ? k_goff1 : k_goff0;                      \
      PA_DMA_K(d_j2, (P));                                                                        \
    }                                                                                             \
    {                                                                                             \
      const uint32_t v_goff = (d_j1.pad[0] & kRunPiece) ? v_goff1 : v_goff0;                      \
      PA_DMA_V(d_j1, (P) ^ 1);                                                                    \
    }                                                                                             \
    if ((jj) + 3 < n_steps) dv_j2 = load_desc_v((jj) + 3);                                        \
    const Flags fn = flags_of(d_j1.code);                                                         \
    const int fl_n = d_j1.pad[0];                                                                 \
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
    if (fl_c & kRunLast) {                                                                        \
      finish((fl_c >> 2) & 1, cur_bh, cur_qb, cur_sg, (P));                                       \
      cur_bh = d_j1.pad[1];                                                                       \
      cur_qb = fl_n >> kRunQbShift;                                                               \
      cur_sg = d_j1.pad[2];                                                                       \
    }                                                                                             \
    if ((fl_n & kRunLast) && (jj) + 2 < n_steps)                                                  \
      load_q((d_j2.pad[0] >> 2) & 1, d_j2.pad[1], d_j2.pad[0] >> kRunQbShift);                    \
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
    fl_c = fl_n;                                                                                  \
    d_j1 = d_j2;                                                                                  \
  } while (0)

  // The last step of the run: its V (slot P) arrives, then its softmax and P.V.
#define PA_RLAST(P)                                                                               \
  do {                                                                                            \
    dma_wait_all();                                                                               \
    __syncthreads();                                                                              \
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

  // Prologue: the first item's Q, step 0's K, bitmaps and V, then step 1's K; QK, shaping
  // and maximum of step 0.
  // d_j1 / d_j2: run rows of the steps one and two ahead; dv_j2: the raw row (one word per
  // lane) that becomes d_j2 at the top of the next iteration
  StepDesc d_j1{}, d_j2{};
  int32_t dv_j2 = 0;
  Flags fc{0u, 0u};
  int fl_c;
  int cur_bh, cur_qb, cur_sg;
  f32x16 sc0, sc1;
  {
    const StepDesc d0 = load_desc(0);
    if (n_steps > 1) d_j1 = load_desc(1);
    if (n_steps > 2) dv_j2 = load_desc_v(2);
    cur_bh = d0.pad[1];
    cur_qb = d0.pad[0] >> kRunQbShift;
    cur_sg = d0.pad[2];
    fl_c = d0.pad[0];
    load_q((fl_c >> 2) & 1, cur_bh, cur_qb);
    {
      const uint32_t k_goff = (d0.pad[0] & kRunPiece) ? k_goff1 : k_goff0;
      const uint32_t v_goff = (d0.pad[0] & kRunPiece) ? v_goff1 : v_goff0;
      PA_DMA_K(d0, 0);
      PA_DMA_V(d0, 0);
    }
    dma_wait_all();
#pragma unroll
    for (int kc = 0; kc < NQF; ++kc) asm volatile("" ::"v"(qf[kc]));
    __syncthreads();
    if (n_steps > 1) {
      const uint32_t k_goff = (d_j1.pad[0] & kRunPiece) ? k_goff1 : k_goff0;
      PA_DMA_K(d_j1, 1);
    }
    fc = flags_of(d0.code);
    PA_QK(sc0, sc1, 0);
    PA_QK_ORDER();
    PA_SHAPE(sc0, 0, 0, fc);
    PA_SHAPE(sc1, 0, 1, fc);
    float mx = -INFINITY;
    PA_BLOCK_MAX(mx, sc0);
    PA_BLOCK_MAX(mx, sc1);
    m_run = fmaxf(m_run, row_max(mx) * cexp);
    if (n_steps > 1 && (fl_c & kRunLast))
      load_q((d_j1.pad[0] >> 2) & 1, d_j1.pad[1], d_j1.pad[0] >> kRunQbShift);
  }
  // iterations 0 .. n_steps - 2 (two per trip, so every slot offset is a constant)
  int j = 0;
  for (; j + 1 < n_steps; j += 2) {
    PA_RITER(j, 0);
    if (j + 2 >= n_steps) {
      j += 1;
      break;
    }
    PA_RITER(j + 1, 1);
  }
  if (j & 1) {
    PA_RLAST(1);
    finish((fl_c >> 2) & 1, cur_bh, cur_qb, cur_sg, 1);
  } else {
    PA_RLAST(0);
    finish((fl_c >> 2) & 1, cur_bh, cur_qb, cur_sg, 0);
  }

#undef PA_RITER
#undef PA_RLAST
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
#undef PA_SEG_ROW
}

}  // namespace pa
