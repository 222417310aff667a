// Block-index builder on the GPU: mask predicate -> per-query-block lists of live
// KV tiles.  Replaces gpu/blockindex.py:32-51 (build), which materialises the N x N
// mask on the host and tiles it with numpy any/all.
//
// Phase 1 (classify): work-groups (query block, column split) walk the KV columns in
// chunks of 256 (split j takes chunks j, j + splits, ...), evaluate the predicate for
// the block's BQ rows and fold the result into per-tile codes: 2 bits (some live / all
// live) per wave group of 32 query rows x min(A, 32) columns.  Wave ballots do the
// column reduction; a query block's list length is summed over its splits.
// Phase 2 (compact): one work-group per query block scans the tile codes and
// writes the ascending, zero-padded kv_idx / kv_partial / kv_wave_bits rows.
#include "common.hpp"

namespace pa {
namespace {

constexpr int kThreads = 256;
constexpr int kChunk = 256;  // columns per pass, one per thread

__global__ void zero_totals_kernel(unsigned long long* totals, int32_t* kv_num, int32_t nq) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i < 3) totals[i] = 0ull;
  if (i < nq) kv_num[i] = 0;
}

// The longest list, once every split has added its count.
__global__ void max_list_kernel(const int32_t* kv_num, int32_t nq, unsigned long long* totals) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  int32_t v = i < nq ? kv_num[i] : 0;
  for (int off = 32; off > 0; off >>= 1) v = max(v, __shfl_down(v, off, 64));
  if ((threadIdx.x & 63) == 0 && v > 0) atomicMax(&totals[2], (unsigned long long)v);
}

__global__ __launch_bounds__(kThreads) void classify_kernel(const Pred pred, int32_t N, int32_t BQ,
                                                             int32_t A, uint32_t* __restrict__ codes,
                                                             int32_t* __restrict__ kv_num,
                                                             unsigned long long* __restrict__ totals) {
  __shared__ int32_t q_orig[128];
  __shared__ uint32_t tile_code[kChunk / 16];
  __shared__ int32_t red_live[kThreads / 64];
  __shared__ int32_t red_tiles;

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int qb = blockIdx.x;
  const int split = blockIdx.y, splits = gridDim.y;
  const int nk = N / A;
  const int rg_rows = BQ < 32 ? BQ : 32;   // rows per wave group
  const int n_rg = BQ / rg_rows;
  const int cw = A < 32 ? A : 32;          // columns per wave group
  const int ncg = A / cw;

  if (tid < BQ) {
    const int r = qb * BQ + tid;
    q_orig[tid] = pred.perm_q ? pred.perm_q[r] : r;
  }
  if (tid == 0) red_tiles = 0;
  __syncthreads();

  int32_t live_count = 0;
  int32_t tiles_listed = 0;  // meaningful in thread 0 only

  for (int c0 = split * kChunk; c0 < N; c0 += splits * kChunk) {
    if (tid < kChunk / 16) tile_code[tid] = 0u;
    __syncthreads();

    const int col = c0 + tid;
    const bool valid = col < N;
    uint32_t any_rg = 0u, all_rg = 0u;
    if (valid) {
      const int32_t ko = pred.perm_kv ? pred.perm_kv[col] : col;
      for (int g = 0; g < n_rg; ++g) {
        bool any = false, all = true;
        for (int rr = 0; rr < rg_rows; ++rr) {
          const bool live = pred_live(pred, q_orig[g * rg_rows + rr], ko);
          any |= live;
          all &= live;
          live_count += live ? 1 : 0;
        }
        any_rg |= (any ? 1u : 0u) << g;
        all_rg |= (all ? 1u : 0u) << g;
      }
    }
    // Column reduction inside each wave: a column group never straddles a wave.
    const int wave_col0 = c0 + wave * 64;
    for (int g = 0; g < n_rg; ++g) {
      const unsigned long long b_any = __ballot((any_rg >> g) & 1u);
      const unsigned long long b_all = __ballot((all_rg >> g) & 1u);
      const int ngroups_in_wave = 64 / cw;
      if (lane < ngroups_in_wave) {
        const int gc0 = wave_col0 + lane * cw;  // first column of this column group
        if (gc0 < N) {
          const unsigned long long gm = (cw == 64 ? ~0ull : ((1ull << cw) - 1ull)) << (lane * cw);
          const bool gany = (b_any & gm) != 0ull;
          const bool gall = (b_all & gm) == gm;
          const int cg = (gc0 % A) / cw;
          const int code_g = g * ncg + cg;
          const uint32_t bits = (gany ? 1u : 0u) << (2 * code_g) | (gall ? 1u : 0u) << (2 * code_g + 1);
          if (bits) atomicOr(&tile_code[(gc0 - c0) / A], bits);
        }
      }
    }
    __syncthreads();
    const int tiles_in_chunk = kChunk / A;
    if (tid < tiles_in_chunk) {
      const int kb = c0 / A + tid;
      if (kb < nk) {
        const uint32_t code = tile_code[tid];
        codes[(int64_t)qb * nk + kb] = code;
        if (code & 0x55555555u) atomicAdd(&red_tiles, 1);
      }
    }
    __syncthreads();
  }

  // live pairs: wave reduce, then one atomic per work-group
  for (int off = 32; off > 0; off >>= 1) live_count += __shfl_down(live_count, off, 64);
  if (lane == 0) red_live[wave] = live_count;
  __syncthreads();
  if (tid == 0) {
    long long tot = 0;
    for (int i = 0; i < kThreads / 64; ++i) tot += red_live[i];
    tiles_listed = red_tiles;
    if (tiles_listed) {
      atomicAdd(&kv_num[qb], tiles_listed);
      atomicAdd(&totals[0], (unsigned long long)tiles_listed);
    }
    if (tot) atomicAdd(&totals[1], (unsigned long long)tot);
  }
}

__global__ __launch_bounds__(kThreads) void compact_kernel(const uint32_t* __restrict__ codes,
                                                            const int32_t* __restrict__ kv_num,
                                                            int32_t N, int32_t BQ, int32_t A,
                                                            uint32_t full_mask,
                                                            int32_t* __restrict__ kv_idx,
                                                            int8_t* __restrict__ kv_partial,
                                                            uint32_t* __restrict__ kv_wave_bits,
                                                            int64_t pitch) {
  __shared__ int32_t wave_tot[kThreads / 64];
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int qb = blockIdx.x;
  const int nk = N / A;
  const int64_t row = (int64_t)qb * pitch;
  int base = 0;
  for (int k0 = 0; k0 < nk; k0 += kThreads) {
    const int kb = k0 + tid;
    const uint32_t code = kb < nk ? codes[(int64_t)qb * nk + kb] : 0u;
    const bool listed = (code & 0x55555555u) != 0u;
    const unsigned long long bal = __ballot(listed);
    const int before_in_wave = __popcll(bal & ((1ull << lane) - 1ull));
    if (lane == 0) wave_tot[wave] = __popcll(bal);
    __syncthreads();
    int before = base + before_in_wave;
    int chunk_total = 0;
    for (int i = 0; i < kThreads / 64; ++i) {
      if (i < wave) before += wave_tot[i];
      chunk_total += wave_tot[i];
    }
    if (listed && before < pitch) {  // pitch >= kv_num is the caller's contract; never write past it
      kv_idx[row + before] = kb;
      kv_partial[row + before] = ((code & full_mask) == full_mask) ? 0 : 1;
      if (kv_wave_bits) kv_wave_bits[row + before] = code;
    }
    base += chunk_total;
    __syncthreads();
  }
  // zero padding up to the pitch (gpu/blockindex.py:44-45 allocates with np.zeros)
  const int n = kv_num[qb];
  for (int64_t j = n + tid; j < pitch; j += kThreads) {
    kv_idx[row + j] = 0;
    kv_partial[row + j] = 0;
    if (kv_wave_bits) kv_wave_bits[row + j] = 0u;
  }
}

bool tile_ok(int32_t x) { return x == 16 || x == 32 || x == 64 || x == 128; }

}  // namespace
}  // namespace pa

extern "C" int pa_index_classify(const pa_mask* mask, int64_t N, int32_t BQ, int32_t A,
                                 uint32_t* tile_codes, int32_t* kv_num, unsigned long long* totals,
                                 void* stream) {
  PA_CHECK_ARG(mask != nullptr && tile_codes && kv_num && totals, "pa_index_classify: null argument");
  PA_CHECK_ARG(N >= 1 && N <= (1ll << 30), "pa_index_classify: N=%lld out of range", (long long)N);
  PA_CHECK_ARG(pa::tile_ok(BQ) && pa::tile_ok(A),
               "pa_index_classify: BQ=%d A=%d must each be one of 16, 32, 64, 128", BQ, A);
  PA_CHECK_ARG(N % BQ == 0 && N % A == 0, "pa_index_classify: N=%lld not divisible by BQ=%d and A=%d",
               (long long)N, BQ, A);
  if (int rc = pa::check_mask(mask, N)) return rc;
  hipStream_t s = static_cast<hipStream_t>(stream);
  const pa::Pred pred = pa::make_pred(*mask);
  const int64_t nq = N / BQ;
  hipLaunchKernelGGL(pa::zero_totals_kernel, dim3((unsigned)((nq + 3 + 255) / 256)), dim3(256), 0, s, totals, kv_num,
                     (int32_t)nq);
  PA_LAUNCH_CHECK("zero_totals_kernel");
  // enough column splits for about 2048 work-groups (the chip holds ~2048 of 256 threads)
  const int64_t chunks = (N + pa::kChunk - 1) / pa::kChunk;
  int64_t splits = (2048 + nq - 1) / nq;
  if (splits > chunks) splits = chunks;
  if (splits < 1) splits = 1;
  hipLaunchKernelGGL(pa::classify_kernel, dim3((unsigned)nq, (unsigned)splits), dim3(pa::kThreads), 0, s, pred,
                     (int32_t)N, BQ, A, tile_codes, kv_num, totals);
  PA_LAUNCH_CHECK("classify_kernel");
  hipLaunchKernelGGL(pa::max_list_kernel, dim3((unsigned)((nq + 255) / 256)), dim3(256), 0, s, kv_num,
                     (int32_t)nq, totals);
  PA_LAUNCH_CHECK("max_list_kernel");
  return PA_OK;
}

extern "C" int pa_index_compact(const uint32_t* tile_codes, const int32_t* kv_num, int64_t N, int32_t BQ,
                                int32_t A, int32_t* kv_idx, int8_t* kv_partial, uint32_t* kv_wave_bits,
                                int64_t pitch, void* stream) {
  PA_CHECK_ARG(tile_codes && kv_num, "pa_index_compact: null argument");
  PA_CHECK_ARG(N >= 1 && N <= (1ll << 30), "pa_index_compact: N=%lld out of range", (long long)N);
  PA_CHECK_ARG(pa::tile_ok(BQ) && pa::tile_ok(A) && N % BQ == 0 && N % A == 0,
               "pa_index_compact: bad tile shape BQ=%d A=%d for N=%lld", BQ, A, (long long)N);
  PA_CHECK_ARG(pitch >= 0, "pa_index_compact: negative pitch");
  if (pitch == 0) return PA_OK;  // every query block is empty: nothing to write
  PA_CHECK_ARG(kv_idx && kv_partial, "pa_index_compact: null output");
  const int rg_rows = BQ < 32 ? BQ : 32;
  const int cw = A < 32 ? A : 32;
  const int ngroups = (BQ / rg_rows) * (A / cw);
  uint32_t full_mask = 0u;
  for (int g = 0; g < ngroups; ++g) full_mask |= 2u << (2 * g);
  hipStream_t s = static_cast<hipStream_t>(stream);
  hipLaunchKernelGGL(pa::compact_kernel, dim3((unsigned)(N / BQ)), dim3(pa::kThreads), 0, s, tile_codes,
                     kv_num, (int32_t)N, BQ, A, full_mask, kv_idx, kv_partial, kv_wave_bits, pitch);
  PA_LAUNCH_CHECK("compact_kernel");
  return PA_OK;
}

// ---------------------------------------------------------------------------
// Element bitmaps of the listed partial tiles (phase 3).  One work-group per query
// block walks its list; each partial tile gets BQ x ceil(A/32) words, one thread per
// word, 32 predicate evaluations per word.
namespace pa {
namespace {

__global__ __launch_bounds__(kThreads) void bits_kernel(const Pred pred, int32_t N, int32_t BQ, int32_t A,
                                                         const int32_t* __restrict__ kv_idx,
                                                         const int32_t* __restrict__ kv_num,
                                                         const int8_t* __restrict__ kv_partial, int64_t pitch,
                                                         const int64_t* __restrict__ part_base,
                                                         int32_t* __restrict__ kv_bits_off,
                                                         uint32_t* __restrict__ pool) {
  __shared__ int32_t q_orig[128];
  const int tid = threadIdx.x;
  const int qb = blockIdx.x;
  const int wpr = (A + 31) >> 5;
  const int words = BQ * wpr;
  if (tid < BQ) {
    const int r = qb * BQ + tid;
    q_orig[tid] = pred.perm_q ? pred.perm_q[r] : r;
  }
  __syncthreads();
  const int n = kv_num[qb];
  const int64_t row = (int64_t)qb * pitch;
  int64_t rank = part_base[qb];
  for (int j = 0; j < n; ++j) {
    const bool partial = kv_partial[row + j] != 0;
    if (tid == 0) kv_bits_off[row + j] = partial ? (int32_t)(rank * words) : -1;
    if (!partial) continue;
    const int kb = kv_idx[row + j];
    uint32_t* dst = pool + rank * words;
    for (int wi = tid; wi < words; wi += kThreads) {
      const int rr = wi / wpr, cw = wi % wpr;
      const int c0 = kb * A + cw * 32;
      const int ncol = A - cw * 32 < 32 ? A - cw * 32 : 32;
      uint32_t bits = 0u;
      for (int c = 0; c < ncol; ++c) {
        const int col = c0 + c;
        const int32_t ko = pred.perm_kv ? pred.perm_kv[col] : col;
        bits |= (pred_live(pred, q_orig[rr], ko) ? 1u : 0u) << c;
      }
      dst[wi] = bits;
    }
    ++rank;
  }
  for (int64_t j = n + tid; j < pitch; j += kThreads) kv_bits_off[row + j] = -1;
}

}  // namespace
}  // namespace pa

extern "C" int pa_index_bits(const pa_mask* mask, int64_t N, int32_t BQ, int32_t A, const int32_t* kv_idx,
                             const int32_t* kv_num, const int8_t* kv_partial, int64_t pitch,
                             const int64_t* part_base, int32_t* kv_bits_off, uint32_t* pool, void* stream) {
  PA_CHECK_ARG(mask && kv_num && part_base, "pa_index_bits: null argument");
  PA_CHECK_ARG(N >= 1 && N <= (1ll << 30), "pa_index_bits: N=%lld out of range", (long long)N);
  PA_CHECK_ARG(pa::tile_ok(BQ) && pa::tile_ok(A) && N % BQ == 0 && N % A == 0,
               "pa_index_bits: bad tile shape BQ=%d A=%d for N=%lld", BQ, A, (long long)N);
  if (pitch == 0) return PA_OK;
  PA_CHECK_ARG(kv_idx && kv_partial && kv_bits_off, "pa_index_bits: null list");
  if (int rc = pa::check_mask(mask, N)) return rc;
  const pa::Pred pred = pa::make_pred(*mask);
  hipLaunchKernelGGL(pa::bits_kernel, dim3((unsigned)(N / BQ)), dim3(pa::kThreads), 0,
                     static_cast<hipStream_t>(stream), pred, (int32_t)N, BQ, A, kv_idx, kv_num, kv_partial,
                     pitch, part_base, kv_bits_off, pool);
  PA_LAUNCH_CHECK("bits_kernel");
  return PA_OK;
}

// ---------------------------------------------------------------------------
// Step descriptors of the streaming attention kernel: one thread per (query block,
// step of 64 kv columns), 64 bytes out, written as four 16-byte stores.
namespace pa {
namespace {

__global__ __launch_bounds__(kThreads) void steps_kernel(const int32_t* __restrict__ kv_idx,
                                                          const int32_t* __restrict__ kv_num,
                                                          const int8_t* __restrict__ kv_partial,
                                                          const uint32_t* __restrict__ kv_wave_bits,
                                                          const int32_t* __restrict__ kv_bits_off, int64_t pitch,
                                                          int32_t nq, int32_t BQ, int32_t A, int32_t residue_s,
                                                          int32_t residue_qlog2, const int32_t* __restrict__ order,
                                                          int32_t* __restrict__ steps, int64_t steps_pitch) {
  const int64_t gid = (int64_t)blockIdx.x * kThreads + threadIdx.x;
  if (gid >= (int64_t)nq * steps_pitch) return;
  const int pos = (int)(gid / steps_pitch);  // issue position of the list
  const int qb = order ? order[pos] : pos;
  const int j = (int)(gid % steps_pitch);
  const int spt = A >> 4;                    // 16-column segments per tile
  const int n_seg = kv_num[qb] * spt;
  const int ncg = A >= 32 ? A >> 5 : 1;      // 32-column groups per tile
  const int ngr = BQ >= 32 ? BQ >> 5 : 1;    // 32-row groups per query block
  int32_t d[16];
#pragma unroll
  for (int i = 0; i < 16; ++i) d[i] = 0;
  uint32_t code = 0u;
#pragma unroll
  for (int t = 0; t < 4; ++t) {
    const int seg = 4 * j + t;
    int32_t base = 0, boff = -1;
    uint32_t c8 = 0u;
    if (seg < n_seg) {
      const int64_t ti = (int64_t)qb * pitch + seg / spt;
      const int within = seg % spt;
      base = kv_idx[ti] * A + within * 16;
      if (residue_s > 0) {
        const int32_t rmask = (1 << residue_qlog2) - 1;
        base = (base & rmask) * residue_s + (base >> residue_qlog2);
      }
      if (kv_wave_bits) {
        const int cg = A >= 32 ? within >> 1 : 0;
        const uint32_t wb = kv_wave_bits[ti];
        for (int g = 0; g < ngr && g < 4; ++g) c8 |= ((wb >> (2 * (g * ncg + cg))) & 3u) << (2 * g);
      } else {
        c8 = kv_partial[ti] ? 0x55u : 0xffu;
      }
      if (kv_bits_off && kv_bits_off[ti] >= 0) boff = kv_bits_off[ti] + ((within * 16) >> 5);
    }
    d[t] = base;
    d[5 + t] = boff;
    code |= c8 << (8 * t);
  }
  d[4] = (int32_t)code;
  d[13] = qb;
  d[14] = (kv_num[qb] * A + 63) >> 6;
  d[15] = residue_s > 0 ? residue_s : 0;
  int4* dst = reinterpret_cast<int4*>(steps + gid * 16);
#pragma unroll
  for (int i = 0; i < 4; ++i) dst[i] = int4{d[4 * i], d[4 * i + 1], d[4 * i + 2], d[4 * i + 3]};
}

}  // namespace
}  // namespace pa

extern "C" int pa_index_steps(const int32_t* kv_idx, const int32_t* kv_num, const int8_t* kv_partial,
                              const uint32_t* kv_wave_bits, const int32_t* kv_bits_off, int64_t pitch, int64_t N,
                              int32_t BQ, int32_t A, int32_t residue_s, int32_t residue_qlog2,
                              const int32_t* order, int32_t* steps, int64_t steps_pitch, void* stream) {
  PA_CHECK_ARG(kv_num, "pa_index_steps: null kv_num");
  PA_CHECK_ARG(N >= 1 && N <= (1ll << 30), "pa_index_steps: N=%lld out of range", (long long)N);
  PA_CHECK_ARG(pa::tile_ok(BQ) && pa::tile_ok(A) && N % BQ == 0 && N % A == 0,
               "pa_index_steps: bad tile shape BQ=%d A=%d for N=%lld", BQ, A, (long long)N);
  PA_CHECK_ARG(pitch >= 0, "pa_index_steps: negative pitch");
  PA_CHECK_ARG(residue_s <= 0 || (residue_qlog2 >= 4 && residue_qlog2 < 31 &&
                                  (int64_t)residue_s << residue_qlog2 == N),
               "pa_index_steps: residue_s=%d with N/s = 2^%d does not match N=%lld", residue_s, residue_qlog2,
               (long long)N);
  PA_CHECK_ARG(steps_pitch >= (pitch * A + 63) / 64,
               "pa_index_steps: steps_pitch=%lld < ceil(pitch * A / 64) = %lld", (long long)steps_pitch,
               (long long)((pitch * A + 63) / 64));
  const int64_t nq = N / BQ;
  const int64_t total = nq * steps_pitch;
  if (total == 0) return PA_OK;
  PA_CHECK_ARG(steps, "pa_index_steps: null steps");
  PA_CHECK_ARG(pitch == 0 || (kv_idx && kv_partial), "pa_index_steps: null list");
  PA_CHECK_ARG((reinterpret_cast<uintptr_t>(steps) & 15) == 0, "pa_index_steps: steps must be 16-byte aligned");
  PA_CHECK_ARG(total / pa::kThreads < 0x7fffffffll, "pa_index_steps: too many steps");
  hipLaunchKernelGGL(pa::steps_kernel, dim3((unsigned)((total + pa::kThreads - 1) / pa::kThreads)),
                     dim3(pa::kThreads), 0, static_cast<hipStream_t>(stream), kv_idx, kv_num, kv_partial,
                     kv_wave_bits, kv_bits_off, pitch, (int32_t)nq, BQ, A, residue_s > 0 ? residue_s : 0,
                     residue_qlog2, order, steps, steps_pitch);
  PA_LAUNCH_CHECK("steps_kernel");
  return PA_OK;
}

namespace pa {
namespace {

// One work-group of 64 threads per item: its run rows are its list's steps (from the
// descriptors of its piece) with the K / V rows moved to the item's head, the bitmap
// offsets moved to the piece's part of a shared pool, and the item written into words
// 9 to 11.
struct RunPieces {
  const int32_t* steps[2];
  int64_t pitch[2];
  int32_t boff_base[2];
};

__global__ __launch_bounds__(64) void run_kernel(const RunPieces pcs, int64_t N, const int32_t* __restrict__ item_piece,
                                                 const int32_t* __restrict__ item_bh,
                                                 const int32_t* __restrict__ item_qb,
                                                 const int32_t* __restrict__ item_sync,
                                                 const int32_t* __restrict__ item_off, int32_t* __restrict__ run) {
  const int i = blockIdx.x;
  const int pc = item_piece ? item_piece[i] : 0;
  const int32_t bh = item_bh[i], qb = item_qb[i];
  const int32_t sg = item_sync ? item_sync[i] : -1;
  const int32_t r0 = item_off[i], len = item_off[i + 1] - r0;
  const int32_t* list = (pc ? pcs.steps[1] : pcs.steps[0]) + (int64_t)qb * (pc ? pcs.pitch[1] : pcs.pitch[0]) * 16;
  const int32_t bbase = pc ? pcs.boff_base[1] : pcs.boff_base[0];
  const int32_t n_list = list[14];  // the list's number of steps (0: an empty list)
  const int32_t head_row = (int32_t)(bh * N);
  for (int j = threadIdx.x; j < len; j += 64) {
    int32_t d[16];
    if (j < n_list) {
      const int4* src = reinterpret_cast<const int4*>(list + (int64_t)j * 16);
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const int4 x = src[u];
        d[4 * u] = x.x;
        d[4 * u + 1] = x.y;
        d[4 * u + 2] = x.z;
        d[4 * u + 3] = x.w;
      }
#pragma unroll
      for (int t = 0; t < 4; ++t)
        if (d[5 + t] >= 0) d[5 + t] += bbase;
    } else {
      // the one step of an empty list: every code 0 (the scores are -inf), rows 0 of the
      // head (valid memory), no bitmaps
#pragma unroll
      for (int u = 0; u < 16; ++u) d[u] = 0;
#pragma unroll
      for (int t = 0; t < 4; ++t) d[5 + t] = -1;
    }
#pragma unroll
    for (int t = 0; t < 4; ++t) d[t] += head_row;
    d[9] = (j == 0 ? 1 : 0) | (j == len - 1 ? 2 : 0) | (pc ? 4 : 0) | (qb << 3);
    d[10] = bh;
    d[11] = sg;
    int4* dst = reinterpret_cast<int4*>(run + ((int64_t)r0 + j) * 16);
#pragma unroll
    for (int u = 0; u < 4; ++u) dst[u] = int4{d[4 * u], d[4 * u + 1], d[4 * u + 2], d[4 * u + 3]};
  }
}

}  // namespace
}  // namespace pa

extern "C" int pa_index_run(const int32_t* const* steps, const int64_t* steps_pitch, const int32_t* boff_base,
                            int32_t n_pieces, int64_t N, const int32_t* item_piece, const int32_t* item_bh,
                            const int32_t* item_qb, const int32_t* item_sync, const int32_t* item_off, int32_t n_items,
                            int32_t* run, void* stream) {
  PA_CHECK_ARG(n_items >= 0, "pa_index_run: n_items=%d", n_items);
  if (n_items == 0) return PA_OK;
  PA_CHECK_ARG(n_pieces == 1 || n_pieces == 2, "pa_index_run: n_pieces=%d (1 or 2)", n_pieces);
  PA_CHECK_ARG(steps && steps_pitch && item_bh && item_qb && item_off && run, "pa_index_run: null argument");
  PA_CHECK_ARG(n_pieces == 1 || item_piece, "pa_index_run: two pieces need item_piece");
  PA_CHECK_ARG(N >= 1 && N <= (1ll << 30), "pa_index_run: N=%lld out of range", (long long)N);
  pa::RunPieces pcs{};
  for (int p = 0; p < n_pieces; ++p) {
    PA_CHECK_ARG(steps[p] && steps_pitch[p] >= 1, "pa_index_run: piece %d has no descriptors", p);
    PA_CHECK_ARG((reinterpret_cast<uintptr_t>(steps[p]) & 15) == 0, "pa_index_run: steps not 16-byte aligned");
    pcs.steps[p] = steps[p];
    pcs.pitch[p] = steps_pitch[p];
    pcs.boff_base[p] = boff_base ? boff_base[p] : 0;
    PA_CHECK_ARG(pcs.boff_base[p] >= 0, "pa_index_run: negative bitmap base");
  }
  PA_CHECK_ARG((reinterpret_cast<uintptr_t>(run) & 15) == 0, "pa_index_run: run must be 16-byte aligned");
  hipLaunchKernelGGL(pa::run_kernel, dim3((unsigned)n_items), dim3(64), 0, static_cast<hipStream_t>(stream), pcs, N,
                     item_piece, item_bh, item_qb, item_sync, item_off, run);
  PA_LAUNCH_CHECK("run_kernel");
  return PA_OK;
}
