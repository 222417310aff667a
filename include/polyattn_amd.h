/*
 * polyattn_amd.h -- C ABI of the MI355X (gfx950) block-sparse masked attention path.
 *
 * Every entry point takes plain device pointers, sizes and a hipStream_t (passed as
 * void*), launches asynchronously on that stream and returns 0 on success or a
 * negative PA_E* code; pa_last_error() then describes the failure.  Nothing here
 * allocates device memory: callers own every buffer.
 *
 * The reference (polyattn, gpu/ directory) has no native code; the functions below
 * replace the Python/numpy/Triton functions cited on each declaration.
 */
#ifndef POLYATTN_AMD_H
#define POLYATTN_AMD_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- status codes ------------------------------------------------------------ */
#define PA_OK 0
#define PA_E_INVALID (-1)     /* argument outside what the kernels support        */
#define PA_E_HIP (-2)         /* a HIP runtime call failed (message has the code)  */
#define PA_E_UNSUPPORTED (-3) /* valid request, no kernel variant built for it     */

/* ---- element types ------------------------------------------------------------ */
#define PA_F32 0
#define PA_F16 1
#define PA_BF16 2

/* ---- mask predicate kinds ------------------------------------------------------
 * 0..5 are the integer kind constants of gpu/masks_gpu.py:9 and
 * gpu/triton_attn.py:23-27 and keep their values.  d = q - kv in ORIGINAL
 * coordinates (after perm_q / perm_kv are applied).
 *   CAUSAL         d >= 0
 *   WINDOW         0 <= d < p0
 *   DILATED        d >= 0 and d % p0 == 0
 *   LOCAL_STRIDED  d >= 0 and (d < p0 or d % p1 == 0)
 *   TWOBAND        d >= 0 and (d < p0 or p1 <= d < p1 + p2)
 *   SINKS          d >= 0 and (d < p0 or kv < p1)     (gpu/masks_gpu.py:51-52)
 *   PREFIX_LM      d >= 0 or (q < p0 and kv < p0)      (src/polyattn/masks.py:129-148)
 *   FULL           always live
 *   DENSE          bit (q, kv) of pa_mask.dense_bits
 */
#define PA_CAUSAL 0
#define PA_WINDOW 1
#define PA_DILATED 2
#define PA_LOCAL_STRIDED 3
#define PA_TWOBAND 4
#define PA_SINKS 5
#define PA_PREFIX_LM 6
#define PA_FULL 7
#define PA_DENSE 8

#define PA_MAX_TERMS 8

typedef struct pa_term {
  int32_t kind, p0, p1, p2;
} pa_term;

/* live(q, kv) = (OR over the n_include first terms) AND NOT (OR over the next
 * n_exclude terms).  A single reference kind is n_include = 1, n_exclude = 0. */
typedef struct pa_mask {
  int32_t n_include;
  int32_t n_exclude;
  pa_term terms[PA_MAX_TERMS];
  const int32_t* perm_q;       /* device [N]: index-space row -> original row; NULL = identity */
  const int32_t* perm_kv;      /* device [N]: index-space col -> original col; NULL = identity */
  const uint32_t* dense_bits;  /* device, PA_DENSE only: word[q * dense_words + kv / 32] bit kv % 32 */
  int64_t dense_words;
} pa_mask;

/* ---- library ------------------------------------------------------------------ */
const char* pa_last_error(void);   /* message of the last failing call on this thread */
int32_t pa_abi_version(void);      /* bumped whenever a struct below changes layout   */

/* ---- block index (replaces gpu/blockindex.py:32-51 build) ------------------------
 * Two phases so the caller can size the padded lists exactly as the reference does
 * (row pitch = max kv_num, gpu/blockindex.py:42-43).
 *
 * pa_index_classify evaluates the predicate on every (q, kv) pair and writes, per
 * (BQ x A) tile, a code of 2 bits per wave group (32 query rows x min(A, 32) kv
 * columns; group g = row_group * max(1, A/32) + col_group): bit 2g = some pair live,
 * bit 2g+1 = every pair live.  A tile is listed iff some group is live; it is FULL
 * iff every group is full.  kv_num[i] = listed tiles in query block i.
 * totals[0] = listed tiles, totals[1] = live pairs, totals[2] = max kv_num.
 * Requires N % BQ == 0, N % A == 0, BQ, A in {16, 32, 64, 128}. */
int pa_index_classify(const pa_mask* mask, int64_t N, int32_t BQ, int32_t A,
                      uint32_t* tile_codes /* [N/BQ * N/A] */, int32_t* kv_num /* [N/BQ] */,
                      unsigned long long* totals /* [3] */, void* stream);

/* Compacts the codes into ascending kv tile lists, zero padded to `pitch` columns:
 * kv_idx int32 [N/BQ, pitch], kv_partial int8 [N/BQ, pitch] (1 = not full),
 * kv_wave_bits uint32 [N/BQ, pitch] (the tile code; may be NULL). */
int pa_index_compact(const uint32_t* tile_codes, const int32_t* kv_num, int64_t N, int32_t BQ,
                     int32_t A, int32_t* kv_idx, int8_t* kv_partial, uint32_t* kv_wave_bits,
                     int64_t pitch, void* stream);

/* Element bitmaps of the listed PARTIAL tiles, so the attention kernel masks from a
 * table instead of evaluating the predicate.  part_base[i] = partial tiles listed in
 * query blocks before i (exclusive prefix).  Writes kv_bits_off[i, j] = word offset of
 * tile j's bitmap in `pool` (-1 for a full tile or padding) and, per partial tile,
 * BQ rows x ceil(A/32) words: bit c of word w of row r = pair (row r, column 32 w + c)
 * of the tile is live.  pool holds (total partial tiles) * BQ * ceil(A/32) words. */
int pa_index_bits(const pa_mask* mask, int64_t N, int32_t BQ, int32_t A, const int32_t* kv_idx,
                  const int32_t* kv_num, const int8_t* kv_partial, int64_t pitch,
                  const int64_t* part_base, int32_t* kv_bits_off, uint32_t* pool, void* stream);

/* Step descriptors of the streaming attention kernel (no counterpart in the reference:
 * a re-layout of the lists above).  The kernel consumes a query block's list as steps of
 * 64 kv columns = 4 segments of 16 columns (segment s of the list is column 16 (s mod
 * A/16) of listed tile s div (A/16)).  Lists are written in issue order: list p holds
 * query block i = order[p] (i = p when order is NULL), and its step j is 16 int32 words
 * at steps[(p * steps_pitch + j) * 16]:
 *   [0..3]  K / V row of segment t's first column: the index-space column b, or with
 *           residue_s > 0 its original row (b mod 2^residue_qlog2) * residue_s +
 *           b div 2^residue_qlog2; 0 past the list (that segment's code is 0)
 *   [4]     byte t = codes of segment t for the 4 row groups of 32 query rows:
 *           bit 2g = some pair live, bit 2g+1 = every pair live (from kv_wave_bits, or
 *           from kv_partial when that is NULL: 0x55 partial, 0xff full)
 *   [5..8]  pool word offset of the bitmap word holding segment t's columns
 *           (kv_bits_off + (16 (s mod A/16)) / 32), -1 when the tile has no bitmap
 *   [9..12] zero
 *   [13]    i, the query block of the list
 *   [14]    the list's number of steps, ceil(kv_num[i] * A / 64)
 *   [15]    residue_s (0 for rows in index space)
 * steps_pitch >= ceil(pitch * A / 64).  kv_wave_bits and kv_bits_off may be NULL.
 * A launch that gathers K / V through the residue basis (gather_kv, residue_s) needs
 * steps built with the same residue_s; any other launch needs residue_s = 0. */
int pa_index_steps(const int32_t* kv_idx, const int32_t* kv_num, const int8_t* kv_partial,
                   const uint32_t* kv_wave_bits, const int32_t* kv_bits_off, int64_t pitch, int64_t N,
                   int32_t BQ, int32_t A, int32_t residue_s, int32_t residue_qlog2, const int32_t* order,
                   int32_t* steps, int64_t steps_pitch, void* stream);

/* Persistent run rows of the streaming kernel (no counterpart in the reference): the
 * step descriptors of n_items work items, item i = (piece item_piece[i], batch-head
 * item_bh[i], query block item_qb[i], sync group item_sync[i]), written to run rows
 * item_off[i] .. item_off[i + 1] - 1 (item_off holds n_items + 1 offsets).  steps[p] is
 * pa_index_steps output for piece p's index in index order (order NULL), [nq,
 * steps_pitch[p], 16], in that piece's residue basis; n_pieces is 1 or 2 (item_piece and
 * item_sync may be NULL: piece 0, no sync group).  A row is the list's step j with its K /
 * V rows offset by item_bh * N (rows of the whole [BH, N] tensor), its bitmap offsets
 * (those >= 0) by boff_base[p] (the piece's part of one shared pool; NULL: 0), word 9 =
 * (1 if j is the item's first step) | (2 if its last) | (4 for piece 1) | item_qb << 3,
 * word 10 = item_bh and word 11 = item_sync (-1: none).  An item whose list is empty must
 * be given one row: it gets a step with every code 0 (the kernel writes zeros and
 * log-sum-exp -inf for it, or leaves a merged row as it was).  A run row holds rows of
 * the whole tensor as int32: (max item_bh + 1) * N must stay below 2^31 (not checked here,
 * the heads are on the device; schedule.py checks it before the call). */
int pa_index_run(const int32_t* const* steps, const int64_t* steps_pitch, const int32_t* boff_base, int32_t n_pieces,
                 int64_t N, const int32_t* item_piece, const int32_t* item_bh, const int32_t* item_qb,
                 const int32_t* item_sync, const int32_t* item_off, int32_t n_items, int32_t* run, void* stream);

/* ---- class-A permutation (replaces gpu/permute.py:12-31) -------------------------
 * Row gather dst[b, p, :] = src[b, perm[p], :] (inverse = 0), the index_select of
 * gpu/permute.py:22-24, or row scatter dst[b, perm[p], :] = src[b, p, :] (inverse = 1),
 * the un-permute of gpu/test_correctness.py:77.  Strides are in bytes; row_bytes is
 * the contiguous length of one row. */
int pa_permute_rows(const void* src, void* dst, const int32_t* perm, int64_t BH, int64_t N,
                    int64_t row_bytes, int64_t src_bh_stride, int64_t src_row_stride,
                    int64_t dst_bh_stride, int64_t dst_row_stride, int32_t inverse, void* stream);

/* Once-per-forward relabelling of a stack of tensors (the regime of
 * gpu/exp5_amortisation.py:89-118, where the stack runs in the permuted basis): one
 * launch gathers (inverse = 0) or scatters (inverse = 1) the rows of n_tensors <= 8
 * tensors of one shape and stride, as pa_permute_rows, and moves their position ids
 * with them: pos_out[d] = pos_in[s] for each row moved from s to d (pos_in NULL: the ids
 * are the source rows themselves, pos_out[p] = perm[p] for a gather), so that
 * position-dependent ops (RoPE, gpu/exp5_amortisation.py:44-57) see every token's
 * original position.  srcs / dsts are host arrays of device pointers; pos_in / pos_out
 * are NULL or int64 [N] on the device (shared by every batch-head). */
int pa_permute_stack(const void* const* srcs, void* const* dsts, int32_t n_tensors, const int32_t* perm,
                     int64_t BH, int64_t N, int64_t row_bytes, int64_t src_bh_stride, int64_t src_row_stride,
                     int64_t dst_bh_stride, int64_t dst_row_stride, const int64_t* pos_in, int64_t* pos_out,
                     int32_t inverse, void* stream);

/* inv[perm[p]] = p  (gpu/permute.py:27-31). */
int pa_invert_perm(const int32_t* perm, int32_t* inv, int64_t N, void* stream);

/* perm[p] = original position at permuted position p for the residue-class sort
 * by (i mod s, i div s) (gpu/permute.py:12-15), any N >= 1, s >= 1. */
int pa_residue_perm(int32_t* perm, int64_t N, int32_t s, void* stream);

/* ---- attention forward (replaces gpu/triton_attn.py:62-241) ----------------------- */
typedef struct pa_attn_args {
  const void* q;  /* [BH, N, D] rows of D contiguous elements */
  const void* k;
  const void* v;
  void* o;
  int64_t q_sb, q_sn, k_sb, k_sn, v_sb, v_sn, o_sb, o_sn; /* strides in elements */
  int64_t BH, N;
  int32_t D;      /* 64 or 128 */
  int32_t dtype;  /* PA_F32 / PA_F16 / PA_BF16 for q, k, v and o */
  float scale;    /* softmax scale, usually D ** -0.5 */
  int32_t BQ, A;  /* tile shape of the block index */
  const int32_t* kv_idx;        /* [N/BQ, pitch] */
  const int32_t* kv_num;        /* [N/BQ] */
  const int8_t* kv_partial;     /* [N/BQ, pitch] */
  const uint32_t* kv_wave_bits; /* [N/BQ, pitch] or NULL: per-wave skip and mask bits */
  int64_t pitch;
  const int32_t* kv_bits_off;   /* NULL, or pa_index_bits output: partial tiles are masked */
  const uint32_t* kv_bits;      /*   from these bitmaps instead of evaluating `mask`       */
  pa_mask mask;   /* predicate applied on partial tiles, in original coordinates */
  int32_t gather_q;   /* load query rows through mask.perm_q (Q not physically permuted) */
  int32_t gather_kv;  /* load key/value rows through mask.perm_kv (gpu/triton_attn.py:104-107) */
  int32_t scatter_o;  /* store output row r at mask.perm_q[r] (fused inverse permutation) */
  int32_t residue_s;      /* > 0: perm_q = perm_kv = the residue permutation of stride s     */
  int32_t residue_qlog2;  /*   with N / s = 2^residue_qlog2, computed in closed form:        */
                          /*   perm[p] = (p mod 2^qlog2) * s + p div 2^qlog2 (no table reads) */
  float* lse;         /* NULL or [BH, N] fp32, natural-log sum-exp of the stored rows */
  int64_t lse_sb;
  const void* prev_o;      /* NULL or a partial result over a disjoint sub-mask, same
                              row order as o; merged by log-sum-exp into o */
  int32_t prev_dtype;      /* PA_F32 / PA_F16 / PA_BF16 */
  int64_t prev_sb, prev_sn;
  const float* prev_lse;   /* [BH, N] stride lse_sb, required with prev_o */
  const int32_t* qblock_order; /* NULL or [N/BQ] permutation: order query blocks are issued */
  const int32_t* kv_steps;     /* NULL or pa_index_steps output for this index, written in the */
  int64_t steps_pitch;         /*   order of qblock_order: enables the streaming kernel (f16 /  */
                               /*   bf16, D = 128, BQ = 128, A in 16, 32, 64, bitmaps for the   */
                               /*   partial tiles, no table gather of K/V), which takes each    */
                               /*   list's query block and length from its first descriptor    */
  int32_t heads_desc;          /* nonzero: heads are issued from the last to the first.  A pass */
                               /*   that follows another over the same tensors then starts on   */
                               /*   the heads the previous one touched last (still in cache).   */
                               /*   Results do not depend on it.                                */
  /* Class-B traffic emulation (gpu/triton_attn.py:99-128, 202-205).  gather_mult > 1: for
   * every listed tile the K rows are read as sum_r wsel[b * wsel_sb + r] * K[row_r] over
   * r < gather_mult, row_0 being the tile's row for kv column c and, for r >= 1,
   * gather_scatter = 0: (row_0 + r A) mod N (contiguous extra rows), gather_scatter != 0:
   * perm_kv((c + r A) mod N) (scattered).  wsel is [BH, gather_mult] in the dtype of q,
   * [1, 0, ...] in the reference: the extra rows are read and the result is unchanged.
   * General kernel only (not with kv_steps). */
  int32_t gather_mult;    /* 0 or 1: off */
  int32_t gather_scatter;
  const void* wsel;
  int64_t wsel_sb;
  /* Persistent schedule (no counterpart in the reference: the Triton kernel runs one
   * program per (query block, head), gpu/triton_attn.py:210).  run_groups > 0: the
   * streaming kernel runs as run_groups work-groups, group g taking the run rows
   * run_start[g] .. run_start[g + 1] - 1 of run_steps (pa_index_run output for this
   * index, basis and BH) one after the other as a single stream of steps, so no step
   * pipeline drains between query blocks.  Same preconditions as kv_steps (which is then
   * not read), plus: the residue basis in closed form for any gather / scatter, q, k, v
   * and o with batch stride N * row stride, and BH * N * row bytes below 2^32.  Results
   * are those of the per-block launch. */
  const int32_t* run_steps;
  const int32_t* run_start;   /* [run_groups + 1] */
  int32_t run_groups;
  /* wave_split != 0: the wave-split kernel (no counterpart in the reference), for grids
   * too small to fill the chip: one 8-wave work-group per (batch-head, 16 query rows),
   * the waves splitting the rows' live 16x16 sub-tiles and merging their softmax states
   * in LDS.  float32, D = 64 or 128, BQ and A multiples of 32, kv_wave_bits given, no
   * permutation (perm tables, gathers, scatter, residue basis), no class-B emulation, no
   * prev_o, no kv_steps / run_groups; results within float32 rounding of the general
   * kernel's. */
  int32_t wave_split;
} pa_attn_args;

int pa_attn_fwd(const pa_attn_args* args, void* stream);

/* A two-piece disjoint split in ONE persistent launch (no counterpart in the reference,
 * which prices a split, src/polyattn/experiments/compose.py:107-119, but has no code for
 * it).  `first` and `second` are the arguments each piece would take as a run launch of
 * its own (run_groups > 0, the split's run rows): the first writes o and lse, the second
 * merges into them in place (prev_o = first->o, prev_lse = first->lse), over the same
 * q, k, v, o, lse, shapes, dtype, scale and tile; they may differ in basis (residue_s,
 * gather / scatter flags) and index.  The run rows (pa_index_run, two pieces) carry both
 * pieces' items and each item's sync group: the rows of a second-piece item are covered
 * by `sync_signal` first-piece items of its group, and a group has `sync_wait`
 * second-piece items.  kv_bits is both pieces' bitmaps in one pool (the rows' offsets
 * point into it).  sync is int32 [2 * sync_groups], all zero before the first launch;
 * every launch leaves it zero again.  The launch is cooperative (PA_E_INVALID if the
 * run's work-groups cannot all be resident at once).  *status (int32) is set to 1 if a
 * merge gave up waiting for its group (the results are then invalid; zero it again, and
 * sync, before reuse).  The schedule must list every second-piece item after the
 * first-piece items of its group in each work-group's order. */
typedef struct pa_split_args {
  const pa_attn_args* first;
  const pa_attn_args* second;
  const int32_t* run_steps;
  const int32_t* run_start;   /* [run_groups + 1] */
  int32_t run_groups;
  const uint32_t* kv_bits;
  int32_t* sync;
  int32_t sync_groups;
  int32_t sync_signal;
  int32_t sync_wait;
  int32_t* status;
  /* items != NULL: the split runs as one work-group per item instead of a persistent run
   * (run_steps / run_start / run_groups / kv_bits then unused, and each piece's args have
   * run_groups 0 and their kv_steps in index order).  items is int32 [n_items][4] =
   * (piece, batch-head, query block, sync group), listed in the order the work-groups
   * are to start (the first-piece items of a group before every second-piece item of
   * it); the hardware starts work-groups in id order, and work-group i takes item
   * i' = (i mod 8) * (n / 8) + min(i mod 8, n mod 8) + i div 8 (the items of XCD x are a
   * contiguous range).  Not cooperative. */
  const int32_t* items;
  int64_t n_items;
} pa_split_args;

int pa_attn_fwd_split(const pa_split_args* args, void* stream);

/* ---- log-sum-exp merge of a disjoint split (spec: src/polyattn/experiments/compose.py:7-17)
 * o[b, r, :] = sum_k exp(lse_k - M) o_k / sum_k exp(lse_k - M), M = max_k lse_k;
 * rows with every lse_k = -inf give 0 and lse -inf.  parts are fp32 [BH, N, D]
 * contiguous; o is dtype `out_dtype` contiguous; lse_out may be NULL. */
int pa_lse_merge(const float* const* o_parts, const float* const* lse_parts, int32_t n_parts,
                 void* o, int32_t out_dtype, float* lse_out, int64_t BH, int64_t N, int32_t D,
                 void* stream);

/* ---- decoding against a cache kept in a class-A basis ------------------------------
 * The reference relabels tokens for prefill only and leaves decoding open: new keys
 * arrive in original order and would have to be inserted at permuted positions
 * (docs/NOTES.md:2145-2153, 2201-2203).  These entry points answer it for the residue
 * bases of gpu/permute.py:12-15.  A cache of `capacity` rows per head (a multiple of
 * s; s = residue_s, 0 or 1 = identity, at most 4096) keeps the token at original
 * position t at row (t mod s) * (capacity / s) + t div s, so appending never moves a
 * cached row.
 *
 * pa_kv_append: rows j = 0..n-1 of k_new / v_new [BH, n, D] (strides in elements) are
 * the tokens at original positions pos0 + j; each is written to its basis row of
 * k_cache / v_cache [BH, capacity, D].  pos0 + n <= capacity. */
int pa_kv_append(const void* k_new, const void* v_new, int64_t new_sb, int64_t new_sn, void* k_cache,
                 void* v_cache, int64_t c_sb, int64_t c_sn, int64_t BH, int64_t n, int32_t D, int32_t dtype,
                 int64_t capacity, int64_t pos0, int32_t residue_s, void* stream);

/* pa_decode_fwd: o[b, i] = softmax over the cached tokens t < length that are live for
 * the query at original position qpos0 + i under `mask` (perm_q / perm_kv NULL), of
 * (q[b, i] . k_t) * scale, applied to v_t; a query with no live token gives 0 and lse
 * -inf (gpu/reference.py:5-17 on one row).  1 <= nq <= 8; D = 64 or 128 (float32: 64);
 * q, o [BH, nq, D], lse [BH, nq] fp32 or NULL; scale <= 0 means 1/sqrt(D).  The split
 * partials go to `workspace`, whose size pa_decode_workspace returns for these
 * arguments (it depends on BH, nq, D, capacity, length and residue_s).  A PA_DENSE
 * mask must hold rows up to qpos0 + nq - 1.
 *
 * With n_new > 0 the call also appends: rows j = 0..n_new-1 of k_new / v_new [BH, n_new,
 * D] (strides new_sb / new_sn in elements, 16-byte aligned rows) are the tokens at
 * original positions new_pos0 + j, as pa_kv_append would write them, and the attention
 * reads them from k_new / v_new (the split's work-group that owns a new row also writes
 * it to the cache), so one call does what pa_kv_append followed by pa_decode_fwd does.
 * n_new <= 8, new_pos0 >= 0 and new_pos0 + n_new <= length.  n_new = 0 (the zero-filled
 * default) appends nothing. */
typedef struct pa_decode_args {
  const void* q;
  int64_t q_sb, q_sn;
  int32_t nq;
  int64_t qpos0;
  void* k_cache;  /* read; written only for the rows appended by the call (n_new > 0) */
  void* v_cache;
  int64_t c_sb, c_sn;
  int64_t capacity, length;
  int32_t residue_s;
  pa_mask mask;
  int64_t BH;
  int32_t D, dtype;
  float scale;
  void* o;
  int64_t o_sb, o_sn;
  float* lse;
  int64_t lse_sb;
  void* workspace;
  int64_t workspace_bytes;
  const void* k_new;
  const void* v_new;
  int64_t new_sb, new_sn;
  int64_t n_new, new_pos0;
} pa_decode_args;

int pa_decode_workspace(const pa_decode_args* args, int64_t* bytes);
int pa_decode_fwd(const pa_decode_args* args, void* stream);

/* pa_decode_fwd_static: pa_decode_fwd that allocates nothing and takes no workspace
 * (args->workspace NULL, workspace_bytes 0).  No counterpart in the reference: it is for
 * callers that cannot allocate device memory (code under HIP graph capture, serving loops
 * and harnesses that forbid hipMalloc).  The split partials go to an 8 MiB scratch array
 * of the library, one per GPU, held until the process ends; a call whose partials need
 * more (pa_decode_workspace's size) fails with PA_E_INVALID.  Every call on a GPU shares
 * that GPU's scratch: calls that overlap on one GPU (other streams, other threads) race
 * and give wrong results; calls in one stream are ordered and safe. */
int pa_decode_fwd_static(const pa_decode_args* args, void* stream);

/* ---- backward (the reference has none: gpu/triton_attn.py:9-10, README.md:118) ------
 * pa_index_transpose: for each of the nk key blocks, the query blocks whose list
 * (kv_idx / kv_num / kv_partial of an index built at BQ = A, pitch columns) holds it, in
 * ascending order, with the partial flag: q_num [nk], q_idx / q_partial [nk, tpitch].
 * With kv_bits_off (pa_index_bits of the same index; may be NULL) also q_bits_off
 * [nk, tpitch]: the word offset of the tile's bitmap, -1 for a full tile.
 * With q_idx NULL only q_num is written (size tpitch as max q_num, then call again).
 *
 * pa_index_bits_transpose: for every listed tile with kv_bits_off >= 0 (an index built
 * at BQ = A = 64), its bitmap transposed into q_bits at the same word offset: bit c of
 * word w of column k = pair (row 32 w + c, column k) of the tile is live.  q_bits has
 * the size of kv_bits.
 *
 * pa_attn_bwd: gradients of o = softmax(scale q k^T masked) v for f16 / bf16, D = 64
 * or 128, N a multiple of 64, from the forward's lse (natural log, [BH, N], row stride
 * lse_sb; -inf rows get no gradient) and dO.  q, k, v, o, dout, dq, dk, dv are
 * [BH, N, D] with the same element strides sb / sn.  The index is the forward's at
 * BQ = A = 64 and its transpose; the mask is evaluated on partial tiles only, at
 * (perm_q[r], perm_kv[c]) when the tables are given (tensors stay in index space).
 * dvec is a caller-owned fp32 [BH, N] workspace (rowsum(dO * O), same stride as lse).
 * kv_bits_off / kv_bits (pa_index_bits) with q_bits_off / q_bits (their transpose) are
 * all NULL or all given; given, the D = 128 kernels mask partial tiles from them instead
 * of evaluating the mask.  flags: PA_BWD_ACCUMULATE adds the gradients into dq / dk / dv
 * instead of overwriting them (the backward of a mask split into disjoint pieces is the
 * sum of the pieces' backwards, each with the whole mask's lse and dvec);
 * PA_BWD_DVEC_GIVEN takes dvec as already holding rowsum(dO * O) (no pre-pass).
 * residue_s > 1 (D = 128, N / s a power of two and a multiple of 64): the index is in the
 * residue-s basis but q, k, v, o, dout, lse, dvec and the gradients stay in ORIGINAL
 * order; index-space row r is read and written at row (r mod (N/s)) s + r div (N/s)
 * (the basis applied in the loads and stores, as gather_q / gather_kv / scatter_o do in
 * the forward).  0 = every array in index space.
 * kv_order: NULL, or the N / 64 key blocks in the order the dK / dV pass issues them
 * (longest transposed list first balances masks whose few key blocks are held by many
 * query blocks, such as attention sinks). */
#define PA_BWD_ACCUMULATE 1
#define PA_BWD_DVEC_GIVEN 2
int pa_index_transpose(const int32_t* kv_idx, const int32_t* kv_num, const int8_t* kv_partial,
                       const int32_t* kv_bits_off, int32_t nq, int64_t pitch, int32_t nk, int32_t* q_num,
                       int32_t* q_idx, int8_t* q_partial, int32_t* q_bits_off, int64_t tpitch, void* stream);

int pa_index_bits_transpose(const int32_t* kv_bits_off, int32_t nq, int64_t pitch, const uint32_t* kv_bits,
                            uint32_t* q_bits, void* stream);

typedef struct pa_attn_bwd_args {
  const void* q;
  const void* k;
  const void* v;
  const void* o;
  const void* dout;
  void* dq;
  void* dk;
  void* dv;
  int64_t sb, sn;
  const float* lse;
  float* dvec;
  int64_t lse_sb;
  int64_t BH, N;
  int32_t D, dtype;
  float scale;
  const int32_t* kv_idx;
  const int32_t* kv_num;
  const int8_t* kv_partial;
  int64_t pitch;
  const int32_t* q_idx;
  const int32_t* q_num;
  const int8_t* q_partial;
  int64_t tpitch;
  const int32_t* kv_bits_off;
  const uint32_t* kv_bits;
  const int32_t* q_bits_off;
  const uint32_t* q_bits;
  int32_t flags;
  int32_t residue_s;
  const int32_t* kv_order;
  pa_mask mask;
} pa_attn_bwd_args;

int pa_attn_bwd(const pa_attn_bwd_args* args, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* POLYATTN_AMD_H */
