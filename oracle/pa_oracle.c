/*
 * CPU oracle for the block-index path.  TEST INFRASTRUCTURE ONLY: loaded by tests/,
 * __graft_entry__.smoke() and bench.py's cpu_baseline leg, never by the product.
 *
 * Restates, in plain C:
 *   - the mask predicates of gpu/masks_gpu.py:37-52 (flex_mask_mod / dense_bool;
 *     the SINKS sink term on absolute kv, :51-52), PrefixLM of
 *     src/polyattn/masks.py:129-148, set difference, class-A relabelling
 *     (M[perm][:, perm], gpu/test_correctness.py:71) and an explicit bitmap;
 *   - gpu/blockindex.py:32-51 build(): a tile is listed iff any pair in it is live,
 *     FULL iff every pair is live; lists ascending, zero padded to max_kv;
 *     elements = listed tiles * BQ * A; live = live pairs.
 * Unlike the reference it streams one query block at a time (never N x N).
 * It also produces the per-tile wave-group codes the GPU builder emits
 * (2 bits per 32-row x min(A, 32)-column group: some live, all live).
 */
#include <stdint.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

#define O_MAX_TERMS 8

typedef struct {
  int32_t kind, p0, p1, p2;
} oterm;

typedef struct {
  int32_t n_include, n_exclude;
  oterm terms[O_MAX_TERMS];
  const int32_t* perm_q;   /* NULL = identity */
  const int32_t* perm_kv;  /* NULL = identity */
  const uint8_t* dense;    /* kind 8: row-major bool bytes, N x N, index = q * N + kv */
  int64_t dense_n;
} omask;

enum { K_CAUSAL, K_WINDOW, K_DILATED, K_LOCAL_STRIDED, K_TWOBAND, K_SINKS, K_PREFIX_LM, K_FULL, K_DENSE };

static int term_live(const oterm* t, int64_t q, int64_t kv, const omask* m) {
  const int64_t d = q - kv;
  switch (t->kind) {
    case K_CAUSAL: return q >= kv;
    case K_WINDOW: return q >= kv && d < t->p0;
    case K_DILATED: return q >= kv && d % t->p0 == 0;
    case K_LOCAL_STRIDED: return q >= kv && (d < t->p0 || d % t->p1 == 0);
    case K_TWOBAND: return q >= kv && (d < t->p0 || (d >= t->p1 && d < (int64_t)t->p1 + t->p2));
    case K_SINKS: return q >= kv && (d < t->p0 || kv < t->p1);
    case K_PREFIX_LM: return q >= kv || (q < t->p0 && kv < t->p0);
    case K_FULL: return 1;
    case K_DENSE: return m->dense[q * m->dense_n + kv] != 0;
    default: return 0;
  }
}

/* live at index-space (r, c): predicate on original coordinates (perm applied). */
int oracle_live(const omask* m, int64_t r, int64_t c) {
  const int64_t q = m->perm_q ? m->perm_q[r] : r;
  const int64_t kv = m->perm_kv ? m->perm_kv[c] : c;
  int inc = 0;
  for (int i = 0; i < m->n_include && !inc; ++i) inc = term_live(&m->terms[i], q, kv, m);
  if (!inc) return 0;
  for (int i = 0; i < m->n_exclude; ++i)
    if (term_live(&m->terms[m->n_include + i], q, kv, m)) return 0;
  return 1;
}

/* Row r of the mask as bytes: out[c] = live(r, c), c < N. */
void oracle_row(const omask* m, int64_t N, int64_t r, uint8_t* out) {
  for (int64_t c = 0; c < N; ++c) out[c] = (uint8_t)oracle_live(m, r, c);
}

/* Per-tile codes for every (query block, kv tile): codes[qb * nk + kb].
 * Returns live pairs.  threads <= 0 means the OpenMP default. */
int64_t oracle_tile_codes(const omask* m, int64_t N, int32_t BQ, int32_t A, uint32_t* codes, int threads) {
  const int64_t nq = N / BQ, nk = N / A;
  const int rg_rows = BQ < 32 ? BQ : 32;
  const int cw = A < 32 ? A : 32;
  const int ncg = A / cw;
  int64_t live_total = 0;
#ifdef _OPENMP
  if (threads > 0) omp_set_num_threads(threads);
#pragma omp parallel for schedule(dynamic, 1) reduction(+ : live_total)
#endif
  for (int64_t qb = 0; qb < nq; ++qb) {
    uint8_t* row = (uint8_t*)malloc((size_t)N);
    /* any/all per (row group, column group over the whole row) */
    const int n_rg = BQ / rg_rows;
    const int64_t ncol_groups = N / cw;
    uint8_t* any = (uint8_t*)calloc((size_t)(n_rg * ncol_groups), 1);
    uint8_t* all = (uint8_t*)malloc((size_t)(n_rg * ncol_groups));
    memset(all, 1, (size_t)(n_rg * ncol_groups));
    for (int rr = 0; rr < BQ; ++rr) {
      const int64_t r = qb * BQ + rr;
      const int g = rr / rg_rows;
      oracle_row(m, N, r, row);
      for (int64_t cgi = 0; cgi < ncol_groups; ++cgi) {
        uint8_t a = 0, l = 1;
        for (int e = 0; e < cw; ++e) {
          const uint8_t x = row[cgi * cw + e];
          a |= x;
          l &= x;
          live_total += x;
        }
        any[g * ncol_groups + cgi] |= a;
        all[g * ncol_groups + cgi] &= l;
      }
    }
    for (int64_t kb = 0; kb < nk; ++kb) {
      uint32_t code = 0;
      for (int g = 0; g < n_rg; ++g)
        for (int cg = 0; cg < ncg; ++cg) {
          const int64_t cgi = kb * ncg + cg;
          const int bit = g * ncg + cg;
          code |= (uint32_t)any[g * ncol_groups + cgi] << (2 * bit);
          code |= (uint32_t)all[g * ncol_groups + cgi] << (2 * bit + 1);
        }
      codes[qb * nk + kb] = code;
    }
    free(row);
    free(any);
    free(all);
  }
  return live_total;
}

/* Compaction of tile codes into the reference's padded lists.
 * kv_num[nq]; if kv_idx != NULL: kv_idx / kv_partial / wave [nq * pitch] are filled
 * (ascending tiles, zero padded).  Returns max kv_num. */
int32_t oracle_compact(const uint32_t* codes, int64_t N, int32_t BQ, int32_t A, int32_t* kv_num,
                       int32_t* kv_idx, int8_t* kv_partial, uint32_t* wave, int64_t pitch) {
  const int64_t nq = N / BQ, nk = N / A;
  const int rg_rows = BQ < 32 ? BQ : 32;
  const int cw = A < 32 ? A : 32;
  const int ngroups = (BQ / rg_rows) * (A / cw);
  uint32_t anymask = 0, fullmask = 0;
  for (int g = 0; g < ngroups; ++g) {
    anymask |= 1u << (2 * g);
    fullmask |= 2u << (2 * g);
  }
  int32_t mx = 0;
  for (int64_t qb = 0; qb < nq; ++qb) {
    int32_t n = 0;
    for (int64_t kb = 0; kb < nk; ++kb) {
      const uint32_t code = codes[qb * nk + kb];
      if (!(code & anymask)) continue;
      if (kv_idx && n < pitch) {
        kv_idx[qb * pitch + n] = (int32_t)kb;
        kv_partial[qb * pitch + n] = (code & fullmask) == fullmask ? 0 : 1;
        if (wave) wave[qb * pitch + n] = code;
      }
      ++n;
    }
    if (kv_idx)
      for (int64_t j = n; j < pitch; ++j) {
        kv_idx[qb * pitch + j] = 0;
        kv_partial[qb * pitch + j] = 0;
        if (wave) wave[qb * pitch + j] = 0;
      }
    kv_num[qb] = n;
    if (n > mx) mx = n;
  }
  return mx;
}
