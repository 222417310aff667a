// Shared device/host helpers for the gfx950 block-sparse attention library.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stdio.h>

#include "polyattn_amd.h"

namespace pa {

// ---------------------------------------------------------------------------
// Error reporting: a thread-local message read back through pa_last_error().
void set_error(const char* fmt, ...);
int hip_fail(hipError_t e, const char* what);

#define PA_CHECK_ARG(cond, ...)          \
  do {                                   \
    if (!(cond)) {                       \
      ::pa::set_error(__VA_ARGS__);      \
      return PA_E_INVALID;               \
    }                                    \
  } while (0)

#define PA_LAUNCH_CHECK(what)                              \
  do {                                                     \
    hipError_t e_ = hipGetLastError();                     \
    if (e_ != hipSuccess) return ::pa::hip_fail(e_, what); \
  } while (0)

// ---------------------------------------------------------------------------
// Mask predicate.  The kernels receive the pa_mask by value; evaluation is a
// loop over at most PA_MAX_TERMS terms whose kinds are wave-uniform.
struct Pred {
  int32_t n_include, n_exclude;
  pa_term terms[PA_MAX_TERMS];
  const int32_t* perm_q;
  const int32_t* perm_kv;
  const uint32_t* dense_bits;
  int64_t dense_words;
};

static inline Pred make_pred(const pa_mask& m) {
  Pred p;
  p.n_include = m.n_include;
  p.n_exclude = m.n_exclude;
  for (int i = 0; i < PA_MAX_TERMS; ++i) p.terms[i] = m.terms[i];
  p.perm_q = m.perm_q;
  p.perm_kv = m.perm_kv;
  p.dense_bits = m.dense_bits;
  p.dense_words = m.dense_words;
  return p;
}

// One term on original coordinates (q, kv).  d = q - kv as in gpu/masks_gpu.py:37-52.
__device__ __forceinline__ bool term_live(const pa_term& t, int32_t q, int32_t kv,
                                          const uint32_t* dense, int64_t words) {
  const int32_t d = q - kv;
  switch (t.kind) {
    case PA_CAUSAL:
      return d >= 0;
    case PA_WINDOW:
      return d >= 0 && d < t.p0;
    case PA_DILATED:
      return d >= 0 && (d % t.p0) == 0;
    case PA_LOCAL_STRIDED:
      return d >= 0 && (d < t.p0 || (d % t.p1) == 0);
    case PA_TWOBAND:
      return d >= 0 && (d < t.p0 || (d >= t.p1 && d < t.p1 + t.p2));
    case PA_SINKS:
      return d >= 0 && (d < t.p0 || kv < t.p1);
    case PA_PREFIX_LM:
      return d >= 0 || (q < t.p0 && kv < t.p0);
    case PA_FULL:
      return true;
    case PA_DENSE:
      return (dense[(int64_t)q * words + (kv >> 5)] >> (kv & 31)) & 1u;
    default:
      return false;
  }
}

// Unrolled over the fixed term capacity so every terms[i] access has a constant
// index: a runtime index would make the compiler copy the whole kernel-argument
// block into scratch memory.
__device__ __forceinline__ bool pred_live(const Pred& p, int32_t q, int32_t kv) {
  bool inc = false, exc = false;
  const int n = p.n_include + p.n_exclude;
#pragma unroll
  for (int i = 0; i < PA_MAX_TERMS; ++i) {
    if (i < n) {
      const bool l = term_live(p.terms[i], q, kv, p.dense_bits, p.dense_words);
      if (i < p.n_include)
        inc |= l;
      else
        exc |= l;
    }
  }
  return inc && !exc;
}

// Same predicate with the terms read from memory (LDS in the attention kernel) in a
// rolled loop: one copy of the term switch, for code that evaluates it rarely.
__device__ __forceinline__ bool pred_live_rolled(const pa_term* terms, int n_include, int n_exclude,
                                                 int32_t q, int32_t kv, const uint32_t* dense,
                                                 int64_t words) {
  bool inc = false, exc = false;
#pragma unroll 1
  for (int i = 0; i < n_include + n_exclude; ++i) {
    const pa_term t = terms[i];
    const bool l = term_live(t, q, kv, dense, words);
    if (i < n_include)
      inc |= l;
    else
      exc |= l;
  }
  return inc && !exc;
}

// Validates a host-side pa_mask; returns 0 or an error code (message set).
int check_mask(const pa_mask* m, int64_t N);

// Hardware work-group id -> logical id so that consecutive logical ids land on the
// same XCD (MI355X dispatches work-groups round-robin over its 8 XCDs, each with
// its own L2).  Bijective for any total.
__device__ __forceinline__ int64_t xcd_remap(int64_t hw, int64_t total) {
  constexpr int64_t kXcd = 8;
  const int64_t per = total / kXcd;       // full rounds
  const int64_t rem = total % kXcd;       // XCDs that get one extra
  const int64_t x = hw % kXcd;
  const int64_t r = hw / kXcd;
  if (r < per) {
    // x-th XCD owns a contiguous run; earlier XCDs with an extra item shift it.
    const int64_t base = x * per + (x < rem ? x : rem);
    return base + r;
  }
  // tail round (r == per): only XCDs x < rem exist here
  return x * per + x + per;
}
// The same in 32-bit arithmetic (total < 2^31).
__device__ __forceinline__ uint32_t xcd_remap32(uint32_t hw, uint32_t total) {
  const uint32_t per = total >> 3, rem = total & 7u;
  const uint32_t x = hw & 7u, r = hw >> 3;
  if (r < per) return x * per + (x < rem ? x : rem) + r;
  return x * per + x + per;
}

}  // namespace pa
