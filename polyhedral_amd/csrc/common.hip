// Library-wide host helpers: error messages, mask validation, version.
#include <stdarg.h>
#include <string.h>

#include "common.hpp"

namespace pa {

static thread_local char g_err[512] = "";

void set_error(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
}

int hip_fail(hipError_t e, const char* what) {
  set_error("%s: HIP error %d (%s)", what, (int)e, hipGetErrorString(e));
  return PA_E_HIP;
}

int check_mask(const pa_mask* m, int64_t N) {
  if (m->n_include < 1 || m->n_exclude < 0 || m->n_include + m->n_exclude > PA_MAX_TERMS) {
    set_error("mask: n_include=%d n_exclude=%d (need 1 <= n_include, n_include + n_exclude <= %d)",
              m->n_include, m->n_exclude, PA_MAX_TERMS);
    return PA_E_INVALID;
  }
  for (int i = 0; i < m->n_include + m->n_exclude; ++i) {
    const pa_term& t = m->terms[i];
    switch (t.kind) {
      case PA_CAUSAL:
      case PA_FULL:
        break;
      case PA_WINDOW:
      case PA_SINKS:
      case PA_PREFIX_LM:
      case PA_TWOBAND:
        if (t.p0 < 0 || t.p1 < 0 || t.p2 < 0) {
          set_error("mask term %d (kind %d): negative parameter", i, t.kind);
          return PA_E_INVALID;
        }
        break;
      case PA_DILATED:
        if (t.p0 < 1) {
          set_error("mask term %d: DILATED stride p0=%d must be >= 1", i, t.p0);
          return PA_E_INVALID;
        }
        break;
      case PA_LOCAL_STRIDED:
        if (t.p0 < 0 || t.p1 < 1) {
          set_error("mask term %d: LOCAL_STRIDED needs p0 >= 0 and stride p1 >= 1", i);
          return PA_E_INVALID;
        }
        break;
      case PA_DENSE:
        if (!m->dense_bits || m->dense_words < (N + 31) / 32) {
          set_error("mask term %d: DENSE needs dense_bits with >= %lld words per row", i,
                    (long long)((N + 31) / 32));
          return PA_E_INVALID;
        }
        break;
      default:
        set_error("mask term %d: unknown kind %d", i, t.kind);
        return PA_E_INVALID;
    }
  }
  return PA_OK;
}

}  // namespace pa

extern "C" const char* pa_last_error(void) { return pa::g_err; }

extern "C" int32_t pa_abi_version(void) { return 19; }
