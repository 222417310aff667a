// Log-sum-exp merge of attention partials computed over disjoint sub-masks.
// The reference describes the split (src/polyattn/experiments/compose.py:7-17) but
// never implements it; this is the standalone merge.  The attention kernel can
// also fold one partial into its own epilogue (pa_attn_args.prev_o), which is
// the path the split driver uses.
#include "common.hpp"

namespace pa {
namespace {

constexpr int kMaxParts = 8;

struct MergeArgs {
  const float* o[kMaxParts];
  const float* lse[kMaxParts];
  int32_t n;
};

template <typename T>
__device__ __forceinline__ void store_out(T* p, float x);
template <>
__device__ __forceinline__ void store_out<float>(float* p, float x) { *p = x; }
template <>
__device__ __forceinline__ void store_out<_Float16>(_Float16* p, float x) { *p = (_Float16)x; }
template <>
__device__ __forceinline__ void store_out<__bf16>(__bf16* p, float x) { *p = (__bf16)x; }

// One wave per row; lanes stride over D.
template <typename T>
__global__ __launch_bounds__(256) void lse_merge_kernel(const MergeArgs a, T* __restrict__ out,
                                                         float* __restrict__ lse_out, int64_t rows,
                                                         int32_t D) {
  const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (row >= rows) return;
  float mx = -INFINITY;
  for (int k = 0; k < a.n; ++k) mx = fmaxf(mx, a.lse[k][row]);
  float w[kMaxParts];
  float den = 0.f;
  for (int k = 0; k < kMaxParts; ++k) {
    w[k] = (k < a.n && mx != -INFINITY) ? expf(a.lse[k][row] - mx) : 0.f;
    den += w[k];
  }
  const float inv = den > 0.f ? 1.f / den : 0.f;
  for (int d = lane; d < D; d += 64) {
    float acc = 0.f;
    for (int k = 0; k < a.n; ++k)
      if (w[k] != 0.f) acc += w[k] * a.o[k][row * D + d];
    store_out<T>(out + row * D + d, acc * inv);
  }
  if (lse_out && lane == 0) lse_out[row] = den > 0.f ? mx + logf(den) : -INFINITY;
}

}  // namespace
}  // namespace pa

extern "C" int pa_lse_merge(const float* const* o_parts, const float* const* lse_parts, int32_t n_parts,
                            void* o, int32_t out_dtype, float* lse_out, int64_t BH, int64_t N, int32_t D,
                            void* stream) {
  PA_CHECK_ARG(o_parts && lse_parts && o, "pa_lse_merge: null pointer");
  PA_CHECK_ARG(n_parts >= 1 && n_parts <= pa::kMaxParts, "pa_lse_merge: n_parts=%d not in [1, %d]", n_parts,
               pa::kMaxParts);
  PA_CHECK_ARG(BH >= 0 && N >= 0 && D >= 1, "pa_lse_merge: bad shape");
  pa::MergeArgs a;
  for (int k = 0; k < pa::kMaxParts; ++k) {
    a.o[k] = k < n_parts ? o_parts[k] : nullptr;
    a.lse[k] = k < n_parts ? lse_parts[k] : nullptr;
    if (k < n_parts) PA_CHECK_ARG(a.o[k] && a.lse[k], "pa_lse_merge: part %d is null", k);
  }
  a.n = n_parts;
  const int64_t rows = BH * N;
  if (rows == 0) return PA_OK;
  hipStream_t s = static_cast<hipStream_t>(stream);
  const dim3 grid((unsigned)((rows + 3) / 4));
  switch (out_dtype) {
    case PA_F32:
      hipLaunchKernelGGL(pa::lse_merge_kernel<float>, grid, dim3(256), 0, s, a, static_cast<float*>(o),
                         lse_out, rows, D);
      break;
    case PA_F16:
      hipLaunchKernelGGL(pa::lse_merge_kernel<_Float16>, grid, dim3(256), 0, s, a,
                         static_cast<_Float16*>(o), lse_out, rows, D);
      break;
    case PA_BF16:
      hipLaunchKernelGGL(pa::lse_merge_kernel<__bf16>, grid, dim3(256), 0, s, a, static_cast<__bf16*>(o),
                         lse_out, rows, D);
      break;
    default:
      PA_CHECK_ARG(false, "pa_lse_merge: unknown out_dtype %d", out_dtype);
  }
  PA_LAUNCH_CHECK("lse_merge_kernel");
  return PA_OK;
}
