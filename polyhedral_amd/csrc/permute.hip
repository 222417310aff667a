// Class-A residue permutation on the GPU: row gather / scatter of [BH, N, D]
// tensors, permutation inverse and the closed-form residue permutation.
// Replaces gpu/permute.py:12-31 (numpy argsort + torch index_select).
//
// The copy is HBM-bound: each work-item moves one 16-byte unit, consecutive
// lanes cover consecutive units of a row, so every row (256 B for bf16 D=128)
// is read and written as whole 64-B segments.
#include "common.hpp"

namespace pa {
namespace {

template <int VB>
struct Unit;
template <>
struct Unit<16> { using type = uint4; };
template <>
struct Unit<8> { using type = uint2; };
template <>
struct Unit<4> { using type = uint32_t; };
template <>
struct Unit<1> { using type = uint8_t; };

template <int VB, typename I>
__global__ __launch_bounds__(256) void permute_rows_kernel(const char* __restrict__ src,
                                                            char* __restrict__ dst,
                                                            const int32_t* __restrict__ perm, I BH, I N,
                                                            I units_per_row, int64_t s_bh, int64_t s_row,
                                                            int64_t d_bh, int64_t d_row, int32_t inverse) {
  using U = typename Unit<VB>::type;
  const I total = BH * N * units_per_row;
  for (I i = (I)blockIdx.x * blockDim.x + threadIdx.x; i < total; i += (I)gridDim.x * blockDim.x) {
    const I u = i % units_per_row;
    const I rp = i / units_per_row;  // (bh, p) flattened
    const I p = rp % N;
    const I b = rp / N;
    const int32_t other = perm[p];
    if (other < 0 || (I)other >= N) continue;  // not a permutation entry: touch nothing
    const int64_t sr = inverse ? (int64_t)p : (int64_t)other;
    const int64_t dr = inverse ? (int64_t)other : (int64_t)p;
    const U val = *reinterpret_cast<const U*>(src + (int64_t)b * s_bh + sr * s_row + (int64_t)u * VB);
    *reinterpret_cast<U*>(dst + (int64_t)b * d_bh + dr * d_row + (int64_t)u * VB) = val;
  }
}

__global__ void invert_kernel(const int32_t* __restrict__ perm, int32_t* __restrict__ inv, int64_t N) {
  const int64_t p = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (p < N) {
    const int32_t t = perm[p];
    if (t >= 0 && t < N) inv[t] = (int32_t)p;
  }
}

// Permuted position p -> original i for the stable sort by (i mod s, i div s).
// With N = Q s + R, classes c < R hold Q + 1 positions and classes c >= R hold Q.
__global__ void residue_perm_kernel(int32_t* __restrict__ perm, int64_t N, int64_t s) {
  const int64_t p = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (p >= N) return;
  const int64_t Q = N / s, R = N % s;
  int64_t c, u;
  if (p < R * (Q + 1)) {
    c = p / (Q + 1);
    u = p % (Q + 1);
  } else {
    const int64_t pp = p - R * (Q + 1);
    c = R + pp / Q;
    u = pp % Q;
  }
  perm[p] = (int32_t)(u * s + c);
}

unsigned grid_for(int64_t work, int64_t per_block) {
  int64_t g = (work + per_block - 1) / per_block;
  const int64_t cap = 1 << 20;
  return (unsigned)(g < 1 ? 1 : (g > cap ? cap : g));
}

bool aligned(const void* p, int64_t a) { return (reinterpret_cast<uintptr_t>(p) % a) == 0; }

}  // namespace
}  // namespace pa

extern "C" int pa_permute_rows(const void* src, void* dst, const int32_t* perm, int64_t BH, int64_t N,
                               int64_t row_bytes, int64_t src_bh_stride, int64_t src_row_stride,
                               int64_t dst_bh_stride, int64_t dst_row_stride, int32_t inverse,
                               void* stream) {
  PA_CHECK_ARG(src && dst && perm, "pa_permute_rows: null pointer");
  PA_CHECK_ARG(BH >= 0 && N >= 0 && row_bytes >= 0, "pa_permute_rows: negative size");
  PA_CHECK_ARG(src != dst, "pa_permute_rows: in-place permutation is not supported");
  if (BH == 0 || N == 0 || row_bytes == 0) return PA_OK;
  hipStream_t s = static_cast<hipStream_t>(stream);
  auto fits = [&](int64_t vb) {
    return row_bytes % vb == 0 && src_bh_stride % vb == 0 && src_row_stride % vb == 0 &&
           dst_bh_stride % vb == 0 && dst_row_stride % vb == 0 && pa::aligned(src, vb) &&
           pa::aligned(dst, vb);
  };
#define PA_PERM_LAUNCH(VB)                                                                         \
  do {                                                                                             \
    const int64_t upr = row_bytes / VB;                                                            \
    const unsigned grid = pa::grid_for(BH * N * upr, 256);                                         \
    if (BH * N * upr < (1ll << 31))                                                                \
      hipLaunchKernelGGL((pa::permute_rows_kernel<VB, uint32_t>), dim3(grid), dim3(256), 0, s,     \
                         static_cast<const char*>(src), static_cast<char*>(dst), perm,             \
                         (uint32_t)BH, (uint32_t)N, (uint32_t)upr, src_bh_stride, src_row_stride,  \
                         dst_bh_stride, dst_row_stride, inverse);                                  \
    else                                                                                           \
      hipLaunchKernelGGL((pa::permute_rows_kernel<VB, uint64_t>), dim3(grid), dim3(256), 0, s,     \
                         static_cast<const char*>(src), static_cast<char*>(dst), perm,             \
                         (uint64_t)BH, (uint64_t)N, (uint64_t)upr, src_bh_stride, src_row_stride,  \
                         dst_bh_stride, dst_row_stride, inverse);                                  \
  } while (0)
  if (fits(16))
    PA_PERM_LAUNCH(16);
  else if (fits(8))
    PA_PERM_LAUNCH(8);
  else if (fits(4))
    PA_PERM_LAUNCH(4);
  else
    PA_PERM_LAUNCH(1);
#undef PA_PERM_LAUNCH
  PA_LAUNCH_CHECK("permute_rows_kernel");
  return PA_OK;
}

extern "C" int pa_invert_perm(const int32_t* perm, int32_t* inv, int64_t N, void* stream) {
  PA_CHECK_ARG(perm && inv && N >= 0, "pa_invert_perm: bad argument");
  if (N == 0) return PA_OK;
  hipLaunchKernelGGL(pa::invert_kernel, dim3(pa::grid_for(N, 256)), dim3(256), 0,
                     static_cast<hipStream_t>(stream), perm, inv, N);
  PA_LAUNCH_CHECK("invert_kernel");
  return PA_OK;
}

extern "C" int pa_residue_perm(int32_t* perm, int64_t N, int32_t s, void* stream) {
  PA_CHECK_ARG(perm && N >= 0 && s >= 1, "pa_residue_perm: bad argument (N=%lld, s=%d)", (long long)N, s);
  PA_CHECK_ARG(N <= (1ll << 31) - 1, "pa_residue_perm: N=%lld exceeds int32 positions", (long long)N);
  if (N == 0) return PA_OK;
  hipLaunchKernelGGL(pa::residue_perm_kernel, dim3(pa::grid_for(N, 256)), dim3(256), 0,
                     static_cast<hipStream_t>(stream), perm, N, (int64_t)s);
  PA_LAUNCH_CHECK("residue_perm_kernel");
  return PA_OK;
}
