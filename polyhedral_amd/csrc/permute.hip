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
typedef uint32_t pu32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t pu32x2 __attribute__((ext_vector_type(2)));
template <>
struct Unit<16> { using type = pu32x4; };
template <>
struct Unit<8> { using type = pu32x2; };
template <>
struct Unit<4> { using type = uint32_t; };
template <>
struct Unit<1> { using type = uint8_t; };

// Up to kMaxStack tensors of one shape moved by the same launch (the same row index
// serves all of them), and optionally their position ids.
constexpr int kMaxStack = 8;
struct Stack {
  const char* src[kMaxStack];
  char* dst[kMaxStack];
  int32_t n;
};

// Each thread moves kUnroll units (16 bytes each when the rows allow) spaced by the grid
// size, every tensor of the stack for each.  The data moves with non-temporal loads and
// stores: the rows are touched once, and keeping them out of the caches took the gather
// from 3.5 to 6.2 TB/s.  Unrolling over several units per thread was measured slower
// (kUnroll 2 / 4 / 8: 5.9 / 5.8 / 4.6 TB/s), so each thread takes one unit.
constexpr int kUnroll = 1;

template <int VB, typename I>
__global__ __launch_bounds__(256) void permute_rows_kernel(const Stack st, const int32_t* __restrict__ perm,
                                                            I BH, I N, I units_per_row, int64_t s_bh,
                                                            int64_t s_row, int64_t d_bh, int64_t d_row,
                                                            int32_t inverse, const int64_t* __restrict__ pos_in,
                                                            int64_t* __restrict__ pos_out) {
  using U = typename Unit<VB>::type;
  const I total = BH * N * units_per_row;
  const I T = (I)gridDim.x * blockDim.x;
  for (I i0 = (I)blockIdx.x * blockDim.x + threadIdx.x; i0 < total; i0 += (I)kUnroll * T) {
    I p[kUnroll], b[kUnroll], u[kUnroll];
    int32_t other[kUnroll];
#pragma unroll
    for (int k = 0; k < kUnroll; ++k) {
      const I i = i0 + (I)k * T;
      const I ii = i < total ? i : 0;
      u[k] = ii % units_per_row;
      const I rp = ii / units_per_row;  // (bh, p) flattened
      p[k] = rp % N;
      b[k] = rp / N;
      other[k] = i < total ? perm[p[k]] : -1;
    }
    int64_t so[kUnroll], dof[kUnroll];
    bool ok[kUnroll];
#pragma unroll
    for (int k = 0; k < kUnroll; ++k) {
      ok[k] = other[k] >= 0 && (I)other[k] < N;  // not a permutation entry: touch nothing
      const int64_t sr = inverse ? (int64_t)p[k] : (int64_t)other[k];
      const int64_t dr = inverse ? (int64_t)other[k] : (int64_t)p[k];
      so[k] = (int64_t)b[k] * s_bh + sr * s_row + (int64_t)u[k] * VB;
      dof[k] = (int64_t)b[k] * d_bh + dr * d_row + (int64_t)u[k] * VB;
      // position ids travel with the tokens (written once, by the first unit of batch-head 0)
      if (ok[k] && pos_out && b[k] == 0 && u[k] == 0) pos_out[dr] = pos_in ? pos_in[sr] : sr;
    }
    for (int t = 0; t < st.n; ++t) {
      U val[kUnroll];
#pragma unroll
      for (int k = 0; k < kUnroll; ++k)
        if (ok[k]) val[k] = __builtin_nontemporal_load(reinterpret_cast<const U*>(st.src[t] + so[k]));
#pragma unroll
      for (int k = 0; k < kUnroll; ++k)
        if (ok[k]) __builtin_nontemporal_store(val[k], reinterpret_cast<U*>(st.dst[t] + dof[k]));
    }
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

namespace pa {
namespace {

int permute_stack(const void* const* srcs, void* const* dsts, int32_t n, const int32_t* perm, int64_t BH,
                  int64_t N, int64_t row_bytes, int64_t src_bh_stride, int64_t src_row_stride,
                  int64_t dst_bh_stride, int64_t dst_row_stride, const int64_t* pos_in, int64_t* pos_out,
                  int32_t inverse, void* stream, const char* name) {
  PA_CHECK_ARG(srcs && dsts && perm, "%s: null pointer", name);
  PA_CHECK_ARG(n >= 0 && n <= kMaxStack, "%s: %d tensors (at most %d)", name, n, kMaxStack);
  PA_CHECK_ARG(BH >= 0 && N >= 0 && row_bytes >= 0, "%s: negative size", name);
  Stack st{};
  st.n = n;
  for (int t = 0; t < n; ++t) {
    PA_CHECK_ARG(srcs[t] && dsts[t], "%s: null tensor %d", name, t);
    PA_CHECK_ARG(srcs[t] != dsts[t], "%s: in-place permutation is not supported", name);
    st.src[t] = static_cast<const char*>(srcs[t]);
    st.dst[t] = static_cast<char*>(dsts[t]);
  }
  if (BH == 0 || N == 0 || (row_bytes == 0 && !pos_out) || (n == 0 && !pos_out)) return PA_OK;
  hipStream_t s = static_cast<hipStream_t>(stream);
  auto fits = [&](int64_t vb) {
    if (row_bytes % vb || src_bh_stride % vb || src_row_stride % vb || dst_bh_stride % vb || dst_row_stride % vb)
      return false;
    for (int t = 0; t < n; ++t)
      if (!aligned(st.src[t], vb) || !aligned(st.dst[t], vb)) return false;
    return true;
  };
  // positions only: one unit per row
  const int64_t rb = row_bytes > 0 && n > 0 ? row_bytes : 1;
  if (row_bytes == 0 || n == 0) st.n = 0;
#define PA_PERM_LAUNCH(VB)                                                                         \
  do {                                                                                             \
    const int64_t upr = rb / VB;                                                                   \
    const unsigned grid = grid_for(BH * N * upr, 256 * kUnroll);                                   \
    if (BH * N * upr < (1ll << 31))                                                                \
      hipLaunchKernelGGL((permute_rows_kernel<VB, uint32_t>), dim3(grid), dim3(256), 0, s, st, perm, \
                         (uint32_t)BH, (uint32_t)N, (uint32_t)upr, src_bh_stride, src_row_stride,  \
                         dst_bh_stride, dst_row_stride, inverse, pos_in, pos_out);                 \
    else                                                                                           \
      hipLaunchKernelGGL((permute_rows_kernel<VB, uint64_t>), dim3(grid), dim3(256), 0, s, st, perm, \
                         (uint64_t)BH, (uint64_t)N, (uint64_t)upr, src_bh_stride, src_row_stride,  \
                         dst_bh_stride, dst_row_stride, inverse, pos_in, pos_out);                 \
  } while (0)
  if (st.n == 0)
    PA_PERM_LAUNCH(1);
  else if (fits(16))
    PA_PERM_LAUNCH(16);
  else if (fits(8))
    PA_PERM_LAUNCH(8);
  else if (fits(4))
    PA_PERM_LAUNCH(4);
  else
    PA_PERM_LAUNCH(1);
#undef PA_PERM_LAUNCH
  PA_LAUNCH_CHECK(name);
  return PA_OK;
}

}  // namespace
}  // namespace pa

extern "C" int pa_permute_rows(const void* src, void* dst, const int32_t* perm, int64_t BH, int64_t N,
                               int64_t row_bytes, int64_t src_bh_stride, int64_t src_row_stride,
                               int64_t dst_bh_stride, int64_t dst_row_stride, int32_t inverse,
                               void* stream) {
  PA_CHECK_ARG(src && dst && perm, "pa_permute_rows: null pointer");
  void* d = dst;
  return pa::permute_stack(&src, &d, 1, perm, BH, N, row_bytes, src_bh_stride, src_row_stride, dst_bh_stride,
                           dst_row_stride, nullptr, nullptr, inverse, stream, "pa_permute_rows");
}

extern "C" int pa_permute_stack(const void* const* srcs, void* const* dsts, int32_t n_tensors,
                                const int32_t* perm, int64_t BH, int64_t N, int64_t row_bytes,
                                int64_t src_bh_stride, int64_t src_row_stride, int64_t dst_bh_stride,
                                int64_t dst_row_stride, const int64_t* pos_in, int64_t* pos_out,
                                int32_t inverse, void* stream) {
  return pa::permute_stack(srcs, dsts, n_tensors, perm, BH, N, row_bytes, src_bh_stride, src_row_stride,
                           dst_bh_stride, dst_row_stride, pos_in, pos_out, inverse, stream, "pa_permute_stack");
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
