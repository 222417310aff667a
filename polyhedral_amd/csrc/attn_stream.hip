// Instantiations and launches of the streaming attention kernels (f16, bf16; D = 128,
// BQ = 128): one work-group per (query block, head), or a persistent run of items per
// work-group.
#include "attn_run.hpp"

namespace pa {

template <typename K>
static int raise_lds_limit(K kernel, unsigned long long& configured, const char* what) {
  // the dynamic LDS limit is raised once per device
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return hip_fail(e, "hipGetDevice");
  if (dev >= 64 || !((configured >> dev) & 1ull)) {
    e = hipFuncSetAttribute(reinterpret_cast<const void*>(kernel), hipFuncAttributeMaxDynamicSharedMemorySize,
                            kStreamSmem);
    if (e != hipSuccess) return hip_fail(e, what);
    if (dev < 64) configured |= 1ull << dev;
  }
  return PA_OK;
}

template <typename T, bool SPLIT, int MODE = 0>
static int launch_stream_t(const AttnK& a, hipStream_t s, const char* name) {
  static unsigned long long configured = 0ull;
  if (int rc = raise_lds_limit(&attn_stream_kernel<T, SPLIT, MODE>, configured, "hipFuncSetAttribute(attn_stream_kernel)"))
    return rc;
  hipLaunchKernelGGL((attn_stream_kernel<T, SPLIT, MODE>), dim3((unsigned)a.total_wg), dim3(256), kStreamSmem, s, a);
  PA_LAUNCH_CHECK(name);
  return PA_OK;
}

// the mode a launch's arguments allow (0: every option read at run time)
static int stream_mode(const AttnK& a) {
  if (a.A != 32) return 0;
  // a merge input must be 2-byte (the previous partial in the output's layout) for modes 3, 4
  const int merge = !a.prev_o ? 0 : a.prev_dtype != PA_F32 ? 2 : -1;
  if (merge < 0) return 0;
  const bool none = a.residue_s == 0 && !a.gather_q && !a.gather_kv && !a.scatter_o && !a.pred.perm_q && !a.pred.perm_kv;
  if (none) return 1 + merge;
  // (a query block of 128 rows then lies inside one class's segment of N / s rows)
  if (a.residue_s > 0 && a.residue_qlog2 >= 7 && a.gather_q && a.gather_kv && a.scatter_o) return 2 + merge;
  return 0;
}

template <typename T>
static int launch_run_t(const AttnK& a, int groups, bool cooperative, hipStream_t s, const char* name) {
  static unsigned long long configured = 0ull;
  if (int rc = raise_lds_limit(&attn_run_kernel<T>, configured, "hipFuncSetAttribute(attn_run_kernel)")) return rc;
  if (!cooperative) {
    hipLaunchKernelGGL(attn_run_kernel<T>, dim3((unsigned)groups), dim3(256), kStreamSmem, s, a);
    PA_LAUNCH_CHECK(name);
    return PA_OK;
  }
  // A run whose items wait for each other needs every work-group resident at once: a
  // cooperative launch, refused by the runtime when the grid cannot be.
  int dev = 0, per_cu = 0, cus = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e == hipSuccess) e = hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev);
  if (e == hipSuccess)
    e = hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, reinterpret_cast<const void*>(&attn_run_kernel<T>), 256,
                                                     kStreamSmem);
  if (e != hipSuccess) return hip_fail(e, "occupancy of attn_run_kernel");
  PA_CHECK_ARG((int64_t)groups <= (int64_t)per_cu * cus,
               "pa_attn_fwd_split: %d work-groups cannot all be resident (%d per CU x %d CUs)", groups, per_cu, cus);
  AttnK args = a;
  void* params[] = {&args};
  e = hipLaunchCooperativeKernel(reinterpret_cast<const void*>(&attn_run_kernel<T>), dim3((unsigned)groups), dim3(256),
                                 params, kStreamSmem, s);
  if (e != hipSuccess) return hip_fail(e, name);
  return PA_OK;
}

int launch_attn_stream(const AttnK& a, int dtype, hipStream_t s) {
  const int mode = stream_mode(a);
  if (dtype == PA_BF16) {
    switch (mode) {
      case 1: return launch_stream_t<__bf16, false, 1>(a, s, "attn_stream_kernel<bf16, index space>");
      case 2: return launch_stream_t<__bf16, false, 2>(a, s, "attn_stream_kernel<bf16, residue basis>");
      case 3: return launch_stream_t<__bf16, false, 3>(a, s, "attn_stream_kernel<bf16, index space, merge>");
      case 4: return launch_stream_t<__bf16, false, 4>(a, s, "attn_stream_kernel<bf16, residue basis, merge>");
      default: return launch_stream_t<__bf16, false>(a, s, "attn_stream_kernel<bf16>");
    }
  }
  switch (mode) {
    case 1: return launch_stream_t<_Float16, false, 1>(a, s, "attn_stream_kernel<f16, index space>");
    case 2: return launch_stream_t<_Float16, false, 2>(a, s, "attn_stream_kernel<f16, residue basis>");
    case 3: return launch_stream_t<_Float16, false, 3>(a, s, "attn_stream_kernel<f16, index space, merge>");
    case 4: return launch_stream_t<_Float16, false, 4>(a, s, "attn_stream_kernel<f16, residue basis, merge>");
    default: return launch_stream_t<_Float16, false>(a, s, "attn_stream_kernel<f16>");
  }
}

int launch_attn_split_grid(const AttnK& a, int dtype, hipStream_t s) {
  if (dtype == PA_BF16) return launch_stream_t<__bf16, true>(a, s, "attn_stream_kernel<bf16, split>");
  return launch_stream_t<_Float16, true>(a, s, "attn_stream_kernel<f16, split>");
}

int launch_attn_run(const AttnK& a, int groups, int dtype, bool cooperative, hipStream_t s) {
  if (dtype == PA_BF16) return launch_run_t<__bf16>(a, groups, cooperative, s, "attn_run_kernel<bf16>");
  return launch_run_t<_Float16>(a, groups, cooperative, s, "attn_run_kernel<f16>");
}

}  // namespace pa
