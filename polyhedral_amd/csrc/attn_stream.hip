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

template <typename T, bool SPLIT>
static int launch_stream_t(const AttnK& a, hipStream_t s, const char* name) {
  static unsigned long long configured = 0ull;
  if (int rc = raise_lds_limit(&attn_stream_kernel<T, SPLIT>, configured, "hipFuncSetAttribute(attn_stream_kernel)"))
    return rc;
  hipLaunchKernelGGL((attn_stream_kernel<T, SPLIT>), dim3((unsigned)a.total_wg), dim3(256), kStreamSmem, s, a);
  PA_LAUNCH_CHECK(name);
  return PA_OK;
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
  if (dtype == PA_BF16) return launch_stream_t<__bf16, false>(a, s, "attn_stream_kernel<bf16>");
  return launch_stream_t<_Float16, false>(a, s, "attn_stream_kernel<f16>");
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
