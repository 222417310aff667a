// Instantiations and launch of the streaming attention kernel (f16, bf16; D = 128, BQ = 128).
#include "attn_stream.hpp"

namespace pa {

template <typename T>
static int launch_stream_t(const AttnK& a, hipStream_t s, const char* name) {
  // the dynamic LDS limit is raised once per device
  static unsigned long long configured = 0ull;
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return hip_fail(e, "hipGetDevice");
  if (dev >= 64 || !((configured >> dev) & 1ull)) {
    e = hipFuncSetAttribute(reinterpret_cast<const void*>(&attn_stream_kernel<T>),
                            hipFuncAttributeMaxDynamicSharedMemorySize, kStreamSmem);
    if (e != hipSuccess) return hip_fail(e, "hipFuncSetAttribute(attn_stream_kernel)");
    if (dev < 64) configured |= 1ull << dev;
  }
  hipLaunchKernelGGL(attn_stream_kernel<T>, dim3((unsigned)a.total_wg), dim3(256), kStreamSmem, s, a);
  PA_LAUNCH_CHECK(name);
  return PA_OK;
}

int launch_attn_stream(const AttnK& a, int dtype, hipStream_t s) {
  if (dtype == PA_BF16) return launch_stream_t<__bf16>(a, s, "attn_stream_kernel<bf16>");
  return launch_stream_t<_Float16>(a, s, "attn_stream_kernel<f16>");
}

}  // namespace pa
