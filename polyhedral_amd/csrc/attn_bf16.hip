// Instantiations of the attention kernel for element type __bf16 (D = 64, 128; 1, 2, 4 waves).
#include "attn_kernel.hpp"

namespace pa {

template <int D, int NW>
static int launch_one(const AttnK& a, hipStream_t s) {
  constexpr int smem = attn_smem_bytes<__bf16, D, NW>();
  static bool configured = false;
  if (!configured) {
    hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(&attn_fwd_kernel<__bf16, D, NW>),
                                       hipFuncAttributeMaxDynamicSharedMemorySize, smem);
    if (e != hipSuccess) return hip_fail(e, "hipFuncSetAttribute(attn_fwd_kernel)");
    configured = true;
  }
  hipLaunchKernelGGL((attn_fwd_kernel<__bf16, D, NW>), dim3((unsigned)a.total_wg), dim3(NW * 64), smem, s, a);
  PA_LAUNCH_CHECK("attn_fwd_kernel<bf16>");
  return PA_OK;
}

int launch_attn_bf16(const AttnK& a, int D, int NW, hipStream_t s) {
  if (D == 64 && NW == 1) return launch_one<64, 1>(a, s);
  if (D == 64 && NW == 2) return launch_one<64, 2>(a, s);
  if (D == 64 && NW == 4) return launch_one<64, 4>(a, s);
  if (D == 128 && NW == 1) return launch_one<128, 1>(a, s);
  if (D == 128 && NW == 2) return launch_one<128, 2>(a, s);
  if (D == 128 && NW == 4) return launch_one<128, 4>(a, s);
  set_error("attention: no bf16 kernel for D=%d with %d waves", D, NW);
  return PA_E_UNSUPPORTED;
}

}  // namespace pa
