// rk_decode_f32.hip -- the fp32 decode kernel (decode32_kernel) and its merge,
// and their launcher (declared in rk_decode.h).
#include "rk_decode_dev.h"

namespace rk {

hipError_t decode_launch_f32(bool has_vis, bool vec, const DecodeArgs& a, dim3 grid, hipStream_t s) {
  if (has_vis) {
    if (vec)
      hipLaunchKernelGGL((decode32_kernel<true, true>), grid, dim3(kThreads), 0, s, a);
    else
      hipLaunchKernelGGL((decode32_kernel<true, false>), grid, dim3(kThreads), 0, s, a);
  } else {
    if (vec)
      hipLaunchKernelGGL((decode32_kernel<false, true>), grid, dim3(kThreads), 0, s, a);
    else
      hipLaunchKernelGGL((decode32_kernel<false, false>), grid, dim3(kThreads), 0, s, a);
  }
  hipError_t e = hipGetLastError();
  if (e != hipSuccess || a.fused) return e;
  hipLaunchKernelGGL((merge_kernel<F32>), dim3(merge_grid(a)), dim3(kThreads), 0, s, a);
  return hipGetLastError();
}

}  // namespace rk
