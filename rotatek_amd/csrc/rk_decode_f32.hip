// rk_decode_f32.hip -- the fp32 decode kernel (decode32_kernel) and its merge,
// and their launcher (declared in rk_decode.h).
#include "rk_decode_dev.h"

namespace rk {

template <int HG>
hipError_t launch32(bool has_vis, bool vec, const DecodeArgs& a, dim3 grid, hipStream_t s) {
  if (has_vis) {
    if (vec)
      hipLaunchKernelGGL((decode32_kernel<true, true, HG>), grid, dim3(kThreads), 0, s, a);
    else
      hipLaunchKernelGGL((decode32_kernel<true, false, HG>), grid, dim3(kThreads), 0, s, a);
  } else {
    if (vec)
      hipLaunchKernelGGL((decode32_kernel<false, true, HG>), grid, dim3(kThreads), 0, s, a);
    else
      hipLaunchKernelGGL((decode32_kernel<false, false, HG>), grid, dim3(kThreads), 0, s, a);
  }
  return hipGetLastError();
}

// One query head per unit (hpu 1), or up to 8 of one KV head
hipError_t decode_launch_f32(bool has_vis, bool vec, const DecodeArgs& a, dim3 grid, hipStream_t s) {
  if (a.hpu > 8) return hipErrorInvalidValue;
  hipError_t e = a.hpu > 1 ? launch32<8>(has_vis, vec, a, grid, s) : launch32<1>(has_vis, vec, a, grid, s);
  if (e != hipSuccess || a.fused) return e;
  hipLaunchKernelGGL((merge_kernel<F32>), dim3(merge_grid(a)), dim3(kThreads), 0, s, a);
  return hipGetLastError();
}

}  // namespace rk
