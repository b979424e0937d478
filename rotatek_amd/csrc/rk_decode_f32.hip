// rk_decode_f32.hip -- the fp32 decode kernels (decode32_kernel, decode32g_kernel) and their merge,
// and their launcher (declared in rk_decode.h).
#include "rk_decode_dev.h"

namespace rk {

template <bool G8, bool DFULL>
hipError_t launch32(bool has_vis, bool vec, const DecodeArgs& a, dim3 grid, hipStream_t s) {
  auto go = [&](auto kernel) { hipLaunchKernelGGL(kernel, grid, dim3(kThreads), 0, s, a); };
  if constexpr (G8) {
    if (has_vis)
      vec ? go(decode32g_kernel<true, true, 8, DFULL>) : go(decode32g_kernel<true, false, 8, DFULL>);
    else
      vec ? go(decode32g_kernel<false, true, 8, DFULL>) : go(decode32g_kernel<false, false, 8, DFULL>);
  } else {
    if (has_vis)
      vec ? go(decode32_kernel<true, true, DFULL>) : go(decode32_kernel<true, false, DFULL>);
    else
      vec ? go(decode32_kernel<false, true, DFULL>) : go(decode32_kernel<false, false, DFULL>);
  }
  return hipGetLastError();
}

// One query head per unit (hpu 1), or up to 8 of one KV head
hipError_t decode_launch_f32(bool has_vis, bool vec, const DecodeArgs& a, dim3 grid, hipStream_t s) {
  if (a.hpu > 8) return hipErrorInvalidValue;
  const bool full = a.D == 128;
  hipError_t e = a.hpu > 1 ? (full ? launch32<true, true>(has_vis, vec, a, grid, s)
                                   : launch32<true, false>(has_vis, vec, a, grid, s))
                           : (full ? launch32<false, true>(has_vis, vec, a, grid, s)
                                   : launch32<false, false>(has_vis, vec, a, grid, s));
  if (e != hipSuccess || a.fused) return e;
  hipLaunchKernelGGL((merge_kernel<F32>), dim3(merge_grid(a)), dim3(kThreads), 0, s, a);
  return hipGetLastError();
}

}  // namespace rk
