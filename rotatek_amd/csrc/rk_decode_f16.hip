// rk_decode_f16.hip -- the F16 instantiations of the decode kernels and
// their launcher (declared in rk_decode.h).
#include "rk_decode_dev.h"

namespace rk {

hipError_t decode_launch_f16(int dkb, bool vec, int hmax, bool has_vis, const DecodeArgs& a, dim3 grid,
                             hipStream_t s) {
  return launch_dk<F16>(dkb, vec, hmax, has_vis, a, grid, s);
}

}  // namespace rk
