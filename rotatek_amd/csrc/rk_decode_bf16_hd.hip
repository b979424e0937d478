// rk_decode_bf16_hd.hip -- the BF16 decode kernels with 16-byte row loads
// for head_dim < 128 (channels past head_dim masked), and their launcher
// (declared in rk_decode.h).
#include "rk_decode_dev.h"

namespace rk {

hipError_t decode_launch_bf16_hd(int dkb, int hmax, bool has_vis, const DecodeArgs& a, dim3 grid, hipStream_t s) {
  return launch_dk<BF16, true>(dkb, true, hmax, has_vis, a, grid, s);
}

}  // namespace rk
