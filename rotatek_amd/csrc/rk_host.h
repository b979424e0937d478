// rk_host.h -- host-side helpers shared by the C ABI entry points:
// descriptor validation (no HIP calls, so it runs without a GPU), dtype
// sizes, the 16-byte fast-path test and the per-device CU cache.
#pragma once

#include <stdint.h>

#include "rotatek_hip.h"

namespace rk {

inline int dtype_size(int d) {
  switch (d) {
    case RK_F16:
    case RK_BF16: return 2;
    case RK_F32:
    case RK_I32: return 4;
    case RK_F64:
    case RK_I64: return 8;
    case RK_U8: return 1;
    default: return 0;
  }
}

inline bool is_half(int d) { return d == RK_F16 || d == RK_BF16; }

// torch's mean scale factor, float(n_out) / float(n_in), formed in float as
// ATen's GPU mean kernels form it (MeanOps multiplies the fp32 sum by it).
// n_in == 0 gives inf, so the mean of nothing is NaN, as torch's is.
inline float mean_factor(int64_t n_out, int64_t n_in) {
  return static_cast<float>(n_out) / static_cast<float>(n_in);
}
inline bool is_float_param(int d) { return d == RK_F16 || d == RK_BF16 || d == RK_F32; }

// Rank, non-negative sizes and strides, and no int64 overflow of the
// largest element offset.  `data` may be NULL here (host-only checks).
inline int check_desc(const rk_tensor* t, int ndim) {
  if (!t) return RK_ERR_NULL;
  if (t->ndim != ndim) return RK_ERR_RANK;
  int64_t span = 0;
  for (int i = 0; i < ndim; ++i) {
    if (t->shape[i] < 0) return RK_ERR_SHAPE;
    if (t->stride[i] < 0) return RK_ERR_STRIDE;
    if (t->shape[i] > 0) {
      const int64_t ext = t->shape[i] - 1;
      if (t->stride[i] != 0 && ext > (INT64_C(1) << 61) / t->stride[i]) return RK_ERR_STRIDE;
      span += ext * t->stride[i];
      if (span > (INT64_C(1) << 61)) return RK_ERR_STRIDE;
    }
  }
  return RK_OK;
}

inline int64_t numel(const rk_tensor* t) {
  int64_t n = 1;
  for (int i = 0; i < t->ndim; ++i) n *= t->shape[i];
  return n;
}

// 16-byte vector loads along the last dim are legal: unit last stride,
// every other stride a multiple of 8 elements, 16-byte aligned base.
inline bool vec_ok(const rk_tensor* t) {
  if (!t) return true;
  if (t->stride[t->ndim - 1] != 1 && t->shape[t->ndim - 1] > 1) return false;
  for (int i = 0; i < t->ndim - 1; ++i)
    if (t->shape[i] > 1 && (t->stride[i] % 8) != 0) return false;
  return (((uintptr_t)t->data) & 15) == 0;
}

// CU count of the current HIP device (cached per device); 0 on failure.
int current_device_cus(int* device_out);

// Whether the current device is gfx942 or gfx950, whose write-through
// agent-scope stores and coherent agent-scope loads the single-launch
// decode merge relies on (cached per device; false on failure).
bool device_has_coherent_tickets();

}  // namespace rk
