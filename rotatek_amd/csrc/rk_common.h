// rk_common.h -- device helpers shared by the RotateK HIP kernels (gfx950).
//
// Wave64 conventions used throughout: lane = threadIdx.x & 63, the wave is
// four 16-lane rows, g = lane >> 4 is the row and n = lane & 15 the column.
// The MFMA helpers wrap v_mfma_f32_16x16x32_{f16,bf16}: for D = A x B + C
// (A 16x32, B 32x16) lane (g, n) supplies A[n][8g..8g+7] and B[8g..8g+7][n]
// and receives D[4g+i][n], i = 0..3.  Only the pairing of A's and B's k
// index matters to the kernels, so they never depend on how the hardware
// orders k inside a lane.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace rk {

typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

constexpr float kLog2e = 1.4426950408889634f;
constexpr float kNegInit = -1e30f;  // running-max start (fused_decode.py:151)
constexpr float kDenomEps = 1e-6f;  // output guard (fused_decode.py:293)

// ------------------------------------------------------------ dtype traits
struct F16 {
  using elem = _Float16;
  using vec8 = f16x8;
  static constexpr int kBytes = 2;
  static constexpr int32_t kRk = 0;  // its rk_dtype code (RK_F16)
  static __device__ __forceinline__ float to_f32(uint16_t b) {
    return (float)__builtin_bit_cast(_Float16, b);
  }
  static __device__ __forceinline__ uint16_t from_f32(float x) {
    return __builtin_bit_cast(uint16_t, (_Float16)x);
  }
  // (lo, hi) rounded to nearest even and packed into one dword
  static __device__ __forceinline__ uint32_t pack2(float lo, float hi) {
    typedef float f2 __attribute__((ext_vector_type(2)));
    typedef _Float16 h2 __attribute__((ext_vector_type(2)));
    return __builtin_bit_cast(uint32_t, __builtin_convertvector((f2){lo, hi}, h2));
  }
  static __device__ __forceinline__ f32x4 mfma(uint4 a, uint4 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a),
                                                  __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
  }
  // lo 16 bits of the result hold x rounded; hi/lo split helper
  static __device__ __forceinline__ void split(float x, uint16_t& hi, uint16_t& lo) {
    _Float16 h = (_Float16)x;
    hi = __builtin_bit_cast(uint16_t, h);
    lo = __builtin_bit_cast(uint16_t, (_Float16)(x - (float)h));
  }
  // split() of eight values packed as two MFMA operands (element r in half
  // r of the words): one value per conversion, which measured faster in the
  // decode kernel than the packed two-value conversion
  static __device__ __forceinline__ void split8(const float (&x)[8], uint4& hi, uint4& lo) {
    uint32_t h[8], l[8];
#pragma unroll
    for (int r = 0; r < 8; ++r) {
      uint16_t a, b;
      split(x[r], a, b);
      h[r] = a;
      l[r] = b;
    }
    hi = make_uint4(h[0] | (h[1] << 16), h[2] | (h[3] << 16), h[4] | (h[5] << 16), h[6] | (h[7] << 16));
    lo = make_uint4(l[0] | (l[1] << 16), l[2] | (l[3] << 16), l[4] | (l[5] << 16), l[6] | (l[7] << 16));
  }
};

struct BF16 {
  using elem = __bf16;
  using vec8 = bf16x8;
  static constexpr int kBytes = 2;
  static constexpr int32_t kRk = 1;  // its rk_dtype code (RK_BF16)
  static __device__ __forceinline__ float to_f32(uint16_t b) {
    return __builtin_bit_cast(float, (uint32_t)b << 16);
  }
  // round to nearest even (v_cvt_pk_bf16_f32 on gfx950)
  static __device__ __forceinline__ uint16_t from_f32(float x) {
    return __builtin_bit_cast(uint16_t, (__bf16)x);
  }
  // (lo, hi) rounded to nearest even and packed into one dword
  static __device__ __forceinline__ uint32_t pack2(float lo, float hi) {
    typedef float f2 __attribute__((ext_vector_type(2)));
    typedef __bf16 b2 __attribute__((ext_vector_type(2)));
    return __builtin_bit_cast(uint32_t, __builtin_convertvector((f2){lo, hi}, b2));
  }
  // the two halves of a packed dword as fp32
  static __device__ __forceinline__ float lo_f32(uint32_t w) { return __builtin_bit_cast(float, w << 16); }
  static __device__ __forceinline__ float hi_f32(uint32_t w) { return __builtin_bit_cast(float, w & 0xffff0000u); }
  static __device__ __forceinline__ f32x4 mfma(uint4 a, uint4 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a),
                                                   __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
  }
  static __device__ __forceinline__ void split(float x, uint16_t& hi, uint16_t& lo) {
    hi = from_f32(x);
    lo = from_f32(x - to_f32(hi));
  }
  // split() of eight values packed as two MFMA operands: two values per
  // packed conversion (v_cvt_pk_bf16_f32), the same roundings
  static __device__ __forceinline__ void split8(const float (&x)[8], uint4& hi, uint4& lo) {
    uint32_t h[4], l[4];
#pragma unroll
    for (int w = 0; w < 4; ++w) {
      h[w] = pack2(x[2 * w], x[2 * w + 1]);
      l[w] = pack2(x[2 * w] - lo_f32(h[w]), x[2 * w + 1] - hi_f32(h[w]));
    }
    hi = make_uint4(h[0], h[1], h[2], h[3]);
    lo = make_uint4(l[0], l[1], l[2], l[3]);
  }
};

// fp32 storage (the fp32 decode path: outputs written as they are computed;
// the fp32 prefill path: "rounding to the key dtype" is the identity).
struct F32 {
  static constexpr int kBytes = 4;
  static constexpr int32_t kRk = 2;  // its rk_dtype code (RK_F32)
  static __device__ __forceinline__ float to_f32(uint32_t b) { return __builtin_bit_cast(float, b); }
  static __device__ __forceinline__ uint32_t from_f32(float x) { return __builtin_bit_cast(uint32_t, x); }
  // v_mfma_f32_16x16x4_f32: lane (g, n) supplies A[n][g] and B[g][n] and
  // receives D[4g + i][n], i = 0..3 (fp32 products, fp32 accumulation)
  static __device__ __forceinline__ f32x4 mfma(float a, float b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
  }
};

// Scalar load of one element of a runtime dtype (0 f16, 1 bf16, 2 f32).
__device__ __forceinline__ float load_any(const void* p, int64_t idx, int dtype) {
  if (dtype == 2) return ((const float*)p)[idx];
  uint16_t b = ((const uint16_t*)p)[idx];
  return dtype == 0 ? F16::to_f32(b) : BF16::to_f32(b);
}

// N elements p[idx0 + i * stride] of a launch-uniform dtype: one branch on
// the dtype, then N loads issued back to back (load_any per element puts
// each load in its own branch, and each then waits for its data).
template <int N>
__device__ __forceinline__ void load_any_n(const void* p, int64_t idx0, int64_t stride, int dtype,
                                           float (&out)[N]) {
  if (dtype == 2) {
    const float* f = (const float*)p;
#pragma unroll
    for (int i = 0; i < N; ++i) out[i] = f[idx0 + i * stride];
  } else {
    const uint16_t* h = (const uint16_t*)p;
    uint16_t r[N];
#pragma unroll
    for (int i = 0; i < N; ++i) r[i] = h[idx0 + i * stride];
    if (dtype == 0) {
#pragma unroll
      for (int i = 0; i < N; ++i) out[i] = F16::to_f32(r[i]);
    } else {
#pragma unroll
      for (int i = 0; i < N; ++i) out[i] = BF16::to_f32(r[i]);
    }
  }
}

// Rows row0 .. row0 + N - 1 of one column (element base + row * stride) of a
// launch-uniform dtype, as load_any_n; rows at or past nrows are zero (their
// loads read the column's first row, in bounds).  Addresses step from the
// column pointer one row at a time, so none is held across the loads.
template <int N>
__device__ __forceinline__ void load_any_rows(const void* p, int64_t base, int64_t stride, int dtype, int row0,
                                              int nrows, float (&out)[N]) {
  if (dtype == 2) {
    const float* f = (const float*)p + base;
#pragma unroll
    for (int i = 0; i < N; ++i) out[i] = f[row0 + i < nrows ? (int64_t)(row0 + i) * stride : 0];
  } else {
    const uint16_t* h = (const uint16_t*)p + base;
    uint16_t r[N];
#pragma unroll
    for (int i = 0; i < N; ++i) r[i] = h[row0 + i < nrows ? (int64_t)(row0 + i) * stride : 0];
    if (dtype == 0) {
#pragma unroll
      for (int i = 0; i < N; ++i) out[i] = F16::to_f32(r[i]);
    } else {
#pragma unroll
      for (int i = 0; i < N; ++i) out[i] = BF16::to_f32(r[i]);
    }
  }
#pragma unroll
  for (int i = 0; i < N; ++i) out[i] = row0 + i < nrows ? out[i] : 0.f;
}

// Split form of load_any for prologues: load_raw issues the load (32 bits
// for F32, 16 bits otherwise, chosen by a dtype that is uniform across the
// launch), raw_to_f32 converts later, so the wait for the data can be placed
// after other loads have been issued.
__device__ __forceinline__ uint32_t load_raw(const void* p, int64_t idx, int dtype) {
  return dtype == 2 ? ((const uint32_t*)p)[idx] : (uint32_t)((const uint16_t*)p)[idx];
}
__device__ __forceinline__ float raw_to_f32(uint32_t v, int dtype) {
  return dtype == 2 ? __builtin_bit_cast(float, v)
                    : (dtype == 0 ? F16::to_f32((uint16_t)v) : BF16::to_f32((uint16_t)v));
}

// ------------------------------------------------------------ memory
// Eight 16-bit elements starting at `p` with element stride `sd`; `nvalid`
// of them (from the front) are read, the rest are zero.  VEC: one 16-byte
// load (caller guarantees sd == 1, 16-byte alignment, nvalid in {0, 8}).
template <bool VEC>
__device__ __forceinline__ uint4 load8(const uint16_t* p, int64_t sd, int nvalid) {
  if constexpr (VEC) {
    if (nvalid <= 0) return make_uint4(0, 0, 0, 0);
    return *(const uint4*)p;
  } else {
    uint32_t w[4] = {0, 0, 0, 0};
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      uint32_t v = (e < nvalid) ? (uint32_t)p[e * sd] : 0u;
      w[e >> 1] |= v << ((e & 1) * 16);
    }
    return make_uint4(w[0], w[1], w[2], w[3]);
  }
}

__device__ __forceinline__ uint32_t word(const uint4& v, int i) {
  return i == 0 ? v.x : i == 1 ? v.y : i == 2 ? v.z : v.w;
}

// Pack (lo16 of a, lo16 of b) or (hi16 of a, hi16 of b) into one dword.
__device__ __forceinline__ uint32_t pack_lo(uint32_t a, uint32_t b) {
  return __builtin_amdgcn_perm(b, a, 0x05040100u);
}
__device__ __forceinline__ uint32_t pack_hi(uint32_t a, uint32_t b) {
  return __builtin_amdgcn_perm(b, a, 0x07060302u);
}

// ------------------------------------------------------------ cross-lane
__device__ __forceinline__ float shfl_xor(float v, int mask) {
  return __builtin_bit_cast(float, __shfl_xor(__builtin_bit_cast(int, v), mask, 64));
}

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

}  // namespace rk
