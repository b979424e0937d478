// Top-k eigenbasis by truncated subspace iteration with Cholesky-QR
// orthonormalisation (rotation.py:21-91), for the 128 x 128 Key covariances
// of every (batch, KV head), k <= 64.
//
// Per iteration, as the reference:
//   W = C V;  G = W^T W;  G += eps * mean(diag G) * I;  G = L L^T;  V = W L^-T
// One 256-thread workgroup owns one matrix and keeps everything in LDS
// (C 128 x 129, V/W 128 x (KP+1), G/L KP x (KP+1), padded rows: ~116 KB at
// KP = 64):
//   W = C V       thread tile 4 rows x KP/8 columns, fp32 FMA
//   G = W^T W     thread tile (KP/16) x (KP/16)
//   Cholesky      wave 0, lane i holds row i of G in registers; the pivot
//                 and column entries are read across lanes (readlane)
//   V = W L^-T    right-looking forward substitution per row (threads 0..127)
// The start block V0 comes from the caller (the reference draws it with
// torch.randn from a seeded device generator, rotation.py:88-90).  Columns
// k..KP-1 are zero padding; their G block is set to the identity so they
// stay zero.
#include <math.h>

#include "rk_common.h"
#include "rk_host.h"
#include "rotatek_hip.h"

namespace rk {
namespace rot {

constexpr int kD = 128;
constexpr int kThreads = 256;
constexpr int kCPad = kD + 1;

template <int KP>
__global__ void __launch_bounds__(kThreads) power_iter_kernel(
    const float* cov, int64_t c_sb, int64_t c_sh, int64_t c_sr, int64_t c_sc, const float* v0, int64_t v_sb,
    int64_t v_sh, int64_t v_sr, int64_t v_sc, float* out, int64_t o_sb, int64_t o_sh, int64_t o_sr,
    int64_t o_sc, int H, int k, int iters, float eps) {
  constexpr int TC = KP / 8;    // W tile columns per thread
  constexpr int GT = KP / 16;   // G tile edge per thread
  constexpr int GP = KP + 1;    // padded G row
  constexpr int SP = KP + 1;    // padded V row (row-per-thread access in the solve)
  __shared__ float sC[kD * kCPad];
  __shared__ float sV[kD * SP];
  __shared__ float sG[KP * GP];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int bh = blockIdx.x, b = bh / H, h = bh - b * H;
  const float* C = cov + b * c_sb + (int64_t)h * c_sh;
  const float* V0 = v0 + b * v_sb + (int64_t)h * v_sh;

  // Stage C and V0 in LDS.  The loads of a batch are all issued before any
  // of them is stored, so the copy costs a few memory round trips rather
  // than one per element.
  constexpr int kCB = 16;  // elements per thread per batch
  for (int e0 = 0; e0 < kD * kD; e0 += kThreads * kCB) {
    float v[kCB];
#pragma unroll
    for (int i = 0; i < kCB; ++i) {
      const int e = e0 + i * kThreads + tid, r = e >> 7, c = e & 127;
      v[i] = C[r * c_sr + c * c_sc];
    }
#pragma unroll
    for (int i = 0; i < kCB; ++i) {
      const int e = e0 + i * kThreads + tid;
      sC[(e >> 7) * kCPad + (e & 127)] = v[i];
    }
  }
  constexpr int kVB = kD * KP / kThreads < kCB ? kD * KP / kThreads : kCB;  // divides kD * KP / kThreads
  static_assert((kD * kD) % (kThreads * kCB) == 0 && (kD * KP) % (kThreads * kVB) == 0, "whole batches");
  for (int e0 = 0; e0 < kD * KP; e0 += kThreads * kVB) {
    float v[kVB];
#pragma unroll
    for (int i = 0; i < kVB; ++i) {
      const int e = e0 + i * kThreads + tid, r = e / KP, c = e - r * KP;
      v[i] = c < k ? V0[r * v_sr + c * v_sc] : 0.f;
    }
#pragma unroll
    for (int i = 0; i < kVB; ++i) {
      const int e = e0 + i * kThreads + tid, r = e / KP;
      sV[r * SP + (e - r * KP)] = v[i];
    }
  }
  __syncthreads();

  const int rg = tid >> 3, cg = tid & 7;           // W tile: rows 4 rg.., columns TC cg..
  const int gi = tid >> 4, gj = tid & 15;          // G tile: rows GT gi.., columns GT gj..
  for (int it = 0; it < iters; ++it) {
    // ---- W = C V (registers), then back into sV
    float w[4][TC];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int c = 0; c < TC; ++c) w[i][c] = 0.f;
#pragma unroll 8
    for (int d = 0; d < kD; ++d) {
      float cv[4], vv[TC];
#pragma unroll
      for (int i = 0; i < 4; ++i) cv[i] = sC[(4 * rg + i) * kCPad + d];
#pragma unroll
      for (int c = 0; c < TC; ++c) vv[c] = sV[d * SP + TC * cg + c];
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int c = 0; c < TC; ++c) w[i][c] = fmaf(cv[i], vv[c], w[i][c]);
    }
    __syncthreads();
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int c = 0; c < TC; ++c) sV[(4 * rg + i) * SP + TC * cg + c] = w[i][c];
    __syncthreads();

    // ---- G = W^T W
    {
      float g[GT][GT];
#pragma unroll
      for (int i = 0; i < GT; ++i)
#pragma unroll
        for (int j = 0; j < GT; ++j) g[i][j] = 0.f;
#pragma unroll 8
      for (int r = 0; r < kD; ++r) {
        float a[GT], bb[GT];
#pragma unroll
        for (int i = 0; i < GT; ++i) a[i] = sV[r * SP + GT * gi + i];
#pragma unroll
        for (int j = 0; j < GT; ++j) bb[j] = sV[r * SP + GT * gj + j];
#pragma unroll
        for (int i = 0; i < GT; ++i)
#pragma unroll
          for (int j = 0; j < GT; ++j) g[i][j] = fmaf(a[i], bb[j], g[i][j]);
      }
#pragma unroll
      for (int i = 0; i < GT; ++i)
#pragma unroll
        for (int j = 0; j < GT; ++j) sG[(GT * gi + i) * GP + GT * gj + j] = g[i][j];
    }
    __syncthreads();

    // ---- ridge and Cholesky (wave 0; lane i owns row i)
    if (wave == 0) {
      float dg = lane < k ? sG[lane * GP + lane] : 0.f;
#pragma unroll
      for (int off = 32; off > 0; off >>= 1) dg += shfl_xor(dg, off);
      const float ridge = eps * (dg / (float)k);
      float row[KP];
#pragma unroll
      for (int m = 0; m < KP; ++m) {
        float x = lane < KP ? sG[min(lane, KP - 1) * GP + m] : 0.f;
        if (lane >= k || m >= k) x = (lane == m) ? 1.f : 0.f;  // identity on the padding
        else if (lane == m) x += ridge;
        row[m] = x;
      }
#pragma unroll
      for (int j = 0; j < KP; ++j) {
        const float ljj =
            sqrtf(__builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, row[j]), j)));
        const float lij = lane > j ? row[j] / ljj : (lane == j ? ljj : row[j]);
        row[j] = lij;
#pragma unroll
        for (int m = j + 1; m < KP; ++m) {
          const float lmj = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, lij), m));
          if (lane >= m) row[m] = fmaf(-lij, lmj, row[m]);
        }
      }
      if (lane < KP) {
#pragma unroll
        for (int m = 0; m < KP; ++m) sG[lane * GP + m] = m <= lane ? row[m] : 0.f;
      }
    }
    __syncthreads();

    // ---- V = W L^-T: row r solves L x^T = w^T by forward substitution,
    // right-looking (x_j final, then subtracted from every later unknown), so
    // the dependency chain is two operations per column rather than j
    if (tid < kD) {
      float x[KP];
#pragma unroll
      for (int j = 0; j < KP; ++j) x[j] = sV[tid * SP + j];
#pragma unroll
      for (int j = 0; j < KP; ++j) {
        x[j] = x[j] / sG[j * GP + j];
#pragma unroll
        for (int i = j + 1; i < KP; ++i) x[i] = fmaf(-sG[i * GP + j], x[j], x[i]);
      }
#pragma unroll
      for (int j = 0; j < KP; ++j) sV[tid * SP + j] = x[j];
    }
    __syncthreads();
  }

  float* O = out + b * o_sb + (int64_t)h * o_sh;
  for (int e = tid; e < kD * k; e += kThreads) {
    const int r = e / k, c = e - (e / k) * k;
    O[r * o_sr + c * o_sc] = sV[r * SP + c];
  }
}

template <int KP>
hipError_t launch(const rk_tensor* cov, const rk_tensor* v0, const rk_tensor* out, int64_t BH, int H, int k,
                  int iters, float eps, hipStream_t s) {
  hipLaunchKernelGGL((power_iter_kernel<KP>), dim3((unsigned)BH), dim3(kThreads), 0, s, (const float*)cov->data,
                     cov->stride[0], cov->stride[1], cov->stride[2], cov->stride[3], (const float*)v0->data,
                     v0->stride[0], v0->stride[1], v0->stride[2], v0->stride[3], (float*)out->data, out->stride[0],
                     out->stride[1], out->stride[2], out->stride[3], H, k, iters, eps);
  return hipGetLastError();
}

}  // namespace rot
}  // namespace rk

extern "C" int rk_power_iteration(const rk_tensor* cov, const rk_tensor* v0, const rk_tensor* out,
                                  int32_t num_iters, float eps, void* stream) {
  using namespace rk::rot;
  if (!cov || !v0 || !out) return RK_ERR_NULL;
  int st;
  if ((st = rk::check_desc(cov, 4)) || (st = rk::check_desc(v0, 4)) || (st = rk::check_desc(out, 4))) return st;
  if (cov->dtype != RK_F32 || v0->dtype != RK_F32 || out->dtype != RK_F32) return RK_ERR_DTYPE;
  if (cov->shape[2] != kD || cov->shape[3] != kD) return RK_ERR_HEAD_DIM;
  const int64_t B = cov->shape[0], H = cov->shape[1], k = v0->shape[3];
  for (const rk_tensor* t : {v0, out})
    if (t->shape[0] != B || t->shape[1] != H || t->shape[2] != kD || t->shape[3] != k) return RK_ERR_SHAPE;
  if (k < 1 || k > 64) return RK_ERR_KEEP_DIM;
  if (num_iters < 0 || !(eps >= 0.f)) return RK_ERR_ARG;
  if (B * H == 0) return RK_OK;
  if (B * H > (INT64_C(1) << 31) || H > (INT64_C(1) << 30)) return RK_ERR_SHAPE;
  if (!cov->data || !v0->data || !out->data) return RK_ERR_NULL;
  hipStream_t s = (hipStream_t)stream;
  hipError_t e;
  if (k <= 16)
    e = launch<16>(cov, v0, out, B * H, (int)H, (int)k, num_iters, eps, s);
  else if (k <= 32)
    e = launch<32>(cov, v0, out, B * H, (int)H, (int)k, num_iters, eps, s);
  else
    e = launch<64>(cov, v0, out, B * H, (int)H, (int)k, num_iters, eps, s);
  return e == hipSuccess ? RK_OK : RK_ERR_HIP;
}
