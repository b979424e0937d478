// Top-k eigenbasis by truncated subspace iteration with Cholesky-QR
// orthonormalisation (rotation.py:21-91), for the 128 x 128 Key covariances
// of every (batch, KV head), k <= 128 (k <= 64 here; wider bases in
// power_iter128_kernel below).
//
// Per iteration, as the reference:
//   W = C V;  G = W^T W;  G += eps * mean(diag G) * I;  G = L L^T;  V = W L^-T
// One 256-thread workgroup owns one matrix and keeps everything in LDS
// (C 128 x 132, V/W 128 x (KP+4), G KP x (KP+1), L KP x KP, (L^-1)^T
// KP x (KP+4), 4 KB scratch: 153 KB at KP = 64).  The three products run on v_mfma_f32_16x16x4_f32:
//   W = C V            8 x KP/16 tiles of 16 x 16 over the four waves
//   G = W^T W          (KP/16)^2 tiles
//   Cholesky + L^-1    KP <= 32: one pass in wave 0 (lane i holds row i of
//                      G; column j of L goes through LDS and serves both
//                      the row updates and step j of the substitution
//                      L x = e_c that lane c runs for column c of L^-1).
//                      KP = 64: 16-column panels, each factored in wave 0
//                      with its diagonal block of L^-1; the trailing update
//                      of G and the blocks of L^-1 below the diagonal run
//                      on the MFMA over all waves (141.7 -> 100.5 us for 32
//                      matrices at k = 64; no gain at k <= 32)
//   V = W (L^-1)^T     8 x KP/16 tiles
// Padding columns of V are zero, so their rows and columns of G are too: a
// unit diagonal there makes that block the identity, and V keeps them zero.
// The start block V0 comes from the caller (the reference draws it with
// torch.randn from a seeded device generator, rotation.py:88-90).
#include <math.h>

#include "rk_common.h"
#include "rk_host.h"
#include "rotatek_hip.h"

namespace rk {
namespace rot {

typedef __attribute__((address_space(3))) float lds_f32;
typedef __attribute__((address_space(3))) f32x4 lds_f32x4;

constexpr int kD = 128;
constexpr int kThreads = 256;
constexpr int kCPad = kD + 4;  // C row stride: 16-byte reads of rows n = 0..15 cover all 64 banks
constexpr int kLook = 3;       // single-pass Cholesky: column entries passed by readlane ahead of the LDS broadcast

// D = A B + D on v_mfma_f32_16x16x4_f32 (A 16x4, B 4x16): lane (g, n) supplies
// A[n][g] and B[g][n] and holds D[4g + i][n], i = 0..3.
__device__ __forceinline__ f32x4 mfma4(float a, float b, f32x4 d) {
  return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, d, 0, 0, 0);
}

// The LDS address of p, through an empty asm the compiler cannot see into.
__device__ __forceinline__ lds_f32* opaque_lds(float* p) {
  unsigned a = (unsigned)(uintptr_t)(lds_f32*)p;
  asm volatile("" : "+v"(a));
  return (lds_f32*)(uintptr_t)a;
}

template <int KP>
__global__ void __launch_bounds__(kThreads) power_iter_kernel(
    const float* cov, int64_t c_sb, int64_t c_sh, int64_t c_sr, int64_t c_sc, const float* v0, int64_t v_sb,
    int64_t v_sh, int64_t v_sr, int64_t v_sc, float* out, int64_t o_sb, int64_t o_sh, int64_t o_sr,
    int64_t o_sc, int H, int k, int iters, float eps, int32_t* info, int D) {
  // V / W and (L^-1)^T row stride, 4 mod 16: reads of rows 4g + r (r fixed)
  // at columns n = 0..15 hit banks 16g + n, and 16-byte reads of rows n at
  // column 4g cover all 64 banks
  constexpr int SP = KP + 4;
  constexpr int LP = KP + 4;
  constexpr int GP = KP + 1;        // G row (row per lane in the Cholesky)
  constexpr int NTJ = KP / 16;      // 16-column tiles of W / V
  constexpr int TPW = 8 * NTJ / 4;  // 16 x 16 tiles of W per wave
  constexpr int NG = NTJ * NTJ;     // 16 x 16 tiles of G
  constexpr int TPG = NG >= 4 ? NG / 4 : 1;
  constexpr int NP16 = KP / 16;     // Cholesky panels
  __shared__ __align__(16) float sC[kD * kCPad];
  __shared__ __align__(16) float sV[kD * SP];
  // G, then L by columns; the tail takes the idle lanes' last column writes
  // G (the single-pass path rewrites it as L by columns; its tail takes the
  // idle lanes' last column writes)
  __shared__ __align__(16) float sG[KP * GP > KP * KP + 64 ? KP * GP : KP * KP + 64];
  // blocked path: L by columns, sLc[j * KP + m] = L_mj (1 / L_jj on the diagonal)
  __shared__ __align__(16) float sLc[KP > 32 ? KP * KP : 1];
  // X = L^-1 transposed, sLt[c * LP + i] = X[i][c]; rows >= KP: scratch for
  // the single-pass path's idle lanes
  __shared__ float sLt[64 * LP];
  __shared__ float sT[KP > 32 ? 4 * 256 : 1];  // blocked path: per-wave 16 x 16 product scratch

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, g = lane >> 4, n = lane & 15;
  const int bh = blockIdx.x, b = bh / H, h = bh - b * H;
  const float* C = cov + b * c_sb + (int64_t)h * c_sh;
  const float* V0 = v0 + b * v_sb + (int64_t)h * v_sh;

  // Stage C and V0 in LDS.  The loads of a batch are all issued before any
  // of them is stored, so the copy costs a few memory round trips rather
  // than one per element.  With a head_dim D < 128 the rows and columns
  // past D are zeros (their loads re-read an in-bounds entry): W = C V, G,
  // L and V = W L^-T then equal the D x D iteration's, with exact zeros in
  // the padded rows.
  constexpr int kCB = 16;  // elements per thread per batch
  if (D == kD) {  // (the addresses step by two rows per element, no clamps)
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
  } else {
    for (int e0 = 0; e0 < kD * kD; e0 += kThreads * kCB) {
      float v[kCB];
#pragma unroll
      for (int i = 0; i < kCB; ++i) {
        const int e = e0 + i * kThreads + tid, r = e >> 7, c = e & 127;
        const float x = C[min(r, D - 1) * c_sr + min(c, D - 1) * c_sc];
        v[i] = r < D && c < D ? x : 0.f;
      }
#pragma unroll
      for (int i = 0; i < kCB; ++i) {
        const int e = e0 + i * kThreads + tid;
        sC[(e >> 7) * kCPad + (e & 127)] = v[i];
      }
    }
  }
  constexpr int kVB = kD * KP / kThreads < kCB ? kD * KP / kThreads : kCB;  // divides kD * KP / kThreads
  static_assert((kD * kD) % (kThreads * kCB) == 0 && (kD * KP) % (kThreads * kVB) == 0, "whole batches");
  for (int e0 = 0; e0 < kD * KP; e0 += kThreads * kVB) {
    float v[kVB];
#pragma unroll
    for (int i = 0; i < kVB; ++i) {
      const int e = e0 + i * kThreads + tid, r = e / KP, c = e - r * KP;
      v[i] = c < k && r < D ? V0[r * v_sr + c * v_sc] : 0.f;
    }
#pragma unroll
    for (int i = 0; i < kVB; ++i) {
      const int e = e0 + i * kThreads + tid, r = e / KP;
      sV[r * SP + (e - r * KP)] = v[i];
    }
  }
  for (int e = tid; e < 64 * LP; e += kThreads) sLt[e] = 0.f;  // X's upper blocks are never written
  __syncthreads();

  // Wave w owns the 16 x 16 output tiles w, w + 4, w + 8, ... of each
  // product.  With NTJ column tiles (NTJ divides 4) tile w + 4t sits at row
  // tile ti0 + t * RS and column tile tj0.
  constexpr int RS = 4 / NTJ;
  const int ti0 = wave / NTJ, tj0 = wave - (wave / NTJ) * NTJ;
  // a pivot that is not positive and finite (wave 0, uniform)
  bool bad = false;

  for (int it = 0; it < iters; ++it) {
    // LDS bases, opaque to the compiler once per iteration: every access
    // below is one of these plus a lane part plus an immediate offset
    // (< 64 KB), so no per-access address is kept in a register across
    // iterations
    lds_f32* const lC = opaque_lds(sC);
    lds_f32* const lV = opaque_lds(sV);
    lds_f32* const lG = opaque_lds(sG);
    lds_f32* const lLt = opaque_lds(sLt);
    lds_f32* const lLc = opaque_lds(sLc);
    lds_f32* const lT = opaque_lds(sT);

    // ---- W = C V on the MFMA.  In the four MFMA steps of k-group q, lane
    // (g, n) supplies k = 16q + 4g + r, r = 0..3 (any assignment of k to
    // (step, g) sums the same products), so one 16-byte read of C's row
    // feeds all four; group q + 1 is read while group q computes
    {
      const lds_f32* pa = lC + (16 * ti0 + n) * kCPad + 4 * g;  // C[16 ti + n][16 q + 4 g + r]
      const lds_f32* pb = lV + 4 * g * SP + 16 * tj0 + n;       // V[16 q + 4 g + r][16 tj + n]
      f32x4 acc[TPW], a[2][TPW];
      float bv[2][4];
#pragma unroll
      for (int t = 0; t < TPW; ++t) acc[t] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int t = 0; t < TPW; ++t) a[0][t] = *(const lds_f32x4*)&pa[16 * RS * t * kCPad];
#pragma unroll
      for (int r = 0; r < 4; ++r) bv[0][r] = pb[r * SP];
#pragma unroll
      for (int q = 0; q < kD / 16; ++q) {
        const int cur = q & 1, nxt = cur ^ 1;
        if (q + 1 < kD / 16) {
#pragma unroll
          for (int t = 0; t < TPW; ++t) a[nxt][t] = *(const lds_f32x4*)&pa[16 * RS * t * kCPad + 16 * (q + 1)];
#pragma unroll
          for (int r = 0; r < 4; ++r) bv[nxt][r] = pb[(16 * (q + 1) + r) * SP];
        }
#pragma unroll
        for (int r = 0; r < 4; ++r)
#pragma unroll
          for (int t = 0; t < TPW; ++t) acc[t] = mfma4(a[cur][t][r], bv[cur][r], acc[t]);
      }
      __syncthreads();
      lds_f32* pw = lV + (16 * ti0 + 4 * g) * SP + 16 * tj0 + n;
#pragma unroll
      for (int t = 0; t < TPW; ++t)
#pragma unroll
        for (int i = 0; i < 4; ++i) pw[(16 * RS * t + i) * SP] = acc[t][i];
    }
    __syncthreads();

    // ---- G = W^T W on the MFMA (NTJ x NTJ tiles; at NTJ = 1 wave 0 alone),
    // k assigned as in C V (lane (g, n) takes rows 16q + 4g + r); two
    // accumulators per tile (even / odd r) so consecutive MFMAs do not wait
    // on each other
    if (wave < NG) {  // wave-uniform
      const lds_f32* pa = lV + 4 * g * SP + 16 * ti0 + n;  // W[16 q + 4 g + r][16 ti + n]
      const lds_f32* pb = lV + 4 * g * SP + 16 * tj0 + n;  // W[16 q + 4 g + r][16 tj + n]
      f32x4 acc[TPG][2];
#pragma unroll
      for (int t = 0; t < TPG; ++t) acc[t][0] = acc[t][1] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll 2
      for (int q = 0; q < kD / 16; ++q) {
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const float bv = pb[(16 * q + r) * SP];
#pragma unroll
          for (int t = 0; t < TPG; ++t)
            acc[t][r & 1] = mfma4(pa[(16 * q + r) * SP + 16 * RS * t], bv, acc[t][r & 1]);
        }
      }
      lds_f32* pg = lG + (16 * ti0 + 4 * g) * GP + 16 * tj0 + n;
#pragma unroll
      for (int t = 0; t < TPG; ++t)
#pragma unroll
        for (int i = 0; i < 4; ++i) pg[(16 * RS * t + i) * GP] = acc[t][0][i] + acc[t][1][i];
    }
    __syncthreads();

    if constexpr (KP <= 32) {
    // ---- ridge, Cholesky G = L L^T and L^-1, one pass in wave 0.
    // Lane i holds row i of G.  Step j takes the pivot from lane j, scales
    // column j by r_j = 1/sqrt(pivot) and publishes it to LDS (column j of
    // L, with r_j in place of L_jj); every lane reads the column back as
    // 16-byte broadcasts and uses it twice: the right-looking update of its
    // row of G, and step j of the forward substitution L x = e_c that lane
    // c runs for column c of L^-1.  Rows of finished lanes (lane <= j) keep
    // being updated in their upper triangle, which is never read.
    if (wave == 0) {
      // the lane index, opaque to the compiler, so that the per-column lane
      // masks below are formed where they are used instead of being hoisted
      // out of the iteration loop (where they would not fit in registers)
      int ln = lane;
      asm volatile("" : "+v"(ln));
      const int lr = min(ln, KP - 1);  // lanes >= KP compute on a copy of row KP-1 and store nothing
      const lds_f32* prow = lG + lr * GP;
      const float dii = prow[lr];
      float dg = ln < k ? dii : 0.f;
#pragma unroll
      for (int off = 32; off > 0; off >>= 1) dg += shfl_xor(dg, off);
      const float ridge = eps * (dg / (float)k);
      // the padding rows and columns of G are zero (V's padding columns
      // are): a unit diagonal there makes them the identity
      if (ln < KP) lG[ln * GP + ln] = ln < k ? dii + ridge : 1.f;
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
      __builtin_amdgcn_wave_barrier();
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
      float row[KP], x[KP];
#pragma unroll
      for (int m = 0; m < KP; ++m) {
        row[m] = prow[m];
        x[m] = ln == m ? 1.f : 0.f;
      }
      // G's storage is rewritten below as L by columns (sL[j * KP + m] =
      // L_mj), after every lane's loads above
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
      __builtin_amdgcn_wave_barrier();
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
      lds_f32* const sL = lG;
      // column j is written unconditionally (a guarded store per step would
      // split the pass into blocks and let the compiler sink the
      // substitution to the end): lanes >= KP write past column j, into
      // columns that are rewritten before they are read, or into the tail
      // of the array
      lds_f32* const pl = lG + ln;
#pragma unroll
      for (int j = 0; j < KP; ++j) {
        const float piv = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, row[j]), j));
        bad |= !(piv > 0.f && piv <= 3.402823466e38f);
        const float rj = __builtin_amdgcn_rsqf(piv);
        const float lij = ln > j ? row[j] * rj : (ln == j ? rj : 0.f);
        pl[j * KP] = lij;
        x[j] *= rj;
        // the entries the next kLook pivots depend on, L_{j+1..j+kLook, j},
        // come straight from their lanes; the rest of the column goes
        // through LDS, whose round trip then has kLook steps to complete
#pragma unroll
        for (int d = 1; d <= kLook; ++d) {
          if (j + d < KP) {  // compile-time
            const float c = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, lij), j + d));
            row[j + d] = fmaf(-lij, c, row[j + d]);
            x[j + d] = fmaf(-c, x[j], x[j + d]);
          }
        }
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
#pragma unroll
        for (int m4 = (j + kLook + 1) & ~3; m4 < KP; m4 += 4) {
          const f32x4 col = *(const lds_f32x4*)&sL[j * KP + m4];
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            const int m = m4 + q;
            if (m > j + kLook) {  // compile-time
              row[m] = fmaf(-lij, col[q], row[m]);
              x[m] = fmaf(-col[q], x[j], x[m]);
            }
          }
        }
      }
      // unconditional (rows KP..63 of the array take the idle lanes'
      // values and are never read): a guarded store would let the compiler
      // sink the whole substitution into it, holding every column read
      // above in registers until the end
      lds_f32* px = lLt + ln * LP;
#pragma unroll
      for (int i = 0; i < KP; ++i) px[i] = x[i];
    }
    __syncthreads();
    } else {
    // ---- ridge: G += eps * mean(diag G) * I (wave 0); the padding rows
    // and columns of G are zero (V's padding columns are): a unit diagonal
    // there makes them the identity
    if (wave == 0) {
      const int lr = min(lane, KP - 1);
      const float dii = lG[lr * GP + lr];
      float dg = lane < k ? dii : 0.f;
#pragma unroll
      for (int off = 32; off > 0; off >>= 1) dg += shfl_xor(dg, off);
      const float ridge = eps * (dg / (float)k);
      if (lane < KP) lG[lane * GP + lane] = lane < k ? dii + ridge : 1.f;
    }
    __syncthreads();

    // ---- blocked Cholesky G = L L^T and X = L^-1, 16-column panels.
    // Panel p: wave 0 factors columns 16p..16p+15 (lane i holds those
    // entries of row i; the entries of column j that the panel's later
    // columns need come lane to lane by readlane), writes them to sLc by
    // columns (r_j = 1 / L_jj on the diagonal) and, in lanes 16p..16p+15,
    // the diagonal block of X by forward substitution.  All waves then
    // subtract the panel's product from the trailing lower tiles of G on
    // the MFMA.  Afterwards X's blocks below the diagonal follow by block
    // rows: X_qr = -X_qq (sum_{s=r}^{q-1} L_qs X_sr), two 16 x 16 MFMA
    // products per tile.  X goes to sLt transposed (row c = column c of X,
    // the layout the solve below reads); its upper blocks stay zero.
#pragma unroll
    for (int p = 0; p < NP16; ++p) {
      const int P0 = 16 * p;
      if (wave == 0) {
        const int lr = min(lane, KP - 1);  // lanes >= KP work on a copy of row KP-1 and store nothing
        const lds_f32* prow = lG + lr * GP + P0;
        float a[16], xv[16], lc[16];
#pragma unroll
        for (int c = 0; c < 16; ++c) {
          a[c] = prow[c];
          xv[c] = lane == P0 + c ? 1.f : 0.f;
        }
#pragma unroll
        for (int jj = 0; jj < 16; ++jj) {
          const int j = P0 + jj;
          const float piv = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, a[jj]), j));
          bad |= !(piv > 0.f && piv <= 3.402823466e38f);
          const float rj = __builtin_amdgcn_rsqf(piv);
          const float lij = lane > j ? a[jj] * rj : (lane == j ? rj : 0.f);
          lc[jj] = lij;
          xv[jj] *= rj;
#pragma unroll
          for (int mm = jj + 1; mm < 16; ++mm) {
            const float c = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, lij), P0 + mm));
            a[mm] = fmaf(-lij, c, a[mm]);
            xv[mm] = fmaf(-c, xv[jj], xv[mm]);
          }
        }
        if (lane < KP) {
#pragma unroll
          for (int jj = 0; jj < 16; ++jj) lLc[(P0 + jj) * KP + lane] = lc[jj];
        }
        if (lane >= P0 && lane < P0 + 16) {
#pragma unroll
          for (int mm = 0; mm < 16; ++mm) lLt[lane * LP + P0 + mm] = xv[mm];
        }
      }
      __syncthreads();
      if (p + 1 < NP16) {
        // G[16 ti + a][16 tj + b] -= sum_c L[16 ti + a][P0 + c] L[16 tj + b][P0 + c]
        // over the lower tiles p < tj <= ti < NP16, tile t to wave t mod 4
        int t = 0;
#pragma unroll
        for (int ti = p + 1; ti < NP16; ++ti) {
#pragma unroll
          for (int tj = p + 1; tj <= ti; ++tj, ++t) {
            if (t % 4 == wave) {  // wave-uniform
              f32x4 acc = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
              for (int st = 0; st < 4; ++st) {
                const int cc = P0 + 4 * st + g;
                acc = mfma4(lLc[cc * KP + 16 * ti + n], lLc[cc * KP + 16 * tj + n], acc);
              }
              lds_f32* pg = lG + (16 * ti + 4 * g) * GP + 16 * tj + n;
#pragma unroll
              for (int i = 0; i < 4; ++i) pg[i * GP] -= acc[i];
            }
          }
        }
        __syncthreads();
      }
    }
#pragma unroll
    for (int q = 1; q < NP16; ++q) {
      if (wave < q) {  // tile (q, r = wave)
        const int r = wave;
        f32x4 tacc = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int s = 0; s < NP16 - 1; ++s) {
          if (s >= r && s < q) {  // wave-uniform
#pragma unroll
            for (int st = 0; st < 4; ++st) {
              const int kk = 16 * s + 4 * st + g;
              tacc = mfma4(lLc[kk * KP + 16 * q + n], lLt[(16 * r + n) * LP + kk], tacc);
            }
          }
        }
        lds_f32* pt = lT + wave * 256;
#pragma unroll
        for (int i = 0; i < 4; ++i) pt[(4 * g + i) * 16 + n] = tacc[i];
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        f32x4 xacc = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int st = 0; st < 4; ++st) {
          const int kk = 4 * st + g;
          xacc = mfma4(lLt[(16 * q + kk) * LP + 16 * q + n], pt[kk * 16 + n], xacc);
        }
#pragma unroll
        for (int i = 0; i < 4; ++i) lLt[(16 * r + n) * LP + 16 * q + 4 * g + i] = -xacc[i];
      }
      __syncthreads();
    }
    }

    // ---- V = W (L^-1)^T on the MFMA: V[r][j] = sum_m W[r][m] (L^-1)^T[m][j],
    // k assigned as in C V, so one 16-byte read of W's row feeds four steps
    {
      const lds_f32* pa = lV + (16 * ti0 + n) * SP + 4 * g;  // W[16 ti + n][16 q + 4 g + r]
      const lds_f32* pb = lLt + 4 * g * LP + 16 * tj0 + n;   // (L^-1)^T[16 q + 4 g + r][16 tj + n]
      f32x4 acc[TPW], a[2][TPW];
      float bv[2][4];
#pragma unroll
      for (int t = 0; t < TPW; ++t) acc[t] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int t = 0; t < TPW; ++t) a[0][t] = *(const lds_f32x4*)&pa[16 * RS * t * SP];
#pragma unroll
      for (int r = 0; r < 4; ++r) bv[0][r] = pb[r * LP];
#pragma unroll
      for (int q = 0; q < KP / 16; ++q) {
        const int cur = q & 1, nxt = cur ^ 1;
        if (q + 1 < KP / 16) {
#pragma unroll
          for (int t = 0; t < TPW; ++t) a[nxt][t] = *(const lds_f32x4*)&pa[16 * RS * t * SP + 16 * (q + 1)];
#pragma unroll
          for (int r = 0; r < 4; ++r) bv[nxt][r] = pb[(16 * (q + 1) + r) * LP];
        }
#pragma unroll
        for (int r = 0; r < 4; ++r)
#pragma unroll
          for (int t = 0; t < TPW; ++t) acc[t] = mfma4(a[cur][t][r], bv[cur][r], acc[t]);
      }
      __syncthreads();
      lds_f32* pw = lV + (16 * ti0 + 4 * g) * SP + 16 * tj0 + n;
#pragma unroll
      for (int t = 0; t < TPW; ++t)
#pragma unroll
        for (int i = 0; i < 4; ++i) pw[(16 * RS * t + i) * SP] = acc[t][i];
    }
    __syncthreads();
  }

  if (info && tid == 0) info[bh] = bad ? 1 : 0;  // thread 0 is in wave 0, which ran the pivots
  float* O = out + b * o_sb + (int64_t)h * o_sh;
  for (int e = tid; e < D * k; e += kThreads) {
    const int r = e / k, c = e - (e / k) * k;
    O[r * o_sr + c * o_sc] = sV[r * SP + c];
  }
}

// ---- 64 < k <= 128.  C, V/W, G, L and L^-1 do not all fit in LDS at this
// width, so C is read from global memory (each matrix's 64 KB stays in its
// XCD's L2 across the iterations) and G, L and X = L^-1 share one array:
//   strict lower triangle  L (rows below the diagonal)
//   diagonal               r_j = 1 / L_jj (= X_jj)
//   strict upper triangle  X^T (X is lower triangular)
// The Cholesky is blocked by 16-column panels as at k = 64 (wave 0 factors
// a panel with two rows per lane; all waves apply the trailing update on
// the MFMA), X's off-diagonal blocks follow by block rows, and V = W X^T
// reads X^T from the upper triangle (masked to zero below it).
constexpr int kW = 128;       // padded basis width
constexpr int kWS = kW + 4;   // V / W row stride
constexpr int kWG = kW + 1;   // G row stride

// X^T[m][j] from the packed array (zero below the diagonal, where L lives)
__device__ __forceinline__ float xt_at(const lds_f32* P, int m, int j) {
  const float v = P[m * kWG + j];
  return m <= j ? v : 0.f;
}

__global__ void __launch_bounds__(kThreads) power_iter128_kernel(
    const float* cov, int64_t c_sb, int64_t c_sh, int64_t c_sr, int64_t c_sc, const float* v0, int64_t v_sb,
    int64_t v_sh, int64_t v_sr, int64_t v_sc, float* out, int64_t o_sb, int64_t o_sh, int64_t o_sr,
    int64_t o_sc, int H, int k, int iters, float eps, int32_t* info, int cvec, int D) {
  __shared__ __align__(16) float sV[kD * kWS];
  __shared__ __align__(16) float sP[kW * kWG];
  __shared__ float sT[4 * 256];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, g = lane >> 4, n = lane & 15;
  const int bh = blockIdx.x, b = bh / H, h = bh - b * H;
  const float* C = cov + b * c_sb + (int64_t)h * c_sh;
  const float* V0 = v0 + b * v_sb + (int64_t)h * v_sh;
  constexpr int kB = 16;
  for (int e0 = 0; e0 < kD * kW; e0 += kThreads * kB) {
    float v[kB];
#pragma unroll
    for (int i = 0; i < kB; ++i) {
      const int e = e0 + i * kThreads + tid, r = e >> 7, c = e & 127;
      v[i] = c < k && r < D ? V0[r * v_sr + c * v_sc] : 0.f;
    }
#pragma unroll
    for (int i = 0; i < kB; ++i) {
      const int e = e0 + i * kThreads + tid;
      sV[(e >> 7) * kWS + (e & 127)] = v[i];
    }
  }
  __syncthreads();
  bool bad = false;
  lds_f32* const lV = (lds_f32*)sV;
  lds_f32* const lP = (lds_f32*)sP;
  lds_f32* const lT = (lds_f32*)sT + wave * 256;
  const int tjw = 2 * wave;  // this wave's output column tiles in C V and W X^T: tjw, tjw + 1

  for (int it = 0; it < iters; ++it) {
    // ---- W = C V: tiles (ti, tjw + t2), ti = 0..7; in k-group q lane (g, n)
    // supplies k = 16 q + 4 g + r (one 16-byte read of C's row feeds four steps)
    {
      f32x4 acc[8][2];
#pragma unroll
      for (int ti = 0; ti < 8; ++ti) acc[ti][0] = acc[ti][1] = f32x4{0.f, 0.f, 0.f, 0.f};
      for (int q = 0; q < kD / 16; ++q) {
        float a[8][4];
#pragma unroll
        for (int ti = 0; ti < 8; ++ti) {
          if (cvec) {  // (D == 128)
            const float* cr = C + (int64_t)(16 * ti + n) * c_sr;
            const float4 v = *(const float4*)(cr + 16 * q + 4 * g);
            a[ti][0] = v.x, a[ti][1] = v.y, a[ti][2] = v.z, a[ti][3] = v.w;
          } else {  // rows and columns of C past D are zeros
            const int row = 16 * ti + n;
            const float* cr = C + (int64_t)min(row, D - 1) * c_sr;
#pragma unroll
            for (int r = 0; r < 4; ++r) {
              const int col = 16 * q + 4 * g + r;
              const float x = cr[(int64_t)min(col, D - 1) * c_sc];
              a[ti][r] = row < D && col < D ? x : 0.f;
            }
          }
        }
        float bv[2][4];
#pragma unroll
        for (int t2 = 0; t2 < 2; ++t2)
#pragma unroll
          for (int r = 0; r < 4; ++r) bv[t2][r] = lV[(16 * q + 4 * g + r) * kWS + 16 * (tjw + t2) + n];
#pragma unroll
        for (int r = 0; r < 4; ++r)
#pragma unroll
          for (int ti = 0; ti < 8; ++ti)
#pragma unroll
            for (int t2 = 0; t2 < 2; ++t2) acc[ti][t2] = mfma4(a[ti][r], bv[t2][r], acc[ti][t2]);
      }
      __syncthreads();
#pragma unroll
      for (int ti = 0; ti < 8; ++ti)
#pragma unroll
        for (int t2 = 0; t2 < 2; ++t2)
#pragma unroll
          for (int i = 0; i < 4; ++i) lV[(16 * ti + 4 * g + i) * kWS + 16 * (tjw + t2) + n] = acc[ti][t2][i];
    }
    __syncthreads();

    // ---- G = W^T W, the 36 lower tiles (ti >= tj), tile t to wave t mod 4
    {
      int t = 0;
      for (int ti = 0; ti < 8; ++ti) {
        for (int tj = 0; tj <= ti; ++tj, ++t) {
          if (t % 4 != wave) continue;  // wave-uniform
          f32x4 acc = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll 8
          for (int q = 0; q < kD / 4; ++q)
            acc = mfma4(lV[(4 * q + g) * kWS + 16 * ti + n], lV[(4 * q + g) * kWS + 16 * tj + n], acc);
#pragma unroll
          for (int i = 0; i < 4; ++i) lP[(16 * ti + 4 * g + i) * kWG + 16 * tj + n] = acc[i];
        }
      }
    }
    __syncthreads();

    // ---- ridge: G += eps * mean(diag G) * I over the first k; padding
    // rows and columns are zero (V's padding columns are): unit diagonal
    if (wave == 0) {
      const float d0 = lP[lane * kWG + lane], d1 = lP[(lane + 64) * kWG + lane + 64];
      float dg = (lane < k ? d0 : 0.f) + (lane + 64 < k ? d1 : 0.f);
#pragma unroll
      for (int off = 32; off > 0; off >>= 1) dg += shfl_xor(dg, off);
      const float ridge = eps * (dg / (float)k);
      lP[lane * kWG + lane] = lane < k ? d0 + ridge : 1.f;
      lP[(lane + 64) * kWG + lane + 64] = lane + 64 < k ? d1 + ridge : 1.f;
    }
    __syncthreads();

    // ---- blocked Cholesky and the diagonal blocks of X
    for (int p = 0; p < kW / 16; ++p) {
      const int P0 = 16 * p;
      if (wave == 0) {
        // lane holds rows lane and lane + 64 (entries of panel columns P0..P0+15)
        float a0[16], a1[16], lc0[16], lc1[16], xv[16];
        const bool hi = P0 >= 64;  // the panel's rows sit in the second half
        const int prow = (hi ? lane + 64 : lane);  // the half whose lanes hold the panel rows
#pragma unroll
        for (int c = 0; c < 16; ++c) {
          a0[c] = lP[lane * kWG + P0 + c];
          a1[c] = lP[(lane + 64) * kWG + P0 + c];
          xv[c] = prow == P0 + c ? 1.f : 0.f;
        }
#pragma unroll
        for (int jj = 0; jj < 16; ++jj) {
          const int j = P0 + jj;
          const float pv = hi ? a1[jj] : a0[jj];
          const float piv = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, pv), j & 63));
          bad |= !(piv > 0.f && piv <= 3.402823466e38f);
          const float rj = __builtin_amdgcn_rsqf(piv);
          const float l0 = lane > j ? a0[jj] * rj : (lane == j ? rj : 0.f);
          const float l1 = lane + 64 > j ? a1[jj] * rj : (lane + 64 == j ? rj : 0.f);
          lc0[jj] = l0;
          lc1[jj] = l1;
          xv[jj] *= rj;
          const float lp = hi ? l1 : l0;  // column j of L in the panel rows' half
#pragma unroll
          for (int mm = jj + 1; mm < 16; ++mm) {
            const float c = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, lp), (P0 + mm) & 63));
            a0[mm] = fmaf(-l0, c, a0[mm]);
            a1[mm] = fmaf(-l1, c, a1[mm]);
            xv[mm] = fmaf(-c, xv[jj], xv[mm]);
          }
        }
        // L (lower triangle and diagonal) in place of G
#pragma unroll
        for (int jj = 0; jj < 16; ++jj) {
          if (lane >= P0 + jj) lP[lane * kWG + P0 + jj] = lc0[jj];
          if (lane + 64 >= P0 + jj) lP[(lane + 64) * kWG + P0 + jj] = lc1[jj];
        }
        // X's diagonal block, transposed into the upper triangle: row prow
        // of X^T holds column prow of X (lanes whose row is in the panel)
        if (prow >= P0 && prow < P0 + 16) {
#pragma unroll
          for (int mm = 0; mm < 16; ++mm)
            if (P0 + mm > prow) lP[prow * kWG + P0 + mm] = xv[mm];
        }
      }
      __syncthreads();
      if (p + 1 < kW / 16) {
        // G[16 ti + a][16 tj + b] -= sum_c L[16 ti + a][P0 + c] L[16 tj + b][P0 + c], p < tj <= ti
        int t = 0;
        for (int ti = p + 1; ti < kW / 16; ++ti) {
          for (int tj = p + 1; tj <= ti; ++tj, ++t) {
            if (t % 4 != wave) continue;  // wave-uniform
            f32x4 acc = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int st = 0; st < 4; ++st) {
              const int cc = P0 + 4 * st + g;
              acc = mfma4(lP[(16 * ti + n) * kWG + cc], lP[(16 * tj + n) * kWG + cc], acc);
            }
#pragma unroll
            for (int i = 0; i < 4; ++i) lP[(16 * ti + 4 * g + i) * kWG + 16 * tj + n] -= acc[i];
          }
        }
        __syncthreads();
      }
    }

    // ---- X's blocks below the diagonal by block rows q:
    // X_qr = -X_qq sum_{s=r}^{q-1} L_qs X_sr, stored transposed in the upper triangle
    for (int q = 1; q < kW / 16; ++q) {
      for (int r = wave; r < q; r += 4) {  // wave-uniform
        f32x4 tacc = f32x4{0.f, 0.f, 0.f, 0.f};
        for (int kk0 = 16 * r; kk0 < 16 * q; kk0 += 4) {
          const int kk = kk0 + g;
          tacc = mfma4(lP[(16 * q + n) * kWG + kk], xt_at(lP, 16 * r + n, kk), tacc);
        }
#pragma unroll
        for (int i = 0; i < 4; ++i) lT[(4 * g + i) * 16 + n] = tacc[i];
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        f32x4 xacc = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int st = 0; st < 4; ++st) {
          const int kk = 4 * st + g;
          xacc = mfma4(xt_at(lP, 16 * q + kk, 16 * q + n), lT[kk * 16 + n], xacc);
        }
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
#pragma unroll
        for (int i = 0; i < 4; ++i) lP[(16 * r + n) * kWG + 16 * q + 4 * g + i] = -xacc[i];
      }
      __syncthreads();
    }

    // ---- V = W X^T: V[r][j] = sum_{m <= j} W[r][m] X^T[m][j], tiles (ti, tjw + t2)
    {
      f32x4 acc[8][2];
#pragma unroll
      for (int ti = 0; ti < 8; ++ti) acc[ti][0] = acc[ti][1] = f32x4{0.f, 0.f, 0.f, 0.f};
      for (int q = 0; q <= tjw + 1; ++q) {  // k-blocks of 16 up to the wave's last column tile
#pragma unroll
        for (int st = 0; st < 4; ++st) {
          const int m = 16 * q + 4 * st + g;
          float bv[2];
#pragma unroll
          for (int t2 = 0; t2 < 2; ++t2) bv[t2] = xt_at(lP, m, 16 * (tjw + t2) + n);
#pragma unroll
          for (int ti = 0; ti < 8; ++ti) {
            const float av = lV[(16 * ti + n) * kWS + m];
#pragma unroll
            for (int t2 = 0; t2 < 2; ++t2) acc[ti][t2] = mfma4(av, bv[t2], acc[ti][t2]);
          }
        }
      }
      __syncthreads();
#pragma unroll
      for (int ti = 0; ti < 8; ++ti)
#pragma unroll
        for (int t2 = 0; t2 < 2; ++t2)
#pragma unroll
          for (int i = 0; i < 4; ++i) lV[(16 * ti + 4 * g + i) * kWS + 16 * (tjw + t2) + n] = acc[ti][t2][i];
    }
    __syncthreads();
  }

  if (info && tid == 0) info[bh] = bad ? 1 : 0;
  float* O = out + b * o_sb + (int64_t)h * o_sh;
  for (int e = tid; e < D * k; e += kThreads) {
    const int r = e / k, c = e - (e / k) * k;
    O[r * o_sr + c * o_sc] = sV[r * kWS + c];
  }
}

template <int KP>
hipError_t launch(const rk_tensor* cov, const rk_tensor* v0, const rk_tensor* out, int64_t BH, int H, int k,
                  int iters, float eps, int32_t* info, int D, hipStream_t s) {
  hipLaunchKernelGGL((power_iter_kernel<KP>), dim3((unsigned)BH), dim3(kThreads), 0, s, (const float*)cov->data,
                     cov->stride[0], cov->stride[1], cov->stride[2], cov->stride[3], (const float*)v0->data,
                     v0->stride[0], v0->stride[1], v0->stride[2], v0->stride[3], (float*)out->data, out->stride[0],
                     out->stride[1], out->stride[2], out->stride[3], H, k, iters, eps, info, D);
  return hipGetLastError();
}

}  // namespace rot
}  // namespace rk

extern "C" int rk_power_iteration(const rk_tensor* cov, const rk_tensor* v0, const rk_tensor* out,
                                  int32_t num_iters, float eps, int32_t* info, void* stream) {
  using namespace rk::rot;
  if (!cov || !v0 || !out) return RK_ERR_NULL;
  int st;
  if ((st = rk::check_desc(cov, 4)) || (st = rk::check_desc(v0, 4)) || (st = rk::check_desc(out, 4))) return st;
  if (cov->dtype != RK_F32 || v0->dtype != RK_F32 || out->dtype != RK_F32) return RK_ERR_DTYPE;
  // any head_dim D <= 128 (rotation.py:86-91 takes D = cov.shape[-1])
  const int64_t D = cov->shape[2];
  if (D < 1 || D > kD || cov->shape[3] != D) return RK_ERR_HEAD_DIM;
  const int64_t B = cov->shape[0], H = cov->shape[1], k = v0->shape[3];
  for (const rk_tensor* t : {v0, out})
    if (t->shape[0] != B || t->shape[1] != H || t->shape[2] != D || t->shape[3] != k) return RK_ERR_SHAPE;
  if (k < 1 || k > D) return RK_ERR_KEEP_DIM;
  if (num_iters < 0 || !(eps >= 0.f)) return RK_ERR_ARG;
  if (B * H == 0) return RK_OK;
  if (B * H > (INT64_C(1) << 31) || H > (INT64_C(1) << 30)) return RK_ERR_SHAPE;
  if (!cov->data || !v0->data || !out->data) return RK_ERR_NULL;
  hipStream_t s = (hipStream_t)stream;
  hipError_t e;
  if (k <= 16)
    e = launch<16>(cov, v0, out, B * H, (int)H, (int)k, num_iters, eps, info, (int)D, s);
  else if (k <= 32)
    e = launch<32>(cov, v0, out, B * H, (int)H, (int)k, num_iters, eps, info, (int)D, s);
  else if (k <= 64)
    e = launch<64>(cov, v0, out, B * H, (int)H, (int)k, num_iters, eps, info, (int)D, s);
  else {
    const int cvec = D == kD && cov->stride[3] == 1 && cov->stride[2] % 4 == 0 && cov->stride[1] % 4 == 0 &&
                     cov->stride[0] % 4 == 0 && (((uintptr_t)cov->data) & 15) == 0;
    hipLaunchKernelGGL(power_iter128_kernel, dim3((unsigned)(B * H)), dim3(kThreads), 0, s, (const float*)cov->data,
                       cov->stride[0], cov->stride[1], cov->stride[2], cov->stride[3], (const float*)v0->data,
                       v0->stride[0], v0->stride[1], v0->stride[2], v0->stride[3], (float*)out->data,
                       out->stride[0], out->stride[1], out->stride[2], out->stride[3], (int)H, (int)k, num_iters, eps,
                       info, cvec, (int)D);
    e = hipGetLastError();
  }
  return e == hipSuccess ? RK_OK : RK_ERR_HIP;
}
