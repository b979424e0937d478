// rk_prefill.hip -- RotateK prefill producer kernels for MI355X (gfx950).
//
// Per (batch, KV head) of the visual Keys K [S, D] (D <= 128, any strides;
// F16, BF16 or F32; channels past D are treated as absent):
//
//   covariance   (kv_pruning_utils.py:112-115)
//     mean_kernel   split-S fp32 partial sums of K               (pass 1)
//     cov_kernel    mu = sum / S (fp32), c = dtype(mu); Kc = dtype(K - c);
//                   split-S partial Kc^T Kc on v_mfma_f32_16x16x32 with
//                   fp32 accumulation, upper 36 of 64 16x16 tiles (pass 2)
//     covfin_kernel sum of partials -> dtype -> fp32 -> 0.5 (C + C^T)
//   rotate / score (kv_pruning_utils.py:152; BASELINE config 0 selection)
//     rot_kernel    C^T = R^T K^T on the MFMA, 64 tokens per step; STORE
//                   writes dtype(K R) (the truncated visual-Key write),
//                   SCORE accumulates |K R| per rotated channel
//     scorefin_kernel  fp64 sum of the per-workgroup partial sums / S
//   selection
//     topk_kernel   head-wise top-k by (score desc, index asc) -> ascending
//                   indices + keep mask (kv_pruning_utils.py:158-159)
//     gather_kernel R_partial = dtype(R_full[:, idx]),
//                   delta_mu = dtype(mu - (mu R_partial) R_partial^T)
//                   (kv_pruning_utils.py:150-156)
//
// Operand layout (see rk_common.h): for the covariance a lane (g, n) loads
// rows 8g..8g+7 (tokens) x channels 8n..8n+7 of a 32-token block and
// transposes them in registers; slot i of that transpose is the MFMA
// operand for the channel set {8m + i : m = 0..15}, so tile (i, j) of the
// accumulator holds C[8m + i][8m' + j].  fp32 Keys keep that layout on
// v_mfma_f32_16x16x4_f32, one token row of the lane per MFMA step.
//
// head_dim D < 128: with 16-byte rows (D a multiple of 8) a lane whose
// channel slot lies past D re-reads the row's last slot (in bounds) and its
// values are masked to zero before they meet a valid operand; element-wise
// loads read only channels < D.  Outputs hold D channels.
#include <math.h>
#include <string.h>

#include <type_traits>

#include "rk_common.h"
#include "rk_host.h"
#include "rotatek_hip.h"

namespace rk {
namespace prefill {

constexpr int kThreads = 256;
constexpr int kWaves = 4;

struct KeyView {
  const uint16_t* data;  // element pointer (fp32 Keys: reinterpreted)
  int64_t sb, sh;      // batch / head strides (elements)
  uint32_t ss, sd;     // token / channel strides; a head spans < 2^31 elements
  int64_t S;           // tokens
  int32_t H;
  int32_t D;           // head_dim, 1..128
};

__device__ __forceinline__ const uint16_t* head_base(const KeyView& k, int bh) {
  const int b = bh / k.H, h = bh - b * k.H;
  return k.data + b * k.sb + (int64_t)h * k.sh;
}
template <class TT>
__device__ __forceinline__ const void* head_base_t(const KeyView& k, int bh) {
  const int b = bh / k.H, h = bh - b * k.H;
  return (const char*)k.data + (b * k.sb + (int64_t)h * k.sh) * TT::kBytes;
}

// The channel slot [c0, c0 + 8) a lane loads: with 16-byte rows a slot past
// D re-reads the last one (D is then a multiple of 8); element-wise loads
// take c0 as is and read nv = clamp(D - c0, 0, 8) channels.
template <bool VEC>
__device__ __forceinline__ uint32_t slot_c0(int c0, int D) {
  return VEC ? (uint32_t)min(c0, D - 8) : (uint32_t)c0;
}
__device__ __forceinline__ int slot_nv(int c0, int D) { return max(min(D - c0, 8), 0); }

// Eight 16-bit channels c0..c0+7 of row `t` (clamped by the caller); the
// element-wise form reads the first nv and zeroes the rest.
template <bool VEC>
__device__ __forceinline__ uint4 ldrow(const uint16_t* base, const KeyView& k, uint32_t t, uint32_t c0, int nv = 8) {
  if constexpr (VEC) {
    return *(const uint4*)((const char*)base + (t * k.ss + c0) * 2u);
  } else {
    uint32_t w[4] = {0, 0, 0, 0};
#pragma unroll
    for (int e = 0; e < 8; ++e)
      if (e < nv) w[e >> 1] |= (uint32_t)base[t * k.ss + (c0 + e) * k.sd] << ((e & 1) * 16);
    return make_uint4(w[0], w[1], w[2], w[3]);
  }
}

// Eight fp32 channels c0..c0+7 of row `t`, as ldrow (VEC: two 16-byte loads).
template <bool VEC>
__device__ __forceinline__ void ldrow32(const float* base, const KeyView& k, uint32_t t, uint32_t c0, int nv,
                                        float (&f)[8]) {
  if constexpr (VEC) {
    const float4 a = *(const float4*)((const char*)base + (t * k.ss + c0) * 4u);
    const float4 b = *(const float4*)((const char*)base + (t * k.ss + c0 + 4) * 4u);
    f[0] = a.x; f[1] = a.y; f[2] = a.z; f[3] = a.w;
    f[4] = b.x; f[5] = b.y; f[6] = b.z; f[7] = b.w;
  } else {
#pragma unroll
    for (int e = 0; e < 8; ++e) f[e] = e < nv ? base[t * k.ss + (c0 + e) * k.sd] : 0.f;
  }
}

template <class TT>
__device__ __forceinline__ void unpack8(const uint4& v, float (&f)[8]) {
#pragma unroll
  for (int e = 0; e < 8; ++e) f[e] = TT::to_f32((uint16_t)(word(v, e >> 1) >> ((e & 1) * 16)));
}

// ------------------------------------------------------------------ pass 1
// grid (splits, B*H): workgroup x sums tokens [x*chunk, (x+1)*chunk) of one
// head into part[bh][x][128] (fp32).  Thread (row group rg = t/16, channel
// chunk c8 = t%16) walks rows rg, rg+16, ... four at a time.
// Query-aware weighting inputs (kv_pruning_utils.py:116-140): the window
// query rows of each KV head's G query heads; qn receives the floored norms
// per head ([B*H][128] fp32, in the workspace).
struct QNormArgs {
  const uint16_t* q;  // element pointer (fp32 queries: reinterpreted)
  int64_t q_b, q_h, q_s, q_d, S;
  int W, G, D;
  float inv_g;
  float* qn;
};

template <class TT, bool QV>
__device__ void window_group_sums(const uint16_t* q, int64_t q_b, int64_t q_h, int64_t q_s, int64_t q_d,
                                  int64_t S, int W, int G, int D, int b, int kv, int tid, float (&acc)[2][8]);
template <class TT>
__device__ void floored_query_norms(const float (&acc)[2][8], int W, int D, float inv_g, int tid,
                                    float (*s_part)[128], float* s_qn, float* s_floor);

// The floored query norms of head bh into qa.qn[bh] (the mean launch's
// extra column; s_part: 16 x 128 floats of LDS).
template <class TT, bool QV>
__device__ __forceinline__ void head_query_norms(const KeyView& k, const QNormArgs& qa, int bh, int tid,
                                                 float (*s_part)[128]) {
  __shared__ __align__(16) float s_qn[128];
  __shared__ float s_floor;
  const int b = bh / k.H, kv = bh - b * k.H;
  float acc[2][8];
  window_group_sums<TT, QV>(qa.q, qa.q_b, qa.q_h, qa.q_s, qa.q_d, qa.S, qa.W, qa.G, qa.D, b, kv, tid, acc);
  floored_query_norms<TT>(acc, qa.W, qa.D, qa.inv_g, tid, s_part, s_qn, &s_floor);
  if (tid < 128) qa.qn[(int64_t)bh * 128 + tid] = s_qn[tid];
}

// QN (weighted covariance only): the grid has one more column per head
// (x == splits) that forms the head's floored query norms.  Only these
// instantiations carry that code: its registers would otherwise set the
// occupancy of the summing loop.
template <class TT, bool VEC, bool QN, bool QV>
__global__ void __launch_bounds__(kThreads) mean_kernel(KeyView k, int64_t chunk, int splits, float* part,
                                                        QNormArgs qa) {
  __shared__ float s_sum[16][128];
  const int tid = threadIdx.x, rg = tid >> 4, c8 = tid & 15;
  const int x = blockIdx.x, bh = blockIdx.y;
  if constexpr (QN) {
    if (x == splits) {
      head_query_norms<TT, QV>(k, qa, bh, tid, s_sum);
      return;
    }
  }
  const int64_t t0 = (int64_t)x * chunk, t1 = min(k.S, t0 + chunk);
  float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
  const uint32_t last = (uint32_t)max(t1 - 1, (int64_t)0);
  const uint32_t cl = slot_c0<VEC>(8 * c8, k.D);
  const int nv = slot_nv(8 * c8, k.D);
  if constexpr (TT::kBytes == 2) {
    const uint16_t* base = head_base(k, bh);
    for (int64_t t = t0 + rg; t < t1; t += 64) {
      uint4 v[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) v[i] = ldrow<VEC>(base, k, min((uint32_t)(t + 16 * i), last), cl, nv);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        if (t + 16 * i < t1) {
          float f[8];
          unpack8<TT>(v[i], f);
#pragma unroll
          for (int e = 0; e < 8; ++e) acc[e] += f[e];
        }
      }
    }
  } else {
    const float* base = (const float*)head_base_t<TT>(k, bh);
    for (int64_t t = t0 + rg; t < t1; t += 64) {
      float f[4][8];
#pragma unroll
      for (int i = 0; i < 4; ++i) ldrow32<VEC>(base, k, min((uint32_t)(t + 16 * i), last), cl, nv, f[i]);
#pragma unroll
      for (int i = 0; i < 4; ++i)
        if (t + 16 * i < t1)
#pragma unroll
          for (int e = 0; e < 8; ++e) acc[e] += f[i][e];
    }
  }
  // a slot past D (16-byte rows) summed a duplicate: those channels are zero
#pragma unroll
  for (int e = 0; e < 8; ++e) s_sum[rg][8 * c8 + e] = 8 * c8 < k.D ? acc[e] : 0.f;
  __syncthreads();
  if (tid < 128) {
    float s = 0.f;
#pragma unroll
    for (int r = 0; r < 16; ++r) s += s_sum[r][tid];
    part[((int64_t)bh * splits + x) * 128 + tid] = s;
  }
}

// mean of one head from the pass-1 partials (fixed summation order, so every
// kernel that needs mu gets the same bits).
// Sum of n strided fp32 values, kSumBatch loads issued before any is
// added (the adds keep their index order).
constexpr int kSumBatch = 16;
__device__ __forceinline__ float strided_sum(const float* p, int n, int64_t stride) {
  float s = 0.f;
  for (int x0 = 0; x0 < n; x0 += kSumBatch) {
    float v[kSumBatch];
#pragma unroll
    for (int u = 0; u < kSumBatch; ++u) v[u] = x0 + u < n ? p[(int64_t)(x0 + u) * stride] : 0.f;
#pragma unroll
    for (int u = 0; u < kSumBatch; ++u) s += v[u];
  }
  return s;
}

// fp32 mean of channel c of head bh: the fp32 sum of the split partials
// times torch's mean factor (fp32 1/S), as torch's fp32 mean forms it.  The
// empty asm keeps the product an fp32 value: a caller that converts it to
// the key dtype would otherwise get one v_fma_mix, a single rounding of the
// exact product, where torch rounds to fp32 first (the two differ when the
// fp32 mean lands on a 16-bit midpoint).
__device__ __forceinline__ float head_mean(const float* part, int bh, int splits, int c, float mfac) {
  float m = strided_sum(part + (int64_t)bh * splits * 128 + c, splits, 128) * mfac;
  asm volatile("" : "+v"(m));
  return m;
}

// ------------------------------------------------------------------ pass 2
constexpr int kTiles = 36;  // upper-triangle 16x16 tiles (i <= j) of the 8x8 grid

// Tiles (i, j), i <= j, enumerated row-major: t = 8i - i(i-1)/2 + (j - i).
__host__ __device__ constexpr int tile_index(int i, int j) { return 8 * i - i * (i - 1) / 2 + (j - i); }
__host__ __device__ constexpr int tile_row(int t) {
  return t < 8 ? 0 : t < 15 ? 1 : t < 21 ? 2 : t < 26 ? 3 : t < 30 ? 4 : t < 33 ? 5 : t < 35 ? 6 : 7;
}
__host__ __device__ constexpr int tile_col(int t) { return tile_row(t) + t - tile_index(tile_row(t), tile_row(t)); }

// grid (splits, B*H): each wave accumulates Kc^T Kc over its interleaved
// 32-token blocks for all 36 upper tiles; the four waves are summed in LDS
// and the workgroup writes one [36][256] partial, and, with dpart, its 128
// diagonal entries once more as one contiguous row dpart[bh][x][128] (what
// the weighted finalisation sums for the ridge).
template <class TT, bool VEC>
__global__ void __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(2)))
cov_kernel(KeyView k, int64_t chunk, int splits, const float* mean_part, int mean_splits, float mfac,
           float* part, float* dpart) {
  __shared__ float s_c[128];
  __shared__ float s_red[kTiles * 256];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, g = lane >> 4, n = lane & 15;
  const int x = blockIdx.x, bh = blockIdx.y;
  if (tid < 128) {
    // centre = mean rounded to the key dtype (kv_pruning_utils.py:113);
    // channels past D have none
    s_c[tid] = tid < k.D ? TT::to_f32(TT::from_f32(head_mean(mean_part, bh, mean_splits, tid, mfac))) : 0.f;
  }
  __syncthreads();
  float cen[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) cen[e] = s_c[8 * n + e];
  // channel slot 8n..8n+7 of this lane: past D its (duplicate) values are
  // masked to zero together with the rows past the chunk
  const uint32_t cl = slot_c0<VEC>(8 * n, k.D);
  const int nv = slot_nv(8 * n, k.D);
  const bool ch_ok = 8 * n < k.D;

  f32x4 acc[kTiles];
#pragma unroll
  for (int t = 0; t < kTiles; ++t) acc[t] = f32x4{0.f, 0.f, 0.f, 0.f};
  const int64_t t0 = (int64_t)x * chunk, t1 = min(k.S, t0 + chunk);
  const int64_t nblk = (t1 - t0 + 31) / 32;
  const uint32_t last = (uint32_t)max(t1 - 1, (int64_t)0);
  if constexpr (TT::kBytes == 2) {
    const uint16_t* base = head_base(k, bh);
    // Centre in fp32 and round to the key dtype, two tokens of one channel
    // per conversion, which is already the transposed operand word:
    // op[i] element r = Kc[token 8g + r][channel 8n + i].  MASK: rows past
    // the end (clamped loads) and channel slots past D are masked to zero
    // after the conversion (a select around the conversion itself compiled
    // to one branch per element); whole blocks at head_dim 128 need neither
    // the mask nor the row clamps.
    auto block = [&](int64_t blk, auto mask) {
      constexpr bool MASK = decltype(mask)::value;
      const int64_t tb = t0 + blk * 32 + 8 * g;
      uint4 rows[8];
#pragma unroll
      for (int r = 0; r < 8; ++r)
        rows[r] = ldrow<VEC>(base, k, MASK ? min((uint32_t)(tb + r), last) : (uint32_t)(tb + r), cl, nv);
      const int64_t left = t1 - tb;
      const int nvalid = !ch_ok ? 0 : left >= 8 ? 8 : (left > 0 ? (int)left : 0);
      uint32_t w[8][4];
#pragma unroll
      for (int rp = 0; rp < 4; ++rp) {
        float f0[8], f1[8];
        unpack8<TT>(rows[2 * rp], f0);
        unpack8<TT>(rows[2 * rp + 1], f1);
        const uint32_t keep = (2 * rp < nvalid ? 0xffffu : 0u) | (2 * rp + 1 < nvalid ? 0xffff0000u : 0u);
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          w[i][rp] = TT::pack2(f0[i] - cen[i], f1[i] - cen[i]);
          if constexpr (MASK) w[i][rp] &= keep;
        }
      }
      uint4 op[8];
#pragma unroll
      for (int i = 0; i < 8; ++i) op[i] = make_uint4(w[i][0], w[i][1], w[i][2], w[i][3]);
#pragma unroll
      for (int t = 0; t < kTiles; ++t) acc[t] = TT::mfma(op[tile_row(t)], op[tile_col(t)], acc[t]);
    };
    // whole 32-token blocks of a head_dim-128 head first, then the rest
    const int64_t nfull = VEC && k.D == 128 ? (t1 - t0) / 32 : 0;
    int64_t blk = wave;
    for (; blk < nfull; blk += kWaves) block(blk, std::false_type{});
    for (; blk < nblk; blk += kWaves) block(blk, std::true_type{});
  } else {
    // fp32: Kc = K - mean in fp32 (the reference's fp32 subtraction), one
    // token row per v_mfma_f32_16x16x4_f32 step: at step r lane (g, n)
    // supplies Kc[token 8g + r][8n + i] as the k = g entry of operand i, so
    // tile (i, j) accumulates the same C[8m + i][8m' + j] as above
    const float* base = (const float*)head_base_t<TT>(k, bh);
    for (int64_t blk = wave; blk < nblk; blk += kWaves) {
      const int64_t tb = t0 + blk * 32 + 8 * g;
      float rows[8][8];
#pragma unroll
      for (int r = 0; r < 8; ++r) ldrow32<VEC>(base, k, min((uint32_t)(tb + r), last), cl, nv, rows[r]);
      const int64_t left = t1 - tb;
      const int nvalid = !ch_ok ? 0 : left >= 8 ? 8 : (left > 0 ? (int)left : 0);
#pragma unroll
      for (int r = 0; r < 8; ++r) {
        float op[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          const uint32_t bits = __builtin_bit_cast(uint32_t, rows[r][i] - cen[i]);
          op[i] = __builtin_bit_cast(float, r < nvalid ? bits : 0u);
        }
#pragma unroll
        for (int t = 0; t < kTiles; ++t) acc[t] = F32::mfma(op[tile_row(t)], op[tile_col(t)], acc[t]);
      }
    }
  }
  // reduce the four waves: lane (g, n) of tile t holds C[8(4g+r)+i][8n+j]
  for (int w = 0; w < kWaves; ++w) {
    if (wave == w) {
#pragma unroll
      for (int t = 0; t < kTiles; ++t)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          float& dst = s_red[t * 256 + (4 * g + r) * 16 + n];
          dst = (w == 0) ? acc[t][r] : dst + acc[t][r];
        }
    }
    __syncthreads();
  }
  float* out = part + ((int64_t)bh * splits + x) * (kTiles * 256);
  for (int i = tid; i < kTiles * 256; i += kThreads) out[i] = s_red[i];
  // C[c][c], c = 8 m + i: tile (i, i), entry (m, m)
  if (dpart && tid < 128)
    dpart[((int64_t)bh * splits + x) * 128 + tid] = s_red[tile_index(tid & 7, tid & 7) * 256 + 17 * (tid >> 3)];
}

// grid (kTiles, B*H): one workgroup per upper tile (i, j) of one head.
// Thread (m, n) sums entry (m, n) of the tile over the pass-2 partials
// (consecutive threads read consecutive floats), rounds the sum to the key
// dtype (the einsum output dtype, kv_pruning_utils.py:114) and back to fp32,
// and the tile writes cov[r][c] = 0.5 (C[r][c] + C[c][r])
// (kv_pruning_utils.py:115) for r = 8m + i, c = 8n + j and the mirrored
// entry, both < D.  C[c][r] of an off-diagonal tile is the same stored sum
// (the accumulator holds the upper tiles only); a diagonal tile pairs
// (m, n) with (n, m).  Tile 0 also writes mu [D].
template <class TT>
__global__ void __launch_bounds__(kThreads) covfin_kernel(const float* part, int splits,
                                                          const float* mean_part, int mean_splits,
                                                          float mfac, float* cov, int64_t cs_b, int64_t cs_h,
                                                          int64_t cs_r, int64_t cs_c, float* mu, int64_t ms_b,
                                                          int64_t ms_h, int64_t ms_c, int H, int D) {
  __shared__ float s_t[256];
  const int tid = threadIdx.x, t = blockIdx.x, bh = blockIdx.y;
  const int b = bh / H, h = bh - b * H;
  const float* src = part + (int64_t)bh * splits * (kTiles * 256) + t * 256 + tid;
  float sum = strided_sum(src, splits, kTiles * 256);  // fp32, then the key dtype (two roundings)
  asm volatile("" : "+v"(sum));
  s_t[tid] = TT::to_f32(TT::from_f32(sum));
  __syncthreads();
  const int i = tile_row(t), j = tile_col(t), m = tid >> 4, n = tid & 15;
  float* cb = cov + b * cs_b + (int64_t)h * cs_h;
  const int r = 8 * m + i, c = 8 * n + j;
  const float rc = s_t[tid];
  const float cr = i == j ? s_t[n * 16 + m] : rc;
  if (r < D && c < D) {
    cb[r * cs_r + c * cs_c] = 0.5f * (rc + cr);
    if (i != j) cb[c * cs_r + r * cs_c] = 0.5f * (cr + rc);
  }
  if (t == 0 && tid < D && mu)
    mu[b * ms_b + (int64_t)h * ms_h + tid * ms_c] = head_mean(mean_part, bh, mean_splits, tid, mfac);
}

// ------------------------------------------------------------------ rotate / score
// grid (splits, B*H).  C^T[kept][token] = sum_c R[c][kept] K[token][c]:
// A = R^T tile (from LDS, transposed once per workgroup), B = K^T (lane
// (g, n) loads 16 bytes of token row n at channel 32 ks + 8 g).  A wave
// takes 64 tokens (four 16-token column blocks) per step and reuses each A
// fragment across them.
//   STORE: out[token][16 t + 4 g + r] = dtype(C^T), the truncated write.
//   SCORE: per-lane sums of |C^T| per rotated channel, reduced over the
//          workgroup into spart[bh][x][kept] (fp32).
struct RotArgs {
  KeyView k;
  const void* R;
  int32_t r_dtype;
  int64_t R_sb, R_sh, R_sd, R_sk;
  int32_t Dk;
  uint16_t* out;
  int64_t o_sb, o_sh, o_ss, o_sd;
  float* spart;
  int64_t chunk;
  int32_t splits;
};

template <class TT, int NT, bool VEC, bool SCORE>
__global__ void __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(2)))
rot_kernel(const RotArgs a) {
  __shared__ __attribute__((aligned(16))) uint16_t s_rt[NT * 16][128 + 8];  // R^T, padded rows
  __shared__ float s_sc[kWaves][NT * 16];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, g = lane >> 4, n = lane & 15;
  const int x = blockIdx.x, bh = blockIdx.y;
  const int b = bh / a.k.H, h = bh - b * a.k.H;
  const uint16_t* base = head_base(a.k, bh);
  // stage R^T (kept rows >= Dk are zero) in the key dtype.  Element e of
  // this thread's batch is (c, kk) = (e % 128, e / 128): consecutive threads
  // take consecutive c; all loads are issued before any is converted.
  const int64_t rb = b * a.R_sb + (int64_t)h * a.R_sh;
  const int D = a.k.D;
  constexpr int kPer = NT * 16 * 128 / kThreads;
  uint32_t raw[kPer];
#pragma unroll
  for (int i = 0; i < kPer; ++i) {
    const int e = tid + i * kThreads, kk = e >> 7, c = e & 127;
    raw[i] = load_raw(a.R, rb + min(c, D - 1) * a.R_sd + min(kk, a.Dk - 1) * a.R_sk, a.r_dtype);
  }
#pragma unroll
  for (int i = 0; i < kPer; ++i) {
    const int e = tid + i * kThreads, kk = e >> 7, c = e & 127;
    s_rt[kk][c] = TT::from_f32(kk < a.Dk && c < D ? raw_to_f32(raw[i], a.r_dtype) : 0.f);
  }
  __syncthreads();
  // channel slots 32 ks + 8 g of this lane (past D: see the file comment)
  uint32_t cl[4];
  int nv[4];
  bool cok[4];
#pragma unroll
  for (int ks = 0; ks < 4; ++ks) {
    cl[ks] = slot_c0<VEC>(32 * ks + 8 * g, D);
    nv[ks] = slot_nv(32 * ks + 8 * g, D);
    cok[ks] = 32 * ks + 8 * g < D;
  }
  const bool dpart = VEC && D < 128;  // launch-uniform

  float sc[NT][4];
#pragma unroll
  for (int t = 0; t < NT; ++t)
#pragma unroll
    for (int r = 0; r < 4; ++r) sc[t][r] = 0.f;
  const int64_t t0 = (int64_t)x * a.chunk, t1 = min(a.k.S, t0 + a.chunk);
  // steps of TB 16-token column blocks, double-buffered: the next step's
  // loads are in flight while this one is on the MFMA (steps past the end
  // reload the last token, in bounds, and are not computed).  The score
  // variant takes 64-token steps (each R^T fragment feeds four MFMAs); the
  // store variant 32-token steps, so its output path fits in registers.
  constexpr int TB = SCORE ? 4 : 2;
  constexpr int kStep = 16 * TB;
  const int64_t nstep = (t1 - t0 + kStep - 1) / kStep;
  const uint32_t last = (uint32_t)max(t1 - 1, (int64_t)0);
  auto load = [&](uint4 (&bk)[TB][4], int64_t st) {
    const int64_t ts = t0 + st * kStep;
#pragma unroll
    for (int tb = 0; tb < TB; ++tb) {
      const int64_t tok = ts + 16 * tb + n;
      const uint32_t tr = min((uint32_t)min(tok, (int64_t)last), last);
#pragma unroll
      for (int ks = 0; ks < 4; ++ks) bk[tb][ks] = ldrow<VEC>(base, a.k, tr, cl[ks], nv[ks]);
    }
  };
  auto compute = [&](uint4 (&bk)[TB][4], int64_t st) {
    const int64_t ts = t0 + st * kStep;
    if constexpr (SCORE) {
#pragma unroll
      for (int tb = 0; tb < TB; ++tb)
        if (ts + 16 * tb + n >= t1)
#pragma unroll
          for (int ks = 0; ks < 4; ++ks) bk[tb][ks] = make_uint4(0, 0, 0, 0);
    }
    if (dpart) {  // duplicated slots past D, which would meet R's zero rows
#pragma unroll
      for (int tb = 0; tb < TB; ++tb)
#pragma unroll
        for (int ks = 0; ks < 4; ++ks)
          if (!cok[ks]) bk[tb][ks] = make_uint4(0, 0, 0, 0);
    }
#pragma unroll(NT <= 2 ? NT : 1)
    for (int t = 0; t < NT; ++t) {
      f32x4 c[TB];
#pragma unroll
      for (int tb = 0; tb < TB; ++tb) c[tb] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int ks = 0; ks < 4; ++ks) {
        const uint4 av = *(const uint4*)&s_rt[16 * t + n][32 * ks + 8 * g];
#pragma unroll
        for (int tb = 0; tb < TB; ++tb) c[tb] = TT::mfma(av, bk[tb][ks], c[tb]);
      }
      if constexpr (SCORE) {
#pragma unroll
        for (int tb = 0; tb < TB; ++tb)
#pragma unroll
          for (int r = 0; r < 4; ++r) sc[t][r] += fabsf(c[tb][r]);
      } else {
#pragma unroll
        for (int tb = 0; tb < TB; ++tb) {
          const int64_t tok = ts + 16 * tb + n;
          if (tok < t1) {
            uint16_t* o = a.out + b * a.o_sb + (int64_t)h * a.o_sh + tok * a.o_ss;
            const int k0 = 16 * t + 4 * g;
            if (k0 + 3 < a.Dk && a.o_sd == 1 && (((uintptr_t)(o + k0)) & 7) == 0) {
              uint2 w;
              w.x = TT::from_f32(c[tb][0]) | ((uint32_t)TT::from_f32(c[tb][1]) << 16);
              w.y = TT::from_f32(c[tb][2]) | ((uint32_t)TT::from_f32(c[tb][3]) << 16);
              *(uint2*)(o + k0) = w;
            } else {
#pragma unroll
              for (int r = 0; r < 4; ++r)
                if (k0 + r < a.Dk) o[(k0 + r) * a.o_sd] = TT::from_f32(c[tb][r]);
            }
          }
        }
      }
    }
  };
  uint4 bA[TB][4], bB[TB][4];
  if (wave < nstep) load(bA, wave);
  for (int64_t st = wave; st < nstep; st += 2 * kWaves) {
    load(bB, st + kWaves);
    compute(bA, st);
    if (st + kWaves >= nstep) break;
    load(bA, st + 2 * kWaves);
    compute(bB, st + kWaves);
  }
  if constexpr (SCORE) {
    // lanes of one row (fixed g) hold different tokens of the same channels
#pragma unroll
    for (int t = 0; t < NT; ++t)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        float v = sc[t][r];
        v += shfl_xor(v, 1);
        v += shfl_xor(v, 2);
        v += shfl_xor(v, 4);
        v += shfl_xor(v, 8);
        if (n == 0) s_sc[wave][16 * t + 4 * g + r] = v;
      }
    __syncthreads();
    for (int kk = tid; kk < NT * 16; kk += kThreads) {
      float v = 0.f;
#pragma unroll
      for (int w = 0; w < kWaves; ++w) v += s_sc[w][kk];
      a.spart[((int64_t)bh * a.splits + x) * (NT * 16) + kk] = v;
    }
  }
}

// fp32 Keys (the reference's update_rotatek on fp32 Keys, and BASELINE
// config 0's selection at its precision): C^T = R^T K^T on
// v_mfma_f32_16x16x4_f32 (fp32 products and sums).  Lane (g, n) holds
// channels 32g .. 32g + 31 of token n of the wave's 16-token step and, in
// MFMA step ks, supplies channel 32g + ks as the k = g entry of both
// operands (A = R^T[16t + n][32g + ks] from LDS, B = K[token n][32g + ks]),
// so the 32 steps sum all 128 channel slots (zero past D on both sides).
// STORE writes C^T as fp32 (the Keys' dtype), SCORE sums |C^T| per lane.
// grid (splits, B*H).
template <int NT, bool VEC, bool SCORE>
__global__ void __launch_bounds__(kThreads) rot32_kernel(const RotArgs a) {
  __shared__ __attribute__((aligned(16))) float s_rt[NT * 16][128 + 4];  // R^T, padded rows
  __shared__ float s_sc[kWaves][NT * 16];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, g = lane >> 4, n = lane & 15;
  const int x = blockIdx.x, bh = blockIdx.y;
  const int b = bh / a.k.H, h = bh - b * a.k.H;
  const float* base = (const float*)head_base_t<F32>(a.k, bh);
  const int D = a.k.D;
  const int64_t rb = b * a.R_sb + (int64_t)h * a.R_sh;
  constexpr int kPer = NT * 16 * 128 / kThreads;
  uint32_t raw[kPer];
#pragma unroll
  for (int i = 0; i < kPer; ++i) {
    const int e = tid + i * kThreads, kk = e >> 7, c = e & 127;
    raw[i] = load_raw(a.R, rb + min(c, D - 1) * a.R_sd + min(kk, a.Dk - 1) * a.R_sk, a.r_dtype);
  }
#pragma unroll
  for (int i = 0; i < kPer; ++i) {
    const int e = tid + i * kThreads, kk = e >> 7, c = e & 127;
    s_rt[kk][c] = kk < a.Dk && c < D ? raw_to_f32(raw[i], a.r_dtype) : 0.f;
  }
  __syncthreads();

  float sc[NT][4];
#pragma unroll
  for (int t = 0; t < NT; ++t)
#pragma unroll
    for (int r = 0; r < 4; ++r) sc[t][r] = 0.f;
  const int64_t t0 = (int64_t)x * a.chunk, t1 = min(a.k.S, t0 + a.chunk);
  const int64_t nstep = (t1 - t0 + 15) / 16;
  const uint32_t last = (uint32_t)max(t1 - 1, (int64_t)0);
  // the lane's 32 channels of token n: VEC, eight 16-byte loads (a quad past
  // D re-reads the row's last quad, D a multiple of 8, and is zeroed);
  // otherwise element loads of the channels < D
  auto load = [&](float (&kr)[32], int64_t st) {
    const int64_t tok = t0 + st * 16 + n;
    const uint32_t tr = (uint32_t)min(tok, (int64_t)last);
    const float* row = base + (int64_t)tr * a.k.ss;
    if constexpr (VEC) {
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const float4 v = *(const float4*)(row + min(32 * g + 4 * j, D - 4));
        kr[4 * j] = v.x; kr[4 * j + 1] = v.y; kr[4 * j + 2] = v.z; kr[4 * j + 3] = v.w;
      }
    } else {
#pragma unroll
      for (int j = 0; j < 32; ++j) kr[j] = 32 * g + j < D ? row[(int64_t)(32 * g + j) * a.k.sd] : 0.f;
    }
  };
  auto compute = [&](float (&kr)[32], int64_t st) {
    const int64_t tok = t0 + st * 16 + n;
    const bool tok_ok = tok < t1;
#pragma unroll
    for (int j = 0; j < 32; ++j) kr[j] = tok_ok && 32 * g + j < D ? kr[j] : 0.f;
#pragma unroll(NT <= 2 ? NT : 1)
    for (int t = 0; t < NT; ++t) {
      f32x4 c = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int q4 = 0; q4 < 8; ++q4) {
        const float4 av = *(const float4*)&s_rt[16 * t + n][32 * g + 4 * q4];
        c = F32::mfma(av.x, kr[4 * q4], c);
        c = F32::mfma(av.y, kr[4 * q4 + 1], c);
        c = F32::mfma(av.z, kr[4 * q4 + 2], c);
        c = F32::mfma(av.w, kr[4 * q4 + 3], c);
      }
      if constexpr (SCORE) {
#pragma unroll
        for (int r = 0; r < 4; ++r) sc[t][r] += fabsf(c[r]);
      } else if (tok_ok) {
        float* o = (float*)a.out + b * a.o_sb + (int64_t)h * a.o_sh + tok * a.o_ss;
        const int k0 = 16 * t + 4 * g;
        if (k0 + 3 < a.Dk && a.o_sd == 1 && (((uintptr_t)(o + k0)) & 15) == 0) {
          *(float4*)(o + k0) = make_float4(c[0], c[1], c[2], c[3]);
        } else {
#pragma unroll
          for (int r = 0; r < 4; ++r)
            if (k0 + r < a.Dk) o[(k0 + r) * a.o_sd] = c[r];
        }
      }
    }
  };
  float kA[32], kB[32];
  if (wave < nstep) load(kA, wave);
  for (int64_t st = wave; st < nstep; st += 2 * kWaves) {
    if (st + kWaves < nstep) load(kB, st + kWaves);
    compute(kA, st);
    if (st + kWaves >= nstep) break;
    if (st + 2 * kWaves < nstep) load(kA, st + 2 * kWaves);
    compute(kB, st + kWaves);
  }
  if constexpr (SCORE) {
#pragma unroll
    for (int t = 0; t < NT; ++t)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        float v = sc[t][r];
        v += shfl_xor(v, 1);
        v += shfl_xor(v, 2);
        v += shfl_xor(v, 4);
        v += shfl_xor(v, 8);
        if (n == 0) s_sc[wave][16 * t + 4 * g + r] = v;
      }
    __syncthreads();
    for (int kk = tid; kk < NT * 16; kk += kThreads) {
      float v = 0.f;
#pragma unroll
      for (int w = 0; w < kWaves; ++w) v += s_sc[w][kk];
      a.spart[((int64_t)bh * a.splits + x) * (NT * 16) + kk] = v;
    }
  }
}

// grid (B*H): scores[c] = (sum of partials in fp64) / S for c < nk;
// partial rows are `pstride` floats apart.
__global__ void __launch_bounds__(128) scorefin_kernel(const float* spart, int splits, int pstride, int nk,
                                                       int64_t S, double* scores, int64_t s_b, int64_t s_h,
                                                       int64_t s_c, int H) {
  const int c = threadIdx.x, bh = blockIdx.x;
  if (c >= nk) return;
  const int b = bh / H, h = bh - b * H;
  double s = 0.0;
  for (int x = 0; x < splits; ++x) s += (double)spart[((int64_t)bh * splits + x) * pstride + c];
  scores[b * s_b + (int64_t)h * s_h + c * s_c] = S > 0 ? s / (double)S : 0.0;
}

// ------------------------------------------------------------------ selection
// grid (B*H), 128 threads: rank of channel c = #{j : s_j > s_c or
// (s_j == s_c and j < c)}; kept iff rank < k; the output indices are the
// kept channels in ascending order.
__global__ void __launch_bounds__(128) topk_kernel(const double* scores, int64_t s_b, int64_t s_h,
                                                   int64_t s_c, int D, int k, int H, int64_t* idx,
                                                   int64_t i_b, int64_t i_h, int64_t i_k, uint8_t* mask,
                                                   int64_t m_b, int64_t m_h, int64_t m_c) {
  __shared__ double s_v[128];
  __shared__ int s_keep[128];
  const int c = threadIdx.x, bh = blockIdx.x;
  const int b = bh / H, h = bh - b * H;
  if (c < D) s_v[c] = scores[b * s_b + (int64_t)h * s_h + c * s_c];
  __syncthreads();
  int keep = 0;
  if (c < D) {
    const double v = s_v[c];
    int rank = 0;
    for (int j = 0; j < D; ++j) {
      const double w = s_v[j];
      rank += (w > v) || (w == v && j < c);
    }
    keep = rank < k;
    if (mask) mask[b * m_b + (int64_t)h * m_h + c * m_c] = (uint8_t)keep;
  }
  s_keep[c] = keep;
  __syncthreads();
  if (c < D && keep) {
    int pos = 0;
    for (int j = 0; j < c; ++j) pos += s_keep[j];
    idx[b * i_b + (int64_t)h * i_h + pos * i_k] = c;
  }
}

// grid (B*H), 128 threads: R_partial[:, kk] = dtype(R_full[:, idx[kk]]);
// delta_mu = dtype(mu - (mu Rp) Rp^T) with Rp already in the key dtype
// (TT = F32: both stay fp32).  Rows d < D (head_dim).
template <class TT>
__global__ void __launch_bounds__(128) gather_kernel(const void* R, int r_dtype, int64_t R_sb, int64_t R_sh,
                                                     int64_t R_sd, int64_t R_sk, const int64_t* idx,
                                                     int64_t i_b, int64_t i_h, int64_t i_k, int k,
                                                     const float* mu, int64_t u_b, int64_t u_h, int64_t u_c,
                                                     void* Rp, int64_t p_b, int64_t p_h, int64_t p_d,
                                                     int64_t p_k, void* dm, int64_t d_b, int64_t d_h,
                                                     int64_t d_c, int H, int D) {
  __shared__ float s_mu[128];
  __shared__ float s_proj[128];
  __shared__ int64_t s_col[128];
  __shared__ float s_rp[128][129];  // R_partial (rounded to the key dtype), row d
  const int d = threadIdx.x, bh = blockIdx.x;
  const int b = bh / H, h = bh - b * H;
  const int dd = min(d, D - 1);
  s_mu[d] = d < D ? mu[b * u_b + (int64_t)h * u_h + dd * u_c] : 0.f;
  if (d < k) s_col[d] = idx[b * i_b + (int64_t)h * i_h + d * i_k];
  __syncthreads();
  // row d of R_partial, 32 columns per pass: all loads of a pass are issued
  // before any store (the stores could alias them otherwise)
  const int64_t rb = b * R_sb + (int64_t)h * R_sh + dd * R_sd;
  for (int k0 = 0; k0 < k; k0 += 32) {
    uint32_t raw[32];
    if (r_dtype == 2) {
#pragma unroll
      for (int j = 0; j < 32; ++j) raw[j] = ((const uint32_t*)R)[rb + s_col[min(k0 + j, k - 1)] * R_sk];
    } else {
#pragma unroll
      for (int j = 0; j < 32; ++j) raw[j] = ((const uint16_t*)R)[rb + s_col[min(k0 + j, k - 1)] * R_sk];
    }
#pragma unroll
    for (int j = 0; j < 32; ++j) {
      if (k0 + j < k) {
        const auto v = TT::from_f32(raw_to_f32(raw[j], r_dtype));
        s_rp[d][k0 + j] = d < D ? TT::to_f32(v) : 0.f;
        if (d < D) {
          if constexpr (TT::kBytes == 4)
            ((uint32_t*)Rp)[b * p_b + (int64_t)h * p_h + d * p_d + (k0 + j) * p_k] = v;
          else
            ((uint16_t*)Rp)[b * p_b + (int64_t)h * p_h + d * p_d + (k0 + j) * p_k] = v;
        }
      }
    }
  }
  __syncthreads();
  if (d < k) {
    float s = 0.f;
    for (int e = 0; e < D; ++e) s += s_mu[e] * s_rp[e][d];
    s_proj[d] = s;
  }
  __syncthreads();
  if (d >= D) return;
  float p = 0.f;
  for (int kk = 0; kk < k; ++kk) p += s_proj[kk] * s_rp[d][kk];
  float dmu = s_mu[d] - p;           // fp32, then the key dtype (two roundings,
  asm volatile("" : "+v"(dmu));      // as the reference; see qweight_kernel)
  const auto o = TT::from_f32(dmu);
  if constexpr (TT::kBytes == 4)
    ((uint32_t*)dm)[b * d_b + (int64_t)h * d_h + d * d_c] = o;
  else
    ((uint16_t*)dm)[b * d_b + (int64_t)h * d_h + d * d_c] = o;
}

// grid (B*H_kv), 256 threads: query-aware weighting of one covariance
// (kv_pruning_utils.py:116-140).  q_norm[d] = || mean_g q[g, S-W+w, d] ||_2
// over the last W queries, the group mean (over the G query heads of the KV
// head) rounded to the query dtype as torch's bf16/fp16 mean is; floored at
// 1e-3 x the lower median of the 128 norms; then
//   out = 0.5 (C o (qn qn^T) + (C o (qn qn^T))^T) + 1e-4 max(mean|diag|, 1e-6) I
// (the clamp binds to the mean).  Every global load (the covariance and the
// G x W query rows) is issued before the first is used, so the kernel costs
// one memory latency plus its LDS work.  Thread (slot rs = t/16, chunk
// c8 = t%16) owns window rows rs and rs + 16 of channels 8 c8..8 c8+7 for all
// G heads.  The covariance goes through LDS (rows padded to 129), so the
// transposed read is conflict-free; out may alias cov.  CV / QV: 16-byte
// row loads of the covariance / the queries (unit inner stride, aligned).
constexpr int kQHeads = 8;  // query heads whose window rows are loaded together (G <= 8: one batch)

// Thread (rs = t/16, c8 = t%16) of 256: the fp32 sums over the G query
// heads of window rows rs and rs + 16 (of the last W rows), channels
// 8 c8..8 c8+7, G in order, the loads of kQHeads heads (16-byte rows) or
// two heads (element-wise) issued at a time.
template <class TT, bool QV>
__device__ void window_group_sums(const uint16_t* q, int64_t q_b, int64_t q_h, int64_t q_s, int64_t q_d,
                                  int64_t S, int W, int G, int D, int b, int kv, int tid, float (&acc)[2][8]) {
  const int rs = tid >> 4, c8 = tid & 15;
  const int w0 = rs, w1 = rs + 16;
  // channel slot 8 c8.. (past D: the last slot re-read, or no element loads;
  // zeroed in floored_query_norms)
  const int c0 = QV ? min(8 * c8, D - 8) : 8 * c8, nv = slot_nv(8 * c8, D);
  const int64_t off = b * q_b + (int64_t)(kv * G) * q_h + (S - W) * q_s + (int64_t)c0 * q_d;
#pragma unroll
  for (int j = 0; j < 2; ++j)
#pragma unroll
    for (int e = 0; e < 8; ++e) acc[j][e] = 0.f;
  // element-wise loads take 64-bit addresses each: two heads at a time
  // keep them in registers (the sums run in the same head order)
  constexpr int kQH = QV ? kQHeads : 2;
  for (int g0 = 0; g0 < G; g0 += kQH) {
    float f[kQH][2][8];
    if constexpr (TT::kBytes == 2) {
      const uint16_t* qb = q + off;
      uint4 v[kQH][2];
#pragma unroll
      for (int u = 0; u < kQH; ++u)
#pragma unroll
        for (int j = 0; j < 2; ++j) {
          const int w = j ? w1 : w0;
          v[u][j] = make_uint4(0u, 0u, 0u, 0u);
          if (g0 + u < G && w < W) {
            const uint16_t* p = qb + (int64_t)(g0 + u) * q_h + (int64_t)w * q_s;
            if constexpr (QV) {
              v[u][j] = *(const uint4*)p;
            } else {
              uint32_t wd[4] = {0, 0, 0, 0};
#pragma unroll
              for (int e = 0; e < 8; ++e)
                if (e < nv) wd[e >> 1] |= (uint32_t)p[e * q_d] << ((e & 1) * 16);
              v[u][j] = make_uint4(wd[0], wd[1], wd[2], wd[3]);
            }
          }
        }
#pragma unroll
      for (int u = 0; u < kQH; ++u)
#pragma unroll
        for (int j = 0; j < 2; ++j) unpack8<TT>(v[u][j], f[u][j]);
    } else {
      const float* qb = (const float*)q + off;
#pragma unroll
      for (int u = 0; u < kQH; ++u)
#pragma unroll
        for (int j = 0; j < 2; ++j) {
          const int w = j ? w1 : w0;
#pragma unroll
          for (int e = 0; e < 8; ++e) f[u][j][e] = 0.f;
          if (g0 + u < G && w < W) {
            const float* p = qb + (int64_t)(g0 + u) * q_h + (int64_t)w * q_s;
            if constexpr (QV) {
              const float4 a = *(const float4*)p, c = *(const float4*)(p + 4);
              f[u][j][0] = a.x; f[u][j][1] = a.y; f[u][j][2] = a.z; f[u][j][3] = a.w;
              f[u][j][4] = c.x; f[u][j][5] = c.y; f[u][j][6] = c.z; f[u][j][7] = c.w;
            } else {
#pragma unroll
              for (int e = 0; e < 8; ++e)
                if (e < nv) f[u][j][e] = p[e * q_d];
            }
          }
        }
    }
#pragma unroll
    for (int u = 0; u < kQH; ++u)
#pragma unroll
      for (int j = 0; j < 2; ++j)
        if (g0 + u < G)
#pragma unroll
          for (int e = 0; e < 8; ++e) acc[j][e] += f[u][j][e];
  }
}

// From the window group sums: the group mean in the query dtype (fp32 sum
// times torch's mean factor inv_g, formed on the host, rounded to fp32
// first and then to the dtype, as torch's MeanOps does; the empty asm keeps
// the product in an fp32 register, otherwise the multiply and the
// conversion fuse into one v_fma_mix, a single rounding), the per-channel
// L2 norms over the window, and the floor at 1e-3 x the lower median of the
// D norms (the norm of rank (D - 1) / 2, ties by index).  Leaves s_qn[c] =
// the floored norms (0 past D).
template <class TT>
__device__ void floored_query_norms(const float (&acc)[2][8], int W, int D, float inv_g, int tid,
                                    float (*s_part)[128], float* s_qn, float* s_floor) {
  const int rs = tid >> 4, c8 = tid & 15;
  float sq[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) sq[e] = 0.f;
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    if ((j ? rs + 16 : rs) < W) {
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        float prod = acc[j][e] * inv_g;
        asm volatile("" : "+v"(prod));
        const float m = TT::to_f32(TT::from_f32(prod));
        sq[e] = fmaf(m, m, sq[e]);
      }
    }
  }
#pragma unroll
  for (int e = 0; e < 8; ++e) s_part[rs][8 * c8 + e] = sq[e];
  __syncthreads();
  if (tid < 128) {
    float t = 0.f;
#pragma unroll
    for (int r = 0; r < 16; ++r) t += s_part[r][tid];
    // channels past D rank above every norm (they are not ranked themselves)
    s_qn[tid] = tid < D ? sqrtf(t) : INFINITY;
  }
  __syncthreads();
  float v = 0.f;
  if (tid < D) {
    v = s_qn[tid];
    int rank = 0;
#pragma unroll
    for (int j4 = 0; j4 < 32; ++j4) {
      const float4 u = *(const float4*)&s_qn[4 * j4];
      const float uu[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
      for (int e = 0; e < 4; ++e) rank += (uu[e] < v) || (uu[e] == v && 4 * j4 + e < tid);
    }
    if (rank == (D - 1) / 2) *s_floor = 1e-3f * v;  // exactly one thread when no norm is NaN
  }
  __syncthreads();
  // torch.median of a row holding a NaN is NaN, and so is the clamp against
  // it: every weight of the head becomes NaN (written after the ranks, which
  // a NaN leaves without a thread of the median's rank)
  if (tid < D && isnan(v)) *s_floor = __builtin_nanf("");
  __syncthreads();
  if (tid < 128) {
    const float fl = *s_floor;
    s_qn[tid] = tid >= D ? 0.f : isnan(fl) ? fl : fmaxf(v, fl);
  }
  __syncthreads();
}

// 1e-4 max(mean|diag(C o qn qn^T)|, 1e-6) from the diagonal dg_in[c] =
// C[c][c] (threads 0..D-1; the sum is a fixed xor tree in each of waves 0
// and 1, then the two halves, times torch's mean factor rfac = fp32(1/D)),
// as the weighted covariance's ridge.
__device__ __forceinline__ float weighted_ridge(float diag, const float* s_qn, int tid, int D, float rfac,
                                                float* s_wsum) {
  if (tid < 128) {
    const float qd = s_qn[tid];
    float dg = tid < D ? fabsf(diag * (qd * qd)) : 0.f;
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) dg += shfl_xor(dg, off);
    if ((tid & 63) == 0) s_wsum[tid >> 6] = dg;
  }
  __syncthreads();
  return 1e-4f * fmaxf((s_wsum[0] + s_wsum[1]) * rfac, 1e-6f);
}

// grid (B*H_kv), 256 threads: query-aware weighting of one covariance
// (kv_pruning_utils.py:116-140).  q_norm[d] = || mean_g q[g, S-W+w, d] ||_2
// over the last W queries, the group mean (over the G query heads of the KV
// head) rounded to the query dtype as torch's bf16/fp16 mean is; floored at
// 1e-3 x the lower median of the 128 norms; then
//   out = 0.5 (C o (qn qn^T) + (C o (qn qn^T))^T) + 1e-4 max(mean|diag|, 1e-6) I
// (the clamp binds to the mean).  Every global load (the covariance and the
// G x W query rows) is issued before the first is used, so the kernel costs
// one memory latency plus its LDS work.  The covariance goes through LDS
// (rows padded to 129), so the transposed read is conflict-free; out may
// alias cov.  CV / QV: 16-byte row loads of the covariance / the queries
// (unit inner stride, aligned).
template <class TT, bool CV, bool QV>
__global__ void __launch_bounds__(256) qweight_kernel(const float* cov, int64_t c_b, int64_t c_h, int64_t c_r,
                                                      int64_t c_c, const uint16_t* q, int64_t q_b, int64_t q_h,
                                                      int64_t q_s, int64_t q_d, int64_t S, int W, int G, int D,
                                                      float inv_g, float rfac, float* out, int64_t o_b,
                                                      int64_t o_h, int64_t o_r, int64_t o_c, int H) {
  constexpr int CP = 129;
  __shared__ float s_C[128 * CP];
  __shared__ float s_part[16][128];
  __shared__ __align__(16) float s_qn[128];
  __shared__ float s_wsum[2];
  __shared__ float s_floor;
  const int tid = threadIdx.x;
  const int bh = blockIdx.x, b = bh / H, kv = bh - b * H;
  const float* C = cov + b * c_b + (int64_t)kv * c_h;

  // ---- covariance loads (64 floats per thread; entries past D are zero,
  // their loads re-read an in-bounds entry)
  float cv[64];
  if constexpr (CV) {  // (D a multiple of 4)
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const int e4 = tid + 256 * i, r = e4 >> 5, c = (e4 & 31) * 4;
      const bool ok = r < D && c < D;
      const float4 v = *(const float4*)(C + min(r, D - 1) * c_r + min(c, D - 4));
      cv[4 * i] = ok ? v.x : 0.f, cv[4 * i + 1] = ok ? v.y : 0.f, cv[4 * i + 2] = ok ? v.z : 0.f,
      cv[4 * i + 3] = ok ? v.w : 0.f;
    }
  } else {
#pragma unroll
    for (int i = 0; i < 64; ++i) {
      const int e = tid + 256 * i, r = e >> 7, c = e & 127;
      const float v = C[min(r, D - 1) * c_r + min(c, D - 1) * c_c];
      cv[i] = r < D && c < D ? v : 0.f;
    }
  }
  float acc[2][8];
  window_group_sums<TT, QV>(q, q_b, q_h, q_s, q_d, S, W, G, D, b, kv, tid, acc);

  // ---- the covariance into LDS
  if constexpr (CV) {
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const int e4 = tid + 256 * i, r = e4 >> 5, c = (e4 & 31) * 4;
#pragma unroll
      for (int u = 0; u < 4; ++u) s_C[r * CP + c + u] = cv[4 * i + u];
    }
  } else {
#pragma unroll
    for (int i = 0; i < 64; ++i) {
      const int e = tid + 256 * i;
      s_C[(e >> 7) * CP + (e & 127)] = cv[i];
    }
  }
  floored_query_norms<TT>(acc, W, D, inv_g, tid, s_part, s_qn, &s_floor);
  const float ridge = weighted_ridge(tid < 128 ? s_C[tid * CP + tid] : 0.f, s_qn, tid, D, rfac, s_wsum);
  // ---- out[r][c] = 0.5 (C[r][c] w + C[c][r] w) + ridge [r == c], w = qn[r] qn[c]
  float* O = out + b * o_b + (int64_t)kv * o_h;
#pragma unroll 8
  for (int i = 0; i < 64; ++i) {
    const int e = tid + 256 * i, r = e >> 7, c = e & 127;
    const float w = s_qn[r] * s_qn[c];
    const float a = s_C[r * CP + c] * w, bt = s_C[c * CP + r] * w;
    if (r < D && c < D) O[r * o_r + c * o_c] = 0.5f * (a + bt) + (r == c ? ridge : 0.f);
  }
}

// grid (kTiles, B*H), 256 threads: covfin_kernel and the query-aware
// weighting in one launch, bit-identical to covfin_kernel followed by
// qweight_kernel.  The floored query norms come from the mean launch's
// extra column (qn [B*H][128]).  Each tile workgroup sums its tile's
// partials (as covfin) and the 128 diagonal entries' partials (for the
// ridge; the contiguous copies dpart[bh][x][128], the same values in the
// same order), loads in flight together, then writes its weighted tile and
// the mirror:  out[r][c] = 0.5 (a + a) + ridge [r == c],  a = sym[r][c] (qn[r] qn[c]),
// sym = 0.5 (C[r][c] + C[c][r]) the symmetrised covariance, which is what
// qweight_kernel reads back from covfin's output.
template <class TT>
__global__ void __launch_bounds__(kThreads) covfin_qw_kernel(const float* part, const float* dpart, int splits,
                                                             const float* mean_part, int mean_splits, float mfac,
                                                             const float* qn, float* cov, int64_t cs_b,
                                                             int64_t cs_h, int64_t cs_r, int64_t cs_c, float* mu,
                                                             int64_t ms_b, int64_t ms_h, int64_t ms_c, int H, int D,
                                                             float rfac) {
  __shared__ float s_t[256];
  __shared__ __align__(16) float s_qn[128];
  __shared__ float s_wsum[2];
  const int tid = threadIdx.x, t = blockIdx.x, bh = blockIdx.y;
  const int b = bh / H, h = bh - b * H;
  const float* pb = part + (int64_t)bh * splits * (kTiles * 256);
  // tile entry tid and (threads < 128) diagonal entry C[tid][tid]
  float sum = strided_sum(pb + t * 256 + tid, splits, kTiles * 256);
  float dsum = strided_sum(dpart + (int64_t)bh * splits * 128 + (tid & 127), splits, 128);
  const float qv = qn[(int64_t)bh * 128 + (tid & 127)];
  asm volatile("" : "+v"(sum));  // fp32, then the key dtype (two roundings)
  asm volatile("" : "+v"(dsum));
  s_t[tid] = TT::to_f32(TT::from_f32(sum));
  if (tid < 128) s_qn[tid] = qv;
  const float dx = TT::to_f32(TT::from_f32(dsum));
  const float diag = 0.5f * (dx + dx);  // the symmetrised diagonal, as covfin writes it
  __syncthreads();
  const float ridge = weighted_ridge(diag, s_qn, tid, D, rfac, s_wsum);
  const int i = tile_row(t), j = tile_col(t), m = tid >> 4, n = tid & 15;
  float* cb = cov + b * cs_b + (int64_t)h * cs_h;
  const int r = 8 * m + i, c = 8 * n + j;
  const float rc = s_t[tid];
  const float cr = i == j ? s_t[n * 16 + m] : rc;
  const float sym = 0.5f * (rc + cr), symt = 0.5f * (cr + rc);
  const float w = s_qn[r] * s_qn[c];
  const float a = sym * w, bt = symt * w;
  if (r < D && c < D) {
    cb[r * cs_r + c * cs_c] = 0.5f * (a + bt) + (r == c ? ridge : 0.f);
    if (i != j) cb[c * cs_r + r * cs_c] = 0.5f * (bt + a);
  }
  if (t == 0 && tid < D && mu)
    mu[b * ms_b + (int64_t)h * ms_h + tid * ms_c] = head_mean(mean_part, bh, mean_splits, tid, mfac);
}

}  // namespace prefill
}  // namespace rk

// =====================================================================
// host side
// =====================================================================
namespace {

using namespace rk::prefill;

int64_t cdiv(int64_t a, int64_t b) { return (a + b - 1) / b; }
size_t align256(size_t x) { return (x + 255) & ~size_t(255); }

// Row loads of 16 bytes along the last dim: unit channel stride, 16-byte
// aligned rows and base, whole 8-channel slots (D a multiple of 8).
bool rows_vec(const rk_tensor* t, int64_t D) {
  if (D % 8 != 0) return false;
  const int64_t per16 = 16 / rk::dtype_size(t->dtype);
  if (t->stride[t->ndim - 1] != 1 && t->shape[t->ndim - 1] > 1) return false;
  for (int i = 0; i < t->ndim - 1; ++i)
    if (t->shape[i] > 1 && (t->stride[i] % per16) != 0) return false;
  return (((uintptr_t)t->data) & 15) == 0;
}

// Keys descriptor [B, H, S, D] (F16, BF16 or F32; 1 <= D <= 128).  Sets the
// view and the fast-path flag.
int key_view(const rk_tensor* t, KeyView* k, bool* vec) {
  int st = rk::check_desc(t, 4);
  if (st) return st;
  if (!rk::is_float_param(t->dtype)) return RK_ERR_DTYPE;
  const int64_t D = t->shape[3];
  if (D < 1 || D > 128) return RK_ERR_HEAD_DIM;
  const int64_t span = (t->shape[2] > 0 ? (t->shape[2] - 1) * t->stride[2] : 0) + (D - 1) * t->stride[3] + 8;
  if (span >= (INT64_C(1) << 31) || t->stride[2] >= (INT64_C(1) << 31)) return RK_ERR_STRIDE;
  if (t->shape[0] * t->shape[1] > (INT64_C(1) << 30)) return RK_ERR_SHAPE;
  k->data = (const uint16_t*)t->data;
  k->sb = t->stride[0];
  k->sh = t->stride[1];
  k->ss = (uint32_t)t->stride[2];
  k->sd = (uint32_t)t->stride[3];
  k->S = t->shape[2];
  k->H = (int32_t)t->shape[1];
  k->D = (int32_t)D;
  *vec = rows_vec(t, D);
  return RK_OK;
}

// Token split of a per-head pass: about 2 workgroups per CU in total, at
// least 256 tokens per workgroup.
int splits_for(int64_t bh, int64_t S, int cus, int64_t min_tokens) {
  if (S <= 0 || bh <= 0) return 1;
  int64_t want = cdiv(2 * (int64_t)cus, bh);
  const int64_t cap = cdiv(S, min_tokens);
  if (want > cap) want = cap;
  if (want < 1) want = 1;
  if (want > 4096) want = 4096;
  return (int)want;
}

struct CovPlan {
  int mean_splits, cov_splits;
  int64_t mean_chunk, cov_chunk;
  size_t off_mean, off_cov, off_diag, off_qn, total;
};

CovPlan cov_plan(int64_t B, int64_t H, int64_t S, int cus) {
  CovPlan p;
  const int64_t bh = B * H;
  p.mean_splits = splits_for(bh, S, cus, 256);
  p.mean_chunk = cdiv(S > 0 ? S : 1, p.mean_splits);
  p.cov_splits = splits_for(bh, S, cus, 512);
  p.cov_chunk = cdiv(S > 0 ? S : 1, p.cov_splits);
  p.off_mean = 0;
  p.off_cov = align256((size_t)bh * p.mean_splits * 128 * sizeof(float));
  p.off_diag = p.off_cov + align256((size_t)bh * p.cov_splits * kTiles * 256 * sizeof(float));
  // the partials' diagonals and the floored query norms (weighted only)
  p.off_qn = p.off_diag + align256((size_t)bh * p.cov_splits * 128 * sizeof(float));
  p.total = p.off_qn + align256((size_t)bh * 128 * sizeof(float));
  return p;
}

int resolve_cus(int32_t num_cus, int* st) {
  *st = RK_OK;
  if (num_cus > 0) return num_cus;
  int dev = 0;
  const int cus = rk::current_device_cus(&dev);
  if (cus <= 0) *st = RK_ERR_NO_DEVICE;
  return cus;
}

int check_f32_out(const rk_tensor* t, int ndim, int64_t B, int64_t H, int64_t last, int dtype) {
  int st = rk::check_desc(t, ndim);
  if (st) return st;
  if (t->dtype != dtype) return RK_ERR_DTYPE;
  if (t->shape[0] != B || t->shape[1] != H || t->shape[ndim - 1] != last) return RK_ERR_SHAPE;
  if (ndim == 4 && t->shape[2] != last) return RK_ERR_SHAPE;
  return RK_OK;
}

// Query-aware weighting fused into the covariance's last launch.
struct QwArgs {
  const rk_tensor* q;
  int64_t G;
  int W;
  float inv_g;
  bool vec;
};

template <class TT>
hipError_t launch_cov(const KeyView& k, bool vec, const CovPlan& p, int64_t B, float* ws, float* cov,
                      const rk_tensor* cov_t, float* mu, const rk_tensor* mu_t, hipStream_t s,
                      const QwArgs* qw = nullptr) {
  const int64_t bh = B * k.H;
  float* mpart = (float*)((char*)ws + p.off_mean);
  float* cpart = (float*)((char*)ws + p.off_cov);
  const dim3 gm((unsigned)p.mean_splits, (unsigned)bh), gc((unsigned)p.cov_splits, (unsigned)bh);
  // mean over the token dim of [B, H, S, D] (kv_pruning_utils.py:112)
  const float mfac = rk::mean_factor(bh * k.D, bh * k.S * k.D);
  // the ridge's mean over the D diagonal entries of each [D, D] matrix
  const float rfac = rk::mean_factor(bh, bh * k.D);
  // with the weighting, the mean launch has one more column per head that
  // forms the head's floored query norms, and the covariance launch writes
  // its partials' diagonals once more, contiguously
  QNormArgs qa;
  memset(&qa, 0, sizeof(qa));
  float* qn = (float*)((char*)ws + p.off_qn);
  float* dpart = nullptr;
  dim3 gmq = gm;
  if (qw) {
    const rk_tensor* q = qw->q;
    qa = QNormArgs{(const uint16_t*)q->data, q->stride[0], q->stride[1], q->stride[2], q->stride[3], q->shape[2],
                   qw->W, (int)qw->G, k.D, qw->inv_g, qn};
    dpart = (float*)((char*)ws + p.off_diag);
    gmq.x += 1;
  }
  const int64_t mc = p.mean_chunk, cc = p.cov_chunk;
  const int ms = p.mean_splits, cs = p.cov_splits;
  if (vec) {
    if (!qw)
      hipLaunchKernelGGL((mean_kernel<TT, true, false, false>), gm, dim3(kThreads), 0, s, k, mc, ms, mpart, qa);
    else if (qw->vec)
      hipLaunchKernelGGL((mean_kernel<TT, true, true, true>), gmq, dim3(kThreads), 0, s, k, mc, ms, mpart, qa);
    else
      hipLaunchKernelGGL((mean_kernel<TT, true, true, false>), gmq, dim3(kThreads), 0, s, k, mc, ms, mpart, qa);
    hipLaunchKernelGGL((cov_kernel<TT, true>), gc, dim3(kThreads), 0, s, k, cc, cs, mpart, ms, mfac, cpart, dpart);
  } else {
    if (!qw)
      hipLaunchKernelGGL((mean_kernel<TT, false, false, false>), gm, dim3(kThreads), 0, s, k, mc, ms, mpart, qa);
    else if (qw->vec)
      hipLaunchKernelGGL((mean_kernel<TT, false, true, true>), gmq, dim3(kThreads), 0, s, k, mc, ms, mpart, qa);
    else
      hipLaunchKernelGGL((mean_kernel<TT, false, true, false>), gmq, dim3(kThreads), 0, s, k, mc, ms, mpart, qa);
    hipLaunchKernelGGL((cov_kernel<TT, false>), gc, dim3(kThreads), 0, s, k, cc, cs, mpart, ms, mfac, cpart, dpart);
  }
  if (qw) {
    hipLaunchKernelGGL((covfin_qw_kernel<TT>), dim3(kTiles, (unsigned)bh), dim3(kThreads), 0, s, cpart, dpart,
                       p.cov_splits, mpart, p.mean_splits, mfac, qn, cov, cov_t->stride[0], cov_t->stride[1],
                       cov_t->stride[2], cov_t->stride[3], mu, mu_t ? mu_t->stride[0] : 0,
                       mu_t ? mu_t->stride[1] : 0, mu_t ? mu_t->stride[2] : 0, k.H, k.D, rfac);
    return hipGetLastError();
  }
  hipLaunchKernelGGL((covfin_kernel<TT>), dim3(kTiles, (unsigned)bh), dim3(kThreads), 0, s, cpart, p.cov_splits,
                     mpart, p.mean_splits, mfac, cov, cov_t->stride[0], cov_t->stride[1], cov_t->stride[2],
                     cov_t->stride[3], mu, mu_t ? mu_t->stride[0] : 0, mu_t ? mu_t->stride[1] : 0,
                     mu_t ? mu_t->stride[2] : 0, k.H, k.D);
  return hipGetLastError();
}

hipError_t launch_cov_any(int dtype, const KeyView& k, bool vec, const CovPlan& p, int64_t B, float* ws,
                          float* cov, const rk_tensor* cov_t, float* mu, const rk_tensor* mu_t, hipStream_t s,
                          const QwArgs* qw = nullptr) {
  switch (dtype) {
    case RK_F16: return launch_cov<rk::F16>(k, vec, p, B, ws, cov, cov_t, mu, mu_t, s, qw);
    case RK_BF16: return launch_cov<rk::BF16>(k, vec, p, B, ws, cov, cov_t, mu, mu_t, s, qw);
    default: return launch_cov<rk::F32>(k, vec, p, B, ws, cov, cov_t, mu, mu_t, s, qw);
  }
}

}  // namespace

extern "C" int rk_key_covariance_check(const rk_tensor* keys, const rk_tensor* mean_out,
                                       const rk_tensor* cov_out, int32_t num_cus,
                                       size_t* workspace_bytes) {
  KeyView k;
  bool vec;
  int st = key_view(keys, &k, &vec);
  if (st) return st;
  const int64_t B = keys->shape[0], H = keys->shape[1];
  if (!cov_out) return RK_ERR_NULL;
  if ((st = check_f32_out(cov_out, 4, B, H, k.D, RK_F32))) return st;
  if (mean_out && (st = check_f32_out(mean_out, 3, B, H, k.D, RK_F32))) return st;
  const int cus = resolve_cus(num_cus, &st);
  if (st) return st;
  if (workspace_bytes) *workspace_bytes = cov_plan(B, H, k.S, cus).total;
  return RK_OK;
}

extern "C" int rk_key_covariance(const rk_tensor* keys, const rk_tensor* mean_out, const rk_tensor* cov_out,
                                 void* workspace, size_t workspace_bytes, void* stream) {
  KeyView k;
  bool vec;
  int st = key_view(keys, &k, &vec);
  if (st) return st;
  const int64_t B = keys->shape[0], H = keys->shape[1];
  if (!cov_out) return RK_ERR_NULL;
  if ((st = check_f32_out(cov_out, 4, B, H, k.D, RK_F32))) return st;
  if (mean_out && (st = check_f32_out(mean_out, 3, B, H, k.D, RK_F32))) return st;
  const int cus = resolve_cus(0, &st);
  if (st) return st;
  const CovPlan p = cov_plan(B, H, k.S, cus);
  if (!workspace || (((uintptr_t)workspace) & 255) || workspace_bytes < p.total) return RK_ERR_WORKSPACE;
  if (B * H == 0) return RK_OK;
  if ((k.S > 0 && !k.data) || !cov_out->data) return RK_ERR_NULL;
  const hipError_t e = launch_cov_any(keys->dtype, k, vec, p, B, (float*)workspace, (float*)cov_out->data, cov_out,
                                      mean_out ? (float*)mean_out->data : nullptr, mean_out, (hipStream_t)stream);
  return e == hipSuccess ? RK_OK : RK_ERR_HIP;
}

namespace {

// Queries of the fused weighting: [B, H_kv * G, S_q, D] in the key dtype,
// window = min(window, S_q) rows (window 1..32).
int check_queries(const rk_tensor* keys, const rk_tensor* q, int64_t G, int32_t window, QwArgs* qw) {
  if (!q) return RK_ERR_NULL;
  int st = rk::check_desc(q, 4);
  if (st) return st;
  if (q->dtype != keys->dtype) return RK_ERR_DTYPE;
  if (q->shape[3] != keys->shape[3]) return RK_ERR_HEAD_DIM;
  if (G <= 0 || q->shape[0] != keys->shape[0] || q->shape[1] != keys->shape[1] * G) return RK_ERR_HEADS;
  if (window <= 0 || window > 32) return RK_ERR_ARG;
  const int64_t S = q->shape[2], D = q->shape[3];
  qw->q = q;
  qw->G = G;
  qw->W = (int)(S < window ? S : window);
  if (keys->shape[0] * keys->shape[1] > 0 && qw->W == 0) return RK_ERR_SHAPE;
  const int64_t B = keys->shape[0], H = keys->shape[1];
  // the group mean over dim 2 of [B, H_kv, G, W, D] (kv_pruning_utils.py:127-129)
  qw->inv_g = rk::mean_factor(B * H * qw->W * D, B * H * G * qw->W * D);
  qw->vec = rows_vec(q, D);
  return RK_OK;
}

}  // namespace

extern "C" int rk_key_covariance_weighted_check(const rk_tensor* keys, const rk_tensor* queries,
                                                int64_t num_kv_groups, int32_t window, const rk_tensor* mean_out,
                                                const rk_tensor* cov_out, int32_t num_cus, size_t* workspace_bytes) {
  int st = rk_key_covariance_check(keys, mean_out, cov_out, num_cus, workspace_bytes);
  if (st) return st;
  QwArgs qw;
  return check_queries(keys, queries, num_kv_groups, window, &qw);
}

extern "C" int rk_key_covariance_weighted(const rk_tensor* keys, const rk_tensor* queries, int64_t num_kv_groups,
                                          int32_t window, const rk_tensor* mean_out, const rk_tensor* cov_out,
                                          void* workspace, size_t workspace_bytes, void* stream) {
  KeyView k;
  bool vec;
  int st = key_view(keys, &k, &vec);
  if (st) return st;
  const int64_t B = keys->shape[0], H = keys->shape[1];
  if (!cov_out) return RK_ERR_NULL;
  if ((st = check_f32_out(cov_out, 4, B, H, k.D, RK_F32))) return st;
  if (mean_out && (st = check_f32_out(mean_out, 3, B, H, k.D, RK_F32))) return st;
  QwArgs qw;
  if ((st = check_queries(keys, queries, num_kv_groups, window, &qw))) return st;
  const int cus = resolve_cus(0, &st);
  if (st) return st;
  const CovPlan p = cov_plan(B, H, k.S, cus);
  if (!workspace || (((uintptr_t)workspace) & 255) || workspace_bytes < p.total) return RK_ERR_WORKSPACE;
  if (B * H == 0) return RK_OK;
  if ((k.S > 0 && !k.data) || !cov_out->data || !queries->data) return RK_ERR_NULL;
  const hipError_t e = launch_cov_any(keys->dtype, k, vec, p, B, (float*)workspace, (float*)cov_out->data, cov_out,
                                      mean_out ? (float*)mean_out->data : nullptr, mean_out, (hipStream_t)stream,
                                      &qw);
  return e == hipSuccess ? RK_OK : RK_ERR_HIP;
}

namespace {

int check_rotation(const rk_tensor* R, int64_t B, int64_t H, int64_t D, int64_t* Dk) {
  int st = rk::check_desc(R, 4);
  if (st) return st;
  if (!rk::is_float_param(R->dtype)) return RK_ERR_DTYPE;
  if (R->shape[0] != B || R->shape[1] != H || R->shape[2] != D) return RK_ERR_SHAPE;
  *Dk = R->shape[3];
  if (*Dk < 1 || *Dk > 128) return RK_ERR_KEEP_DIM;
  return RK_OK;
}

template <class TT, int NT, bool SCORE>
hipError_t launch_rot(const RotArgs& a, bool vec, dim3 grid, hipStream_t s) {
  if constexpr (TT::kBytes == 4) {
    if (vec)
      hipLaunchKernelGGL((rot32_kernel<NT, true, SCORE>), grid, dim3(kThreads), 0, s, a);
    else
      hipLaunchKernelGGL((rot32_kernel<NT, false, SCORE>), grid, dim3(kThreads), 0, s, a);
  } else {
    if (vec)
      hipLaunchKernelGGL((rot_kernel<TT, NT, true, SCORE>), grid, dim3(kThreads), 0, s, a);
    else
      hipLaunchKernelGGL((rot_kernel<TT, NT, false, SCORE>), grid, dim3(kThreads), 0, s, a);
  }
  return hipGetLastError();
}

template <class TT>
hipError_t launch_rot_nt(int nt, bool score, const RotArgs& a, bool vec, dim3 grid, hipStream_t s) {
  if (score) return launch_rot<TT, 8, true>(a, vec, grid, s);
  switch (nt) {
    case 1: return launch_rot<TT, 1, false>(a, vec, grid, s);
    case 2: return launch_rot<TT, 2, false>(a, vec, grid, s);
    case 3:
    case 4: return launch_rot<TT, 4, false>(a, vec, grid, s);
    default: return launch_rot<TT, 8, false>(a, vec, grid, s);
  }
}

hipError_t launch_rot_any(int dtype, int nt, bool score, const RotArgs& a, bool vec, dim3 grid, hipStream_t s) {
  switch (dtype) {
    case RK_F16: return launch_rot_nt<rk::F16>(nt, score, a, vec, grid, s);
    case RK_BF16: return launch_rot_nt<rk::BF16>(nt, score, a, vec, grid, s);
    default: return launch_rot_nt<rk::F32>(nt, score, a, vec, grid, s);
  }
}

void fill_rot(RotArgs& a, const KeyView& k, const rk_tensor* R, int64_t Dk) {
  a.k = k;
  a.R = R->data;
  a.r_dtype = R->dtype;
  a.R_sb = R->stride[0];
  a.R_sh = R->stride[1];
  a.R_sd = R->stride[2];
  a.R_sk = R->stride[3];
  a.Dk = (int32_t)Dk;
}

int rot_splits(int64_t bh, int64_t S, int cus) { return splits_for(bh, S, cus, 512); }

}  // namespace

extern "C" int rk_rotate_keys(const rk_tensor* keys, const rk_tensor* R_partial, const rk_tensor* out,
                              void* stream) {
  KeyView k;
  bool vec;
  int st = key_view(keys, &k, &vec);
  if (st) return st;
  const int64_t B = keys->shape[0], H = keys->shape[1];
  int64_t Dk = 0;
  if ((st = check_rotation(R_partial, B, H, k.D, &Dk))) return st;
  if ((st = rk::check_desc(out, 4))) return st;
  if (out->dtype != keys->dtype) return RK_ERR_DTYPE;
  if (out->shape[0] != B || out->shape[1] != H || out->shape[2] != k.S || out->shape[3] != Dk)
    return RK_ERR_SHAPE;
  const int cus = resolve_cus(0, &st);
  if (st) return st;
  if (B * H == 0 || k.S == 0) return RK_OK;
  if (!k.data || !R_partial->data || !out->data) return RK_ERR_NULL;
  RotArgs a;
  memset(&a, 0, sizeof(a));
  fill_rot(a, k, R_partial, Dk);
  a.out = (uint16_t*)out->data;
  a.o_sb = out->stride[0];
  a.o_sh = out->stride[1];
  a.o_ss = out->stride[2];
  a.o_sd = out->stride[3];
  a.splits = rot_splits(B * H, k.S, cus);
  a.chunk = cdiv(k.S, a.splits);
  const dim3 grid((unsigned)a.splits, (unsigned)(B * H));
  const int nt = (int)cdiv(Dk, 16);
  const hipError_t e = launch_rot_any(keys->dtype, nt, false, a, vec, grid, (hipStream_t)stream);
  return e == hipSuccess ? RK_OK : RK_ERR_HIP;
}

extern "C" int rk_channel_scores_check(const rk_tensor* keys, const rk_tensor* R_full,
                                       const rk_tensor* scores_out, int32_t num_cus,
                                       size_t* workspace_bytes) {
  KeyView k;
  bool vec;
  int st = key_view(keys, &k, &vec);
  if (st) return st;
  const int64_t B = keys->shape[0], H = keys->shape[1];
  int64_t Dk = 0;
  if ((st = check_rotation(R_full, B, H, k.D, &Dk))) return st;
  if (scores_out && (st = check_f32_out(scores_out, 3, B, H, Dk, RK_F64))) return st;
  const int cus = resolve_cus(num_cus, &st);
  if (st) return st;
  if (workspace_bytes)
    *workspace_bytes = align256((size_t)B * H * rot_splits(B * H, k.S, cus) * 128 * sizeof(float));
  return RK_OK;
}

extern "C" int rk_channel_scores(const rk_tensor* keys, const rk_tensor* R_full, const rk_tensor* scores_out,
                                 void* workspace, size_t workspace_bytes, void* stream) {
  KeyView k;
  bool vec;
  int st = key_view(keys, &k, &vec);
  if (st) return st;
  const int64_t B = keys->shape[0], H = keys->shape[1];
  int64_t Dk = 0;
  if ((st = check_rotation(R_full, B, H, k.D, &Dk))) return st;
  if (!scores_out) return RK_ERR_NULL;
  if ((st = check_f32_out(scores_out, 3, B, H, Dk, RK_F64))) return st;
  const int cus = resolve_cus(0, &st);
  if (st) return st;
  RotArgs a;
  memset(&a, 0, sizeof(a));
  fill_rot(a, k, R_full, Dk);
  a.splits = rot_splits(B * H, k.S, cus);
  a.chunk = cdiv(k.S > 0 ? k.S : 1, a.splits);
  const size_t need = align256((size_t)B * H * a.splits * 128 * sizeof(float));
  if (!workspace || (((uintptr_t)workspace) & 255) || workspace_bytes < need) return RK_ERR_WORKSPACE;
  if (B * H == 0) return RK_OK;
  if ((k.S > 0 && !k.data) || !R_full->data || !scores_out->data) return RK_ERR_NULL;
  a.spart = (float*)workspace;
  hipStream_t s = (hipStream_t)stream;
  const dim3 grid((unsigned)a.splits, (unsigned)(B * H));
  if (launch_rot_any(keys->dtype, 8, true, a, vec, grid, s) != hipSuccess) return RK_ERR_HIP;
  hipLaunchKernelGGL(scorefin_kernel, dim3((unsigned)(B * H)), dim3(128), 0, s, a.spart, a.splits, 128,
                     (int)Dk, k.S, (double*)scores_out->data, scores_out->stride[0], scores_out->stride[1],
                     scores_out->stride[2], k.H);
  return hipGetLastError() == hipSuccess ? RK_OK : RK_ERR_HIP;
}

extern "C" int rk_topk_channels(const rk_tensor* scores, int64_t k, const rk_tensor* idx_out,
                                const rk_tensor* mask_out, void* stream) {
  int st = rk::check_desc(scores, 3);
  if (st) return st;
  if (scores->dtype != RK_F64) return RK_ERR_DTYPE;
  const int64_t B = scores->shape[0], H = scores->shape[1], D = scores->shape[2];
  if (D < 1 || D > 128) return RK_ERR_SHAPE;
  if (k < 0 || k > D) return RK_ERR_KEEP_DIM;
  if (!idx_out) return RK_ERR_NULL;
  if ((st = rk::check_desc(idx_out, 3))) return st;
  if (idx_out->dtype != RK_I64) return RK_ERR_DTYPE;
  if (idx_out->shape[0] != B || idx_out->shape[1] != H || idx_out->shape[2] != k) return RK_ERR_SHAPE;
  if (mask_out) {
    if ((st = rk::check_desc(mask_out, 3))) return st;
    if (mask_out->dtype != RK_U8) return RK_ERR_DTYPE;
    if (mask_out->shape[0] != B || mask_out->shape[1] != H || mask_out->shape[2] != D) return RK_ERR_SHAPE;
  }
  if (B * H == 0) return RK_OK;
  if (!scores->data || (k > 0 && !idx_out->data) || (mask_out && !mask_out->data)) return RK_ERR_NULL;
  if (B * H > (INT64_C(1) << 30)) return RK_ERR_SHAPE;
  hipLaunchKernelGGL(topk_kernel, dim3((unsigned)(B * H)), dim3(128), 0, (hipStream_t)stream,
                     (const double*)scores->data, scores->stride[0], scores->stride[1], scores->stride[2],
                     (int)D, (int)k, (int)H, (int64_t*)idx_out->data, idx_out->stride[0], idx_out->stride[1],
                     idx_out->stride[2], mask_out ? (uint8_t*)mask_out->data : nullptr,
                     mask_out ? mask_out->stride[0] : 0, mask_out ? mask_out->stride[1] : 0,
                     mask_out ? mask_out->stride[2] : 0);
  return hipGetLastError() == hipSuccess ? RK_OK : RK_ERR_HIP;
}

extern "C" int rk_gather_rotation(const rk_tensor* R_full, const rk_tensor* idx, const rk_tensor* mean,
                                  const rk_tensor* R_out, const rk_tensor* delta_mu_out, void* stream) {
  int st = rk::check_desc(R_full, 4);
  if (st) return st;
  if (!rk::is_float_param(R_full->dtype)) return RK_ERR_DTYPE;
  const int64_t B = R_full->shape[0], H = R_full->shape[1], D = R_full->shape[2];
  if (D < 1 || D > 128) return RK_ERR_HEAD_DIM;
  if (!idx || !mean || !R_out || !delta_mu_out) return RK_ERR_NULL;
  if ((st = rk::check_desc(idx, 3))) return st;
  if (idx->dtype != RK_I64) return RK_ERR_DTYPE;
  const int64_t k = idx->shape[2];
  if (idx->shape[0] != B || idx->shape[1] != H) return RK_ERR_SHAPE;
  if (k < 1 || k > 128) return RK_ERR_KEEP_DIM;
  if ((st = check_f32_out(mean, 3, B, H, D, RK_F32))) return st;
  if ((st = rk::check_desc(R_out, 4))) return st;
  if (!rk::is_float_param(R_out->dtype)) return RK_ERR_DTYPE;
  if (R_out->shape[0] != B || R_out->shape[1] != H || R_out->shape[2] != D || R_out->shape[3] != k)
    return RK_ERR_SHAPE;
  if ((st = check_f32_out(delta_mu_out, 3, B, H, D, R_out->dtype))) return st;
  if (B * H == 0) return RK_OK;
  if (!R_full->data || !idx->data || !mean->data || !R_out->data || !delta_mu_out->data) return RK_ERR_NULL;
  if (B * H > (INT64_C(1) << 30)) return RK_ERR_SHAPE;
  hipStream_t s = (hipStream_t)stream;
  auto go = [&](auto tt) {
    using TT = decltype(tt);
    hipLaunchKernelGGL((gather_kernel<TT>), dim3((unsigned)(B * H)), dim3(128), 0, s, R_full->data,
                       (int)R_full->dtype, R_full->stride[0], R_full->stride[1], R_full->stride[2],
                       R_full->stride[3], (const int64_t*)idx->data, idx->stride[0], idx->stride[1],
                       idx->stride[2], (int)k, (const float*)mean->data, mean->stride[0], mean->stride[1],
                       mean->stride[2], R_out->data, R_out->stride[0], R_out->stride[1], R_out->stride[2],
                       R_out->stride[3], delta_mu_out->data, delta_mu_out->stride[0], delta_mu_out->stride[1],
                       delta_mu_out->stride[2], (int)H, (int)D);
  };
  if (R_out->dtype == RK_F16)
    go(rk::F16{});
  else if (R_out->dtype == RK_BF16)
    go(rk::BF16{});
  else
    go(rk::F32{});
  return hipGetLastError() == hipSuccess ? RK_OK : RK_ERR_HIP;
}

extern "C" int rk_query_weight(const rk_tensor* cov, const rk_tensor* queries, int64_t num_kv_groups,
                               int32_t window, const rk_tensor* out, void* stream) {
  if (!cov || !queries || !out) return RK_ERR_NULL;
  int st;
  if ((st = rk::check_desc(cov, 4)) || (st = rk::check_desc(queries, 4)) || (st = rk::check_desc(out, 4)))
    return st;
  if (cov->dtype != RK_F32 || out->dtype != RK_F32 || !rk::is_float_param(queries->dtype)) return RK_ERR_DTYPE;
  const int64_t B = cov->shape[0], H = cov->shape[1], D = cov->shape[2];
  if (D < 1 || D > 128 || cov->shape[3] != D || queries->shape[3] != D) return RK_ERR_HEAD_DIM;
  for (int i = 0; i < 4; ++i)
    if (out->shape[i] != cov->shape[i]) return RK_ERR_SHAPE;
  if (num_kv_groups <= 0 || queries->shape[0] != B || queries->shape[1] != H * num_kv_groups) return RK_ERR_HEADS;
  const int64_t S = queries->shape[2];
  if (window <= 0 || window > 32) return RK_ERR_ARG;
  const int W = (int)(S < window ? S : window);
  if (B * H == 0) return RK_OK;
  if (W == 0) return RK_ERR_SHAPE;
  if (!cov->data || !queries->data || !out->data) return RK_ERR_NULL;
  hipStream_t s = (hipStream_t)stream;
  const dim3 grid((unsigned)(B * H));
  // the group mean over dim 2 of [B, H_kv, G, W, D] (kv_pruning_utils.py:127-129)
  const float inv_g = rk::mean_factor(B * H * W * D, B * H * num_kv_groups * W * D);
  const float rfac = rk::mean_factor(B * H, B * H * D);  // the ridge's mean over the diagonal
  // 16-byte loads: unit inner stride, rows (and the bases) 16-byte aligned
  const bool cvec = D % 4 == 0 && cov->stride[3] == 1 && cov->stride[2] % 4 == 0 && cov->stride[1] % 4 == 0 &&
                    cov->stride[0] % 4 == 0 && ((uintptr_t)cov->data & 15) == 0;
  const bool qvec = rows_vec(queries, D);
  auto go = [&](auto kern) {
    hipLaunchKernelGGL(kern, grid, dim3(256), 0, s, (const float*)cov->data, cov->stride[0], cov->stride[1],
                       cov->stride[2], cov->stride[3], (const uint16_t*)queries->data, queries->stride[0],
                       queries->stride[1], queries->stride[2], queries->stride[3], S, W, (int)num_kv_groups, (int)D,
                       inv_g, rfac, (float*)out->data, out->stride[0], out->stride[1], out->stride[2],
                       out->stride[3], (int)H);
  };
  auto by_layout = [&](auto tt) {
    using TT = decltype(tt);
    if (cvec && qvec) go(qweight_kernel<TT, true, true>);
    else if (cvec) go(qweight_kernel<TT, true, false>);
    else if (qvec) go(qweight_kernel<TT, false, true>);
    else go(qweight_kernel<TT, false, false>);
  };
  if (queries->dtype == RK_F16)
    by_layout(rk::F16{});
  else if (queries->dtype == RK_BF16)
    by_layout(rk::BF16{});
  else
    by_layout(rk::F32{});
  return hipGetLastError() == hipSuccess ? RK_OK : RK_ERR_HIP;
}
