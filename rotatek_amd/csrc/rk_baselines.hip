// rk_baselines.hip -- the ThinK and SparK Key channel-pruning baselines on
// MI355X (gfx950): prefill scoring, selection and compaction, and the
// decode-time recovery of full-width visual Keys that both baselines feed to
// the dense decode kernel.
//
// ThinK (rotatek/baselines/think.py:15-58): one channel subset per KV head.
//   sqsum_kernel         split-S fp32 partial sums of dtype(k^2) per channel
//   think_select_kernel  keys_norm = dtype(sum * f_S), queries_norm =
//                        dtype(mean over the group of dtype(mean over the
//                        window of dtype(q^2))), score = dtype(qn * kn);
//                        prune the prune_count smallest scores -> keep mask
//                        and ascending kept indices
//   compact_kernel       K_compact[..., j] = K[..., idx[j]] over 64-token
//                        tiles staged in LDS
// SparK (rotatek/baselines/spark.py:15-60, with the group mean of the
// queries from kv_pruning_utils.py:76-79): one channel subset per token.
//   spark_qnorm_kernel   q_g = dtype(mean over the G query heads of a KV
//                        head), q_norm = dtype(||q_g||_2 over the window)
//   spark_kernel         4 lanes per token: score = dtype(dtype(k^2) qn);
//                        keep the Dk largest (bitwise search for the
//                        threshold score over packed 15-bit keys, lowest
//                        channels among the ties); writes K_compact, the
//                        per-token mask and dtype(mean of the pruned values)
// Recovery (llama_visionzip.py:216-233):
//   recover_kernel       64-row tiles of [prompt | visual | text]: the
//                        visual rows get the kept channels from K_compact
//                        (staged in LDS) in ascending channel order and 0
//                        (ThinK) or the token's pruned mean (SparK)
//                        elsewhere; prompt and text rows are copied, so the
//                        caller's torch.cat of the three spans is written by
//                        the same pass.
//   selection_kernel     one-hot R[c][j] = (c is the j-th kept channel) from
//                        a per-head mask, so the RotateK decode kernel can
//                        run ThinK's zero-filled attention from K_compact.
//
// Head dim D <= 128: the kernels keep 128 channel slots (lanes, LDS
// columns, workspace rows) and treat slots at or past D as absent: their
// loads are not issued and read as zeros, their selection keys sit below
// every real channel's, and nothing is written for them.  16-byte row
// paths need D % 8 == 0 (whole 8-channel groups in or out).
//
// Mean factors: torch reduces a 16-bit mean as dtype(fp32 sum * f) with
// f = float(n_out) / float(n_in) (ATen MeanOps); the host computes each f
// that way and passes it in.  Ties: torch's GPU topk (largest=False) takes
// equal values at the boundary in index order, so ThinK prunes the lower
// channel first; the GPU sort behind argsort(descending) keeps equal values
// in index order, so SparK keeps the lower channel first.  Scores are compared
// through order-preserving 16-bit keys (NaN highest, -0 == +0).
#include <math.h>

#include "rk_common.h"
#include "rk_host.h"
#include "rotatek_hip.h"

namespace rk {
namespace base {

constexpr int kThreads = 256;
constexpr int kD = 128;

// [B, H, S, C] tensor of 16-bit elements, strides in elements.
struct View {
  const uint16_t* data;
  int64_t sb, sh, ss, sc;
  int64_t S;
  int32_t H, C;
};

struct OutView {
  uint16_t* data;
  int64_t sb, sh, ss, sc;
};

struct MaskView {
  uint8_t* data;
  int64_t sb, sh, ss, sc;  // ss is 0 for a per-head mask
};

__device__ __forceinline__ int64_t head_off(int64_t sb, int64_t sh, int b, int h) {
  return b * sb + (int64_t)h * sh;
}

// Keeps an fp32 result as fp32 so that the conversion which follows rounds
// that fp32 value (fp32 op, then cast, as torch does) instead of being fused
// with the op into one mixed-precision multiply-and-round.
__device__ __forceinline__ float pin(float x) {
  asm volatile("" : "+v"(x));
  return x;
}

template <class TT>
__device__ __forceinline__ float rnd(float x) {
  return TT::to_f32(TT::from_f32(x));
}

// Order-preserving key of a 16-bit float value: larger value -> larger key,
// -0 == +0, every NaN above +inf (torch's sort and topk order NaN highest).
template <class TT>
__device__ __forceinline__ uint32_t order_key(float v) {
  if (v != v) return 0xFFFFu;
  uint32_t b = TT::from_f32(v);
  if (v == 0.f) b = 0u;
  return (b & 0x8000u) ? (~b & 0xFFFFu) : (b | 0x8000u);
}

// Channels c0 .. c0 + 7 of row t; channels at or past D read as zeros (no
// load).  VEC: one 16-byte load (D % 8 == 0, so the group is all in or out).
template <bool VEC>
__device__ __forceinline__ uint4 ld8(const uint16_t* base, int64_t ss, int64_t sc, int64_t t, int c0, int D) {
  if constexpr (VEC) {
    return c0 < D ? *(const uint4*)(base + t * ss + c0) : make_uint4(0u, 0u, 0u, 0u);
  } else {
    uint32_t w[4] = {0, 0, 0, 0};
#pragma unroll
    for (int e = 0; e < 8; ++e)
      if (c0 + e < D) w[e >> 1] |= (uint32_t)base[t * ss + (c0 + e) * sc] << ((e & 1) * 16);
    return make_uint4(w[0], w[1], w[2], w[3]);
  }
}

// Eight elements to row t at channel c0.  VEC: one non-temporal 16-byte
// store (the recovered Keys are written once and read by the next kernel
// far beyond L2 / MALL capacity; measured ~2 % faster recover + decode).
// (channels at or past D are not written)
template <bool VEC>
__device__ __forceinline__ void st8(uint16_t* base, int64_t ss, int64_t sc, int64_t t, int c0, const uint4& v,
                                    int D) {
  if constexpr (VEC) {
    const u32x4 w = {v.x, v.y, v.z, v.w};
    if (c0 < D) __builtin_nontemporal_store(w, (u32x4*)(base + t * ss + c0));
  } else {
#pragma unroll
    for (int e = 0; e < 8; ++e)
      if (c0 + e < D) base[t * ss + (c0 + e) * sc] = (uint16_t)(word(v, e >> 1) >> ((e & 1) * 16));
  }
}

// Kept flags of the eight mask bytes p[0], p[sc], ..., p[7 sc] (bit e set
// when byte e is non-zero), n of them present (the rest read as pruned, not
// loaded); VEC: one 8-byte load (sc == 1, 8-byte aligned, n 0 or 8).
template <bool VEC>
__device__ __forceinline__ uint32_t mask8(const uint8_t* p, int64_t sc, int n) {
  uint32_t f = 0u;
  if constexpr (VEC) {
    if (n <= 0) return 0u;
    const uint64_t m = *(const uint64_t*)p;
#pragma unroll
    for (int e = 0; e < 8; ++e) f |= (((m >> (8 * e)) & 0xFFu) != 0u ? 1u : 0u) << e;
  } else {
#pragma unroll
    for (int e = 0; e < 8; ++e)
      if (e < n) f |= (p[e * sc] != 0 ? 1u : 0u) << e;
  }
  return f;
}

// Exclusive prefix sum of v over the 16 lanes of this lane's row of the
// wave (every lane of the row must call it).
__device__ __forceinline__ int prefix16(int v) {
  const int l16 = threadIdx.x & 15;
  int incl = v;
#pragma unroll
  for (int d = 1; d < 16; d <<= 1) {
    const int y = __shfl_up(incl, d, 16);
    if (l16 >= d) incl += y;
  }
  return incl - v;
}

// Sum of v over the 16 lanes of this lane's row, in every lane of the row
// (DPP row rotations by 8, 4, 2, 1).
__device__ __forceinline__ int sum16(int v) {
  v += __builtin_amdgcn_update_dpp(0, v, 0x128, 0xF, 0xF, false);
  v += __builtin_amdgcn_update_dpp(0, v, 0x124, 0xF, 0xF, false);
  v += __builtin_amdgcn_update_dpp(0, v, 0x122, 0xF, 0xF, false);
  v += __builtin_amdgcn_update_dpp(0, v, 0x121, 0xF, 0xF, false);
  return v;
}

template <int CTL>
__device__ __forceinline__ float fdpp(float v) {
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTL, 0xF, 0xF, false));
}

__device__ __forceinline__ float fsum16(float v) {
  v += fdpp<0x128>(v);
  v += fdpp<0x124>(v);
  v += fdpp<0x122>(v);
  v += fdpp<0x121>(v);
  return v;
}

// Exclusive prefix sum of v over the 16 lanes of this lane's row (DPP row
// shifts by 1, 2, 4, 8 with zero fill).
__device__ __forceinline__ int scan16(int v) {
  int x = v;
  x += __builtin_amdgcn_update_dpp(0, x, 0x111, 0xF, 0xF, true);
  x += __builtin_amdgcn_update_dpp(0, x, 0x112, 0xF, 0xF, true);
  x += __builtin_amdgcn_update_dpp(0, x, 0x114, 0xF, 0xF, true);
  x += __builtin_amdgcn_update_dpp(0, x, 0x118, 0xF, 0xF, true);
  return x - v;
}

constexpr int kTile = 64;     // token rows per workgroup tile
constexpr int kTilePad = 8;   // LDS row padding (elements): 16-byte aligned rows

// ------------------------------------------------------------------ ThinK
// grid (splits, B*H): workgroup x sums dtype(k^2) over tokens
// [x*chunk, (x+1)*chunk) of one head into part[bh][x][128].  Thread (row
// group rg = t/16, channel chunk c8 = t%16) walks rows rg, rg+16, ...
template <class TT, bool VEC>
__global__ void __launch_bounds__(kThreads) sqsum_kernel(View k, int64_t chunk, int splits, float* part) {
  __shared__ float s_sum[16][kD];
  const int tid = threadIdx.x, rg = tid >> 4, c8 = tid & 15;
  const int x = blockIdx.x, bh = blockIdx.y, b = bh / k.H, h = bh - b * k.H;
  const uint16_t* base = k.data + head_off(k.sb, k.sh, b, h);
  const int64_t t0 = (int64_t)x * chunk, t1 = min(k.S, t0 + chunk);
  const int64_t last = max(t1 - 1, (int64_t)0);
  float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
  for (int64_t t = t0 + rg; t < t1; t += 64) {
    uint4 v[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) v[i] = ld8<VEC>(base, k.ss, k.sc, min(t + 16 * i, last), 8 * c8, k.C);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      if (t + 16 * i < t1) {
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const float f = TT::to_f32((uint16_t)(word(v[i], e >> 1) >> ((e & 1) * 16)));
          acc[e] += rnd<TT>(f * f);  // f * f is exact in fp32
        }
      }
    }
  }
#pragma unroll
  for (int e = 0; e < 8; ++e) s_sum[rg][8 * c8 + e] = acc[e];
  __syncthreads();
  if (tid < kD) {
    float s = 0.f;
#pragma unroll
    for (int r = 0; r < 16; ++r) s += s_sum[r][tid];
    part[((int64_t)bh * splits + x) * kD + tid] = s;
  }
}

struct ThinkArgs {
  const float* part;
  int splits;
  View q;        // queries_recent [B, H_q, Q, D]
  int G;         // query heads per KV head
  int keep;      // kept channels
  int H;         // KV heads
  float f_keys;  // mean factor over S_v
  float f_win;   // mean factor over the Q window
  float f_grp;   // mean factor over the G heads
  MaskView mask;
  int32_t* idx;  // [B*H][128] ascending kept channels
  int D;         // head dim (channels past it take no part)
};

// grid (B*H), 128 threads (one per channel slot).
template <class TT>
__global__ void __launch_bounds__(kD) think_select_kernel(const ThinkArgs a) {
  __shared__ uint32_t s_key[kD];
  __shared__ int s_kept[kD];
  const int c = threadIdx.x, bh = blockIdx.x, b = bh / a.H, h = bh - b * a.H;
  float s = 0.f;
  for (int x = 0; x < a.splits; ++x) s += a.part[((int64_t)bh * a.splits + x) * kD + c];
  const float kn = rnd<TT>(pin(s * a.f_keys));
  const bool real = c < a.D;
  float qacc = 0.f;
  for (int gi = 0; gi < (real ? a.G : 0); ++gi) {
    const uint16_t* qb = a.q.data + head_off(a.q.sb, a.q.sh, b, h * a.G + gi) + c * a.q.sc;
    float w = 0.f;
    for (int64_t t = 0; t < a.q.S; ++t) {
      const float x = TT::to_f32(qb[t * a.q.ss]);
      w += rnd<TT>(x * x);
    }
    qacc += rnd<TT>(pin(w * a.f_win));
  }
  const float qn = rnd<TT>(pin(qacc * a.f_grp));
  const float score = rnd<TT>(qn * kn);  // product of two 16-bit values: exact in fp32
  // (order keys are >= 0x7F, so a slot past D, key 0, is below every channel)
  const uint32_t key = real ? (order_key<TT>(score) << 7) | (uint32_t)c : 0u;
  s_key[c] = key;
  __syncthreads();
  int above = 0;
  for (int j = 0; j < kD; ++j) above += s_key[j] > key;
  const int kept = real && above < a.keep;
  s_kept[c] = kept;
  if (real) a.mask.data[head_off(a.mask.sb, a.mask.sh, b, h) + c * a.mask.sc] = (uint8_t)kept;
  __syncthreads();
  if (kept) {
    int pos = 0;
    for (int j = 0; j < c; ++j) pos += s_kept[j];
    a.idx[(int64_t)bh * kD + pos] = c;
  }
}

// grid (splits, B*H): K_compact[b,h,t,j] = K[b,h,t,idx[j]].  Tiles of 64
// tokens are staged in LDS with 16-byte loads (thread t loads channels
// 8(t%16).. of rows t/16 + 16i); thread t then gathers output columns
// 8(t%16)..+7 of the same rows from LDS (threads past Dk idle).  OVEC: one
// 16-byte store per chunk (unit stride, aligned rows, Dk % 8 == 0).
template <bool VEC, bool OVEC>
__global__ void __launch_bounds__(kThreads) compact_kernel(View k, const int32_t* idx, int Dk, int64_t chunk,
                                                           OutView o) {
  __shared__ __align__(16) uint16_t s_k[kTile * (kD + kTilePad)];
  const int tid = threadIdx.x, c8 = tid & 15, rq = tid >> 4;
  const int x = blockIdx.x, bh = blockIdx.y, b = bh / k.H, h = bh - b * k.H;
  int src[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) src[e] = 8 * c8 + e < Dk ? idx[(int64_t)bh * kD + 8 * c8 + e] : 0;
  const uint16_t* base = k.data + head_off(k.sb, k.sh, b, h);
  uint16_t* ob = o.data + head_off(o.sb, o.sh, b, h);
  const int64_t t0 = (int64_t)x * chunk, t1 = min(k.S, t0 + chunk);
  for (int64_t tile = t0; tile < t1; tile += kTile) {
#pragma unroll
    for (int i = 0; i < kTile / 16; ++i) {
      const int64_t t = tile + rq + 16 * i;
      if (t < t1)
        *(uint4*)(s_k + (rq + 16 * i) * (kD + kTilePad) + 8 * c8) = ld8<VEC>(base, k.ss, k.sc, t, 8 * c8, k.C);
    }
    __syncthreads();
    if (8 * c8 < Dk) {
#pragma unroll
      for (int i = 0; i < kTile / 16; ++i) {
        const int64_t t = tile + rq + 16 * i;
        if (t >= t1) continue;
        const uint16_t* row = s_k + (rq + 16 * i) * (kD + kTilePad);
        uint32_t w[4] = {0u, 0u, 0u, 0u};
#pragma unroll
        for (int e = 0; e < 8; ++e) w[e >> 1] |= (uint32_t)row[src[e]] << ((e & 1) * 16);
        if constexpr (OVEC) {
          *(uint4*)(ob + t * o.ss + 8 * c8) = make_uint4(w[0], w[1], w[2], w[3]);
        } else {
#pragma unroll
          for (int e = 0; e < 8; ++e)
            if (8 * c8 + e < Dk) ob[t * o.ss + (8 * c8 + e) * o.sc] = (uint16_t)(w[e >> 1] >> ((e & 1) * 16));
        }
      }
    }
    __syncthreads();
  }
}

// ------------------------------------------------------------------ SparK
// grid (B*H), 128 threads: qn[bh][c] = dtype(sqrt(sum_t q_g[t][c]^2)) with
// q_g[t][c] = dtype(sum over the G query heads * f_grp).
template <class TT>
__global__ void __launch_bounds__(kD) spark_qnorm_kernel(View q, int G, int H, float f_grp, float* qn) {
  const int c = threadIdx.x, bh = blockIdx.x, b = bh / H, h = bh - b * H;
  float acc = 0.f;
  for (int64_t t = 0; t < (c < q.C ? q.S : 0); ++t) {
    float s = 0.f;
    for (int gi = 0; gi < G; ++gi) s += TT::to_f32(q.data[head_off(q.sb, q.sh, b, h * G + gi) + t * q.ss + c * q.sc]);
    const float g = rnd<TT>(pin(s * f_grp));
    acc = fmaf(g, g, acc);  // g * g is exact, so fused or not gives the same sum
  }
  qn[(int64_t)bh * kD + c] = rnd<TT>(sqrtf(acc));
}

struct SparkArgs {
  View k;
  const float* qn;
  int keep;
  int64_t chunk;
  float f_pruned;  // mean factor over the pruned channels
  OutView kc;      // [B, H, S, Dk]
  MaskView mask;   // [B, H, S, D]
  OutView pm;      // [B, H, S, 1]
};

// Packed 16-bit lanes: two channels per dword, the lower channel in the low
// half.
typedef unsigned short u16x2 __attribute__((ext_vector_type(2)));
typedef short i16x2 __attribute__((ext_vector_type(2)));
typedef _Float16 h16x2 __attribute__((ext_vector_type(2)));
typedef __bf16 b16x2 __attribute__((ext_vector_type(2)));

// Scores of one lane's 32 channels, two per dword: dtype(dtype(k^2) qn)
// (spark.py:40-41; every product of two 16-bit values is exact in fp32, so
// one rounding per operation matches torch's op-by-op result).
template <class TT>
struct SparkScore;

template <>
struct SparkScore<F16> {
  uint32_t q[16];  // qn of the lane's channels, packed f16 (qn is f16-exact)
  static constexpr uint32_t kNaNKey = 0x7C01u;
  __device__ __forceinline__ void init(const float* qn) {
#pragma unroll
    for (int i = 0; i < 16; ++i) q[i] = F16::pack2(qn[2 * i], qn[2 * i + 1]);
  }
  __device__ __forceinline__ uint32_t score(uint32_t kw, int i) const {
    const h16x2 k = __builtin_bit_cast(h16x2, kw);
    const h16x2 k2 = k * k;  // rounded to f16, as torch.pow
    const h16x2 s = k2 * __builtin_bit_cast(h16x2, q[i]);
    return __builtin_bit_cast(uint32_t, s);
  }
  // acc + both halves of w (fp32 accumulate)
  static __device__ __forceinline__ float add2(uint32_t w, float acc) {
    const h16x2 one = {(_Float16)1.0f, (_Float16)1.0f};
    return __builtin_amdgcn_fdot2(__builtin_bit_cast(h16x2, w), one, acc, false);
  }
};

template <>
struct SparkScore<BF16> {
  float q[32];  // qn of the lane's channels (bf16-exact)
  static constexpr uint32_t kNaNKey = 0x7F81u;
  __device__ __forceinline__ void init(const float* qn) {
#pragma unroll
    for (int j = 0; j < 32; ++j) q[j] = qn[j];
  }
  __device__ __forceinline__ uint32_t score(uint32_t kw, int i) const {
    const float k0 = __builtin_bit_cast(float, kw << 16), k1 = __builtin_bit_cast(float, kw & 0xFFFF0000u);
    const uint32_t sq = BF16::pack2(k0 * k0, k1 * k1);
    return BF16::pack2(__builtin_bit_cast(float, sq << 16) * q[2 * i],
                       __builtin_bit_cast(float, sq & 0xFFFF0000u) * q[2 * i + 1]);
  }
  static __device__ __forceinline__ float add2(uint32_t w, float acc) {
    const b16x2 one = {(__bf16)1.0f, (__bf16)1.0f};
    return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(b16x2, w), one, acc, false);
  }
};

// Number of the lane's 32 keys (15-bit, two per dword) >= cand, cand >= 1,
// given ksum = the sum of the 32 keys.  Each half of cm - key (packed u16,
// wrapping) is cm - key + 2^16 [key > cm] with cm = cand - 1, so the
// v_dot2_u32_u16 sum of those halves is 32 cm - ksum + 2^16 #{key >= cand}:
// two instructions per two keys.
__device__ __forceinline__ int count_ge(const uint32_t (&key)[16], uint32_t ksum, uint32_t cand) {
  const unsigned short c = (unsigned short)(cand - 1u);
  const u16x2 cm = {c, c}, one = {1, 1};
  uint32_t acc = ksum - 32u * (cand - 1u);  // mod 2^32: ends at 2^16 #{key >= cand}
#pragma unroll
  for (int i = 0; i < 16; ++i) acc = __builtin_amdgcn_udot2(cm - __builtin_bit_cast(u16x2, key[i]), one, acc, false);
  return (int)(acc >> 16);
}

// Sum over the four lanes of this lane's quad (DPP quad permutations).
__device__ __forceinline__ int qsum(int v) {
  v += __builtin_amdgcn_update_dpp(0, v, 0xB1, 0xF, 0xF, false);  // quad_perm [1,0,3,2]
  v += __builtin_amdgcn_update_dpp(0, v, 0x4E, 0xF, 0xF, false);  // quad_perm [2,3,0,1]
  return v;
}
__device__ __forceinline__ float qsumf(float v) {
  v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0xB1, 0xF, 0xF, false));
  v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x4E, 0xF, 0xF, false));
  return v;
}
// Exclusive prefix sum over the lanes of the quad below this one.
__device__ __forceinline__ int qprefix(int v) {
  const int q = threadIdx.x & 3;
  int incl = v;
  int t = __shfl_up(incl, 1, 4);
  if (q >= 1) incl += t;
  t = __shfl_up(incl, 2, 4);
  if (q >= 2) incl += t;
  return incl - v;
}

// grid (splits, B*H).  Each lane quad of a wave owns one token (lane q of
// the quad: channels 32q..32q+31, four 16-byte loads), so a wave selects 16
// tokens at once and a workgroup 64; the next 64 rows are loaded while the
// current ones are selected.  Per token: 15-bit order-preserving score keys
// (NaN highest, every NaN equal), kept two per dword; the keep-th largest
// key T by a bitwise search whose counts take three packed 16-bit
// operations per two keys; every channel above T is kept and, of those
// equal to T, the lowest channels up to keep (a per-channel pass, taken by a
// wave only where some token's ties straddle the boundary).  The kept values
// are compacted through LDS in channel order.  MVEC: 8-byte mask stores.
template <class TT, bool KVEC, bool MVEC, bool CVEC>
__global__ void __launch_bounds__(kThreads) spark_kernel(const SparkArgs a) {
  constexpr int kRow = kD + 8;  // compact row slot; element kD is the sink of pruned values
  __shared__ __align__(16) uint16_t s_row[kThreads / 4][kRow];
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6, qd = lane >> 2, q = lane & 3;
  const int x = blockIdx.x, bh = blockIdx.y, b = bh / a.k.H, h = bh - b * a.k.H;
  SparkScore<TT> sc;
  {
    float qv[32];
#pragma unroll
    for (int j = 0; j < 32; ++j) qv[j] = a.qn[(int64_t)bh * kD + 32 * q + j];
    sc.init(qv);
  }
  const uint16_t* kb = a.k.data + head_off(a.k.sb, a.k.sh, b, h);
  uint16_t* cb = a.kc.data + head_off(a.kc.sb, a.kc.sh, b, h);
  uint8_t* mb = a.mask.data + head_off(a.mask.sb, a.mask.sh, b, h);
  uint16_t* pb = a.pm.data + head_off(a.pm.sb, a.pm.sh, b, h);
  const int64_t t0 = (int64_t)x * a.chunk, t1 = min(a.k.S, t0 + a.chunk);
  const int keep = a.keep;
  uint16_t* row = s_row[threadIdx.x >> 2];
  auto load = [&](uint4 (&v)[4], int64_t tb) {
    const int64_t t = min(tb + qd, t1 - 1);
#pragma unroll
    for (int i = 0; i < 4; ++i) v[i] = ld8<KVEC>(kb, a.k.ss, a.k.sc, t, 32 * q + 8 * i, a.k.C);
  };

  uint4 cur[4], nxt[4];
  int64_t tb = t0 + 16 * w;  // this wave's first token group; groups advance by 64 tokens
  if (tb < t1) load(cur, tb);
  for (; tb < t1; tb += 64) {  // wave-uniform loop
    if (tb + 64 < t1) load(nxt, tb + 64);
    const int64_t t = tb + qd;
    uint32_t kw[16], pm[16];  // raw values; then 0xFFFF per pruned channel
#pragma unroll
    for (int i = 0; i < 16; ++i) kw[i] = word(cur[i >> 2], i & 3);
    if (keep >= kD) {
#pragma unroll
      for (int i = 0; i < 16; ++i) pm[i] = 0u;
    } else if (keep <= 0) {
#pragma unroll
      for (int i = 0; i < 16; ++i) pm[i] = 0xFFFFFFFFu;
    } else {
      uint32_t key[16];
      const u16x2 nan_key = {(unsigned short)SparkScore<TT>::kNaNKey, (unsigned short)SparkScore<TT>::kNaNKey};
#pragma unroll
      for (int i = 0; i < 16; ++i)  // |score| bits (scores are >= 0), every NaN -> one key above inf
        key[i] = __builtin_bit_cast(
            uint32_t, __builtin_elementwise_min(__builtin_bit_cast(u16x2, sc.score(kw[i], i) & 0x7FFF7FFFu), nan_key));
      uint32_t ksum = 0u;
      const u16x2 one = {1, 1};
#pragma unroll
      for (int i = 0; i < 16; ++i) ksum = __builtin_amdgcn_udot2(__builtin_bit_cast(u16x2, key[i]), one, ksum, false);
      uint32_t T = 0u;  // largest T with #{key >= T} >= keep in this token
#pragma unroll
      for (int bit = 14; bit >= 0; --bit) {
        const uint32_t cand = T | (1u << bit);
        T = qsum(count_ge(key, ksum, cand)) >= keep ? cand : T;
      }
      const int ge = T == 0u ? 32 : count_ge(key, ksum, T), gt = count_ge(key, ksum, T + 1u);
      const int need = keep - qsum(gt), eq = qsum(ge - gt);
      const unsigned short Ts = (unsigned short)T;
      const u16x2 T2 = {Ts, Ts};
#pragma unroll
      for (int i = 0; i < 16; ++i)  // key < T: the wrapped 15-bit difference is negative
        pm[i] = __builtin_bit_cast(uint32_t, __builtin_bit_cast(i16x2, __builtin_bit_cast(u16x2, key[i]) - T2) >> 15);
      if (__any(need != eq)) {  // some token keeps only part of its ties: lowest channels first
        int run = qprefix(ge - gt);
#pragma unroll
        for (int i = 0; i < 16; ++i) {
#pragma unroll
          for (int hh = 0; hh < 2; ++hh) {
            const uint32_t k = (key[i] >> (16 * hh)) & 0xFFFFu;
            const bool tie = k == T;
            if (tie && run >= need) pm[i] |= 0xFFFFu << (16 * hh);
            run += tie;
          }
        }
      }
    }
    // kept values -> LDS in channel order, the rest to the sink slot
    int kept = 0;
#pragma unroll
    for (int i = 0; i < 16; ++i) kept += (int)((~pm[i]) & 1u) + (int)((~pm[i] >> 16) & 1u);
    int pos = qprefix(kept);
    float psum = 0.f;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      psum = SparkScore<TT>::add2(kw[i] & pm[i], psum);  // the pruned values (kept ones read as +0)
#pragma unroll
      for (int hh = 0; hh < 2; ++hh) {
        const uint16_t v = (uint16_t)(kw[i] >> (16 * hh));
        const bool k = ((pm[i] >> (16 * hh)) & 1u) == 0u;
        row[k ? pos : kD] = v;
        pos += k;
      }
    }
    psum = qsumf(psum);
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    if (t < t1) {
      if constexpr (CVEC) {
        for (int c = q; 8 * c < keep; c += 4) *(uint4*)(cb + t * a.kc.ss + 8 * c) = *(const uint4*)(row + 8 * c);
      } else {
        for (int e = q; e < keep; e += 4) cb[t * a.kc.ss + e * a.kc.sc] = row[e];
      }
      // kept flags as bytes: bytes 0 and 2 of two mask dwords -> channels 4d..4d+3
      // (none written past D; MVEC: D % 8 == 0)
#pragma unroll
      for (int d = 0; d < 8; ++d) {
        const uint32_t m4 = ~__builtin_amdgcn_perm(pm[2 * d + 1], pm[2 * d], 0x06040200u) & 0x01010101u;
        if constexpr (MVEC) {
          if ((d & 1) == 0 || 32 * q + 4 * (d - 1) >= a.k.C) continue;
          const uint32_t m0 = ~__builtin_amdgcn_perm(pm[2 * d - 1], pm[2 * d - 2], 0x06040200u) & 0x01010101u;
          *(uint64_t*)(mb + t * a.mask.ss + 32 * q + 4 * (d - 1)) = (uint64_t)m0 | ((uint64_t)m4 << 32);
        } else {
#pragma unroll
          for (int e = 0; e < 4; ++e)
            if (32 * q + 4 * d + e < a.k.C)
              mb[t * a.mask.ss + (32 * q + 4 * d + e) * a.mask.sc] = (uint8_t)((m4 >> (8 * e)) & 1u);
        }
      }
      if (q == 0) pb[t * a.pm.ss] = TT::from_f32(pin(psum * a.f_pruned));
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
#pragma unroll
    for (int i = 0; i < 4; ++i) cur[i] = nxt[i];
  }
}

// ------------------------------------------------------------------ recovery
struct RecoverArgs {
  View pr;  // prompt rows (S = 0 when absent)
  View kc;  // K_compact [B, H, S_v, Dk]
  View tx;  // text rows (S = 0 when absent)
  MaskView mask;         // ThinK [B, H, D] (ss = 0) or SparK [B, H, S_v, D]
  const uint16_t* pm;    // SparK pruned mean [B, H, S_v, 1]
  int64_t p_sb, p_sh, p_ss;
  OutView out;           // [B, H, rows, D]
  int64_t rows, chunk;
  int H;
  int D;                 // head dim
};

// grid (splits, B*H); tiles of 64 output rows.  The tile's compact rows are
// staged in LDS (4 threads per row), then thread t writes channels
// 8(t%16)..+7 of rows t/16 + 16i: prompt / text rows are copied, a visual
// row's kept channel of rank r (ascending channel order) takes column r of
// K_compact and the others 0 (ThinK) or the row's pruned mean (SparK).
// Ranks come from 16-lane prefix sums of the mask popcounts; ranks >= Dk (a
// mask row with more than Dk kept channels) are filled like pruned channels,
// so no read leaves the row.  FAST: 16-byte loads and stores of every span
// (unit channel stride, aligned rows), 8-byte mask loads, Dk % 8 == 0.
// DFULL: head dim 128, so the channel guards fold away (they cost the
// SparK recovery 7 % at config 2's shapes when left to run time).
template <bool SPARK, bool FAST, bool DFULL>
__global__ void __launch_bounds__(kThreads) recover_kernel(const RecoverArgs a) {
  __shared__ __align__(16) uint16_t s_c[kTile * kD];
  const int tid = threadIdx.x, c8 = tid & 15, rq = tid >> 4;
  const int x = blockIdx.x, bh = blockIdx.y, b = bh / a.H, h = bh - b * a.H;
  const int Dk = a.kc.C;
  const int64_t Sp = a.pr.S, Sv = a.kc.S;
  const uint16_t* pb = a.pr.data + head_off(a.pr.sb, a.pr.sh, b, h);
  const uint16_t* kb = a.kc.data + head_off(a.kc.sb, a.kc.sh, b, h);
  const uint16_t* tb = a.tx.data + head_off(a.tx.sb, a.tx.sh, b, h);
  const uint8_t* mb = a.mask.data + head_off(a.mask.sb, a.mask.sh, b, h);
  const uint16_t* fb = SPARK ? a.pm + head_off(a.p_sb, a.p_sh, b, h) : nullptr;
  uint16_t* ob = a.out.data + head_off(a.out.sb, a.out.sh, b, h);
  const int D = DFULL ? kD : a.D, nch = min(max(D - 8 * c8, 0), 8);  // this lane's channels present
  int map[8];  // ThinK: K_compact column of channel 8 c8 + e, -1 = pruned
  if constexpr (!SPARK) {
    const uint32_t f = mask8<false>(mb + 8 * c8 * a.mask.sc, a.mask.sc, nch);
    int rank = prefix16(__popc(f));
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const bool kept = (f >> e) & 1u;
      map[e] = (kept && rank < Dk) ? rank : -1;
      rank += kept;
    }
  }
  const int64_t r0 = (int64_t)x * a.chunk, r1 = min(a.rows, r0 + a.chunk);
  for (int64_t tile = r0; tile < r1; tile += kTile) {
    const int64_t v0 = max(tile, Sp), v1 = min(min(tile + kTile, r1), Sp + Sv);
    if (v0 < v1) {  // stage the tile's visual rows (workgroup-uniform)
      const int row = tid >> 2, nrow = (int)(v1 - v0), off = (int)(v0 - tile);
      if (row < nrow) {
        const uint16_t* src = kb + (v0 - Sp + row) * a.kc.ss;
        uint16_t* dst = s_c + (off + row) * kD;
        if constexpr (FAST) {
          for (int cc = tid & 3; cc < (Dk >> 3); cc += 4) *(uint4*)(dst + 8 * cc) = *(const uint4*)(src + 8 * cc);
        } else {
          for (int cc = tid & 3; cc < Dk; cc += 4) dst[cc] = src[cc * a.kc.sc];
        }
      }
    }
    __syncthreads();
#pragma unroll
    for (int i = 0; i < kTile / 16; ++i) {
      const int64_t r = tile + rq + 16 * i;
      const bool live = r < r1, vis = live && r >= Sp && r < Sp + Sv;
      uint32_t f = 0u;
      if constexpr (SPARK) {
        if (vis) f = mask8<FAST>(mb + (r - Sp) * a.mask.ss + 8 * c8 * a.mask.sc, a.mask.sc, nch);
      }
      int rank = SPARK ? prefix16(__popc(f)) : 0;  // every lane of the row takes part
      if (!live) continue;
      uint4 v;
      if (r < Sp) {
        v = ld8<FAST>(pb, a.pr.ss, a.pr.sc, r, 8 * c8, D);
      } else if (vis) {
        const uint16_t* row = s_c + (r - tile) * kD;
        uint32_t w[4] = {0u, 0u, 0u, 0u};
        if constexpr (SPARK) {
          const uint32_t fill = fb[(r - Sp) * a.p_ss];
#pragma unroll
          for (int e = 0; e < 8; ++e) {
            const bool kept = (f >> e) & 1u;
            const uint32_t val = (kept && rank < Dk) ? (uint32_t)row[rank] : fill;
            rank += kept;
            w[e >> 1] |= val << ((e & 1) * 16);
          }
        } else {
#pragma unroll
          for (int e = 0; e < 8; ++e) w[e >> 1] |= (map[e] >= 0 ? (uint32_t)row[map[e]] : 0u) << ((e & 1) * 16);
        }
        v = make_uint4(w[0], w[1], w[2], w[3]);
      } else {
        v = ld8<FAST>(tb, a.tx.ss, a.tx.sc, r - Sp - Sv, 8 * c8, D);
      }
      st8<FAST>(ob, a.out.ss, a.out.sc, r, 8 * c8, v, D);
    }
    __syncthreads();
  }
}

// grid (B*H), 128 threads: R[b,h,c,j] = 1 if c is the j-th kept channel of
// the head's mask (ascending), else 0, for the D rows c < D; `one` is 1.0
// in R's dtype.
template <class E>
__global__ void __launch_bounds__(kD) selection_kernel(MaskView m, int H, int D, int Dk, E* R, int64_t r_sb,
                                                       int64_t r_sh, int64_t r_sr, int64_t r_sc, E one) {
  __shared__ int s_kept[kD];
  const int c = threadIdx.x, bh = blockIdx.x, b = bh / H, h = bh - b * H;
  const int kept = c < D && m.data[head_off(m.sb, m.sh, b, h) + c * m.sc] != 0;
  s_kept[c] = kept;
  __syncthreads();
  if (c >= D) return;
  int pos = 0;
  for (int j = 0; j < c; ++j) pos += s_kept[j];
  E* row = R + head_off(r_sb, r_sh, b, h) + c * r_sr;
  for (int j = 0; j < Dk; ++j) row[j * r_sc] = (kept && pos == j) ? one : (E)0;
}

}  // namespace base
}  // namespace rk

// =====================================================================
// host side
// =====================================================================
namespace {

using namespace rk::base;

int64_t cdiv(int64_t a, int64_t b) { return (a + b - 1) / b; }
size_t align256(size_t x) { return (x + 255) & ~size_t(255); }

using rk::mean_factor;

// [B, H, S, C] descriptor of a 16-bit float tensor: a head dim 1 <= C <=
// 128 (want_c == 0), C == want_c (> 0), or any C <= 128 (want_c < 0).
int view_of(const rk_tensor* t, int want_c, View* v) {
  int st = rk::check_desc(t, 4);
  if (st) return st;
  if (!rk::is_half(t->dtype)) return RK_ERR_DTYPE;
  if (want_c == 0) {
    if (t->shape[3] < 1 || t->shape[3] > 128) return RK_ERR_HEAD_DIM;
  } else if (want_c > 0 ? t->shape[3] != want_c : t->shape[3] > 128) {
    return RK_ERR_SHAPE;
  }
  if (t->shape[1] > (INT64_C(1) << 30) || t->shape[0] * t->shape[1] > (INT64_C(1) << 30)) return RK_ERR_SHAPE;
  v->data = (const uint16_t*)t->data;
  v->sb = t->stride[0];
  v->sh = t->stride[1];
  v->ss = t->stride[2];
  v->sc = t->stride[3];
  v->S = t->shape[2];
  v->H = (int32_t)t->shape[1];
  v->C = (int32_t)t->shape[3];
  return RK_OK;
}

OutView out_of(const rk_tensor* t) {
  OutView o;
  o.data = (uint16_t*)t->data;
  o.sb = t->stride[0];
  o.sh = t->stride[1];
  o.ss = t->stride[2];
  o.sc = t->stride[3];
  return o;
}

// Per-head [B, H, D] or per-token [B, H, S, D] bool/uint8 mask.
int mask_of(const rk_tensor* t, int64_t B, int64_t H, int64_t S, int64_t D, bool per_token, MaskView* m) {
  int st = rk::check_desc(t, per_token ? 4 : 3);
  if (st) return st;
  if (t->dtype != RK_U8) return RK_ERR_DTYPE;
  if (t->shape[0] != B || t->shape[1] != H) return RK_ERR_SHAPE;
  if (per_token ? (t->shape[2] != S || t->shape[3] != D) : t->shape[2] != D) return RK_ERR_SHAPE;
  m->data = (uint8_t*)t->data;
  m->sb = t->stride[0];
  m->sh = t->stride[1];
  m->ss = per_token ? t->stride[2] : 0;
  m->sc = per_token ? t->stride[3] : t->stride[2];
  return RK_OK;
}

bool same_bhs(const rk_tensor* t, int64_t B, int64_t H, int64_t S) {
  return t->shape[0] == B && t->shape[1] == H && t->shape[2] == S;
}

// 16-byte row loads: unit channel stride, 8-element aligned rows and base.
bool rows16(const rk_tensor* t) { return rk::vec_ok(t); }

// 4-byte row stores / loads of channel pairs: unit channel stride, even row
// strides, 4-byte aligned base.
bool pairs4(const rk_tensor* t) {
  if (t->stride[3] != 1) return false;
  for (int i = 0; i < 3; ++i)
    if (t->shape[i] > 1 && (t->stride[i] & 1)) return false;
  return (((uintptr_t)t->data) & 3) == 0;
}

// Token split: about `per_cu` workgroups per CU over all heads, at least
// `min_tokens` tokens per workgroup.
int token_splits(int64_t bh, int64_t S, int cus, int per_cu, int64_t min_tokens) {
  if (S <= 0 || bh <= 0) return 1;
  int64_t want = cdiv((int64_t)per_cu * cus, bh);
  const int64_t cap = cdiv(S, min_tokens);
  if (want > cap) want = cap;
  if (want < 1) want = 1;
  if (want > 65535) want = 65535;
  return (int)want;
}

int resolve_cus(int32_t num_cus, int* st) {
  *st = RK_OK;
  if (num_cus > 0) return num_cus;
  int dev = 0;
  const int cus = rk::current_device_cus(&dev);
  if (cus <= 0) *st = RK_ERR_NO_DEVICE;
  return cus;
}

struct ThinkPlan {
  int splits;
  int64_t chunk;
  size_t off_part, off_idx, total;
};

ThinkPlan think_plan(int64_t bh, int64_t S, int cus) {
  ThinkPlan p;
  p.splits = token_splits(bh, S, cus, 2, 256);
  p.chunk = cdiv(cdiv(S > 0 ? S : 1, p.splits), kTile) * kTile;
  p.splits = (int)cdiv(S > 0 ? S : 1, p.chunk);
  p.off_part = 0;
  p.off_idx = align256((size_t)bh * p.splits * kD * sizeof(float));
  p.total = p.off_idx + align256((size_t)bh * kD * sizeof(int32_t));
  return p;
}

// Shapes of ThinK's inputs and outputs; sets the views and B, H, keep.
int think_check(const rk_tensor* keys, const rk_tensor* queries, int64_t num_kv_heads, int64_t prune_count,
                const rk_tensor* kc_out, const rk_tensor* mask_out, View* kv, View* qv, MaskView* mv,
                int64_t* keep) {
  if (!keys || !queries || !kc_out || !mask_out) return RK_ERR_NULL;
  int st;
  if ((st = view_of(keys, 0, kv)) || (st = view_of(queries, 0, qv))) return st;
  if (queries->dtype != keys->dtype) return RK_ERR_DTYPE;
  const int64_t B = keys->shape[0], H = keys->shape[1], D = keys->shape[3];
  if (queries->shape[0] != B || queries->shape[3] != D) return RK_ERR_SHAPE;
  if (num_kv_heads != H || H < 1 || queries->shape[1] % H != 0) return RK_ERR_HEADS;
  if (prune_count < 0 || prune_count > D) return RK_ERR_KEEP_DIM;
  *keep = D - prune_count;
  if ((st = rk::check_desc(kc_out, 4))) return st;
  if (kc_out->dtype != keys->dtype) return RK_ERR_DTYPE;
  if (!same_bhs(kc_out, B, H, keys->shape[2]) || kc_out->shape[3] != *keep) return RK_ERR_SHAPE;
  if ((st = mask_of(mask_out, B, H, 0, D, false, mv))) return st;
  return RK_OK;
}

template <class TT>
hipError_t launch_think(const View& kv, bool kvec, const View& qv, int G, int keep, const ThinkPlan& p, int64_t B,
                        float f_keys, float f_win, float f_grp, const MaskView& mv, const rk_tensor* kc_out,
                        void* ws, hipStream_t s) {
  const int64_t bh = B * kv.H;
  float* part = (float*)((char*)ws + p.off_part);
  int32_t* idx = (int32_t*)((char*)ws + p.off_idx);
  const dim3 grid((unsigned)p.splits, (unsigned)bh);
  if (kvec)
    hipLaunchKernelGGL((sqsum_kernel<TT, true>), grid, dim3(kThreads), 0, s, kv, p.chunk, p.splits, part);
  else
    hipLaunchKernelGGL((sqsum_kernel<TT, false>), grid, dim3(kThreads), 0, s, kv, p.chunk, p.splits, part);
  ThinkArgs a;
  a.part = part;
  a.splits = p.splits;
  a.q = qv;
  a.G = G;
  a.keep = keep;
  a.H = kv.H;
  a.f_keys = f_keys;
  a.f_win = f_win;
  a.f_grp = f_grp;
  a.mask = mv;
  a.idx = idx;
  a.D = kv.C;
  hipLaunchKernelGGL((think_select_kernel<TT>), dim3((unsigned)bh), dim3(kD), 0, s, a);
  if (keep > 0 && kv.S > 0) {
    const OutView o = out_of(kc_out);
    const bool ovec = rows16(kc_out) && keep % 8 == 0;
    if (kvec && ovec)
      hipLaunchKernelGGL((compact_kernel<true, true>), grid, dim3(kThreads), 0, s, kv, idx, keep, p.chunk, o);
    else if (kvec)
      hipLaunchKernelGGL((compact_kernel<true, false>), grid, dim3(kThreads), 0, s, kv, idx, keep, p.chunk, o);
    else if (ovec)
      hipLaunchKernelGGL((compact_kernel<false, true>), grid, dim3(kThreads), 0, s, kv, idx, keep, p.chunk, o);
    else
      hipLaunchKernelGGL((compact_kernel<false, false>), grid, dim3(kThreads), 0, s, kv, idx, keep, p.chunk, o);
  }
  return hipGetLastError();
}

struct SparkPlan {
  int splits;
  int64_t chunk;
  size_t total;
};

SparkPlan spark_plan(int64_t bh, int64_t S, int cus) {
  SparkPlan p;
  p.splits = token_splits(bh, S, cus, 8, 64);
  p.chunk = cdiv(cdiv(S > 0 ? S : 1, p.splits), 16) * 16;
  p.splits = (int)cdiv(S > 0 ? S : 1, p.chunk);
  p.total = align256((size_t)bh * kD * sizeof(float));
  return p;
}

int spark_check(const rk_tensor* keys, const rk_tensor* queries, int64_t num_kv_groups, int64_t prune_count,
                const rk_tensor* kc_out, const rk_tensor* mask_out, const rk_tensor* pm_out, View* kv, View* qv,
                MaskView* mv, int64_t* keep) {
  if (!keys || !queries || !kc_out || !mask_out || !pm_out) return RK_ERR_NULL;
  int st;
  if ((st = view_of(keys, 0, kv)) || (st = view_of(queries, 0, qv))) return st;
  if (queries->dtype != keys->dtype) return RK_ERR_DTYPE;
  const int64_t B = keys->shape[0], H = keys->shape[1], S = keys->shape[2], D = keys->shape[3];
  if (queries->shape[0] != B || queries->shape[3] != D) return RK_ERR_SHAPE;
  if (num_kv_groups < 1 || queries->shape[1] != H * num_kv_groups) return RK_ERR_HEADS;
  if (prune_count < 0 || prune_count > D) return RK_ERR_KEEP_DIM;
  *keep = D - prune_count;
  if ((st = rk::check_desc(kc_out, 4)) || (st = rk::check_desc(pm_out, 4))) return st;
  if (kc_out->dtype != keys->dtype || pm_out->dtype != keys->dtype) return RK_ERR_DTYPE;
  if (!same_bhs(kc_out, B, H, S) || kc_out->shape[3] != *keep) return RK_ERR_SHAPE;
  if (!same_bhs(pm_out, B, H, S) || pm_out->shape[3] != 1) return RK_ERR_SHAPE;
  if ((st = mask_of(mask_out, B, H, S, D, true, mv))) return st;
  return RK_OK;
}

template <class TT>
hipError_t launch_spark(const View& kv, bool kvec, bool mvec, const View& qv, int G, int keep, const SparkPlan& p,
                        int64_t B,
                        float f_grp, float f_pruned, const MaskView& mv, const rk_tensor* kc_out,
                        const rk_tensor* pm_out, void* ws, hipStream_t s) {
  const int64_t bh = B * kv.H;
  float* qn = (float*)ws;
  hipLaunchKernelGGL((spark_qnorm_kernel<TT>), dim3((unsigned)bh), dim3(kD), 0, s, qv, G, kv.H, f_grp, qn);
  if (kv.S == 0) return hipGetLastError();
  SparkArgs a;
  a.k = kv;
  a.qn = qn;
  a.keep = keep;
  a.chunk = p.chunk;
  a.f_pruned = f_pruned;
  a.kc = out_of(kc_out);
  a.mask = mv;
  a.pm = out_of(pm_out);
  const dim3 grid((unsigned)p.splits, (unsigned)bh);
  const bool cvec = keep % 8 == 0 && rows16(kc_out);
  if (kvec && mvec && cvec)
    hipLaunchKernelGGL((spark_kernel<TT, true, true, true>), grid, dim3(kThreads), 0, s, a);
  else if (kvec && mvec)
    hipLaunchKernelGGL((spark_kernel<TT, true, true, false>), grid, dim3(kThreads), 0, s, a);
  else
    hipLaunchKernelGGL((spark_kernel<TT, false, false, false>), grid, dim3(kThreads), 0, s, a);
  return hipGetLastError();
}

// Optional prompt / text spans of the recovery (head dim D): NULL -> an
// empty view.
int span_of(const rk_tensor* t, const rk_tensor* kc, int D, View* v) {
  if (!t) {
    *v = View{nullptr, 0, 0, 0, 0, 0, (int32_t)kc->shape[1], D};
    return RK_OK;
  }
  int st = view_of(t, D, v);
  if (st) return st;
  if (t->dtype != kc->dtype) return RK_ERR_DTYPE;
  if (t->shape[0] != kc->shape[0] || t->shape[1] != kc->shape[1]) return RK_ERR_SHAPE;
  return RK_OK;
}

int recover(bool spark, const rk_tensor* k_prompt, const rk_tensor* k_pruned, const rk_tensor* k_text,
            const rk_tensor* mask, const rk_tensor* pruned_mean, const rk_tensor* out, int32_t num_cus,
            void* stream, bool launch) {
  if (!k_pruned || !mask || !out || (spark && !pruned_mean)) return RK_ERR_NULL;
  RecoverArgs a;
  int st;
  if ((st = view_of(k_pruned, -1, &a.kc))) return st;
  const int64_t B = k_pruned->shape[0], H = k_pruned->shape[1], Sv = k_pruned->shape[2];
  // the head dim: the output rows' width
  if ((st = rk::check_desc(out, 4))) return st;
  const int64_t D = out->shape[3];
  if (D < 1 || D > 128) return RK_ERR_HEAD_DIM;
  if (a.kc.C > D) return RK_ERR_SHAPE;
  if ((st = span_of(k_prompt, k_pruned, (int)D, &a.pr)) || (st = span_of(k_text, k_pruned, (int)D, &a.tx))) return st;
  if ((st = mask_of(mask, B, H, Sv, D, spark, &a.mask))) return st;
  a.pm = nullptr;
  a.p_sb = a.p_sh = a.p_ss = 0;
  if (spark) {
    if ((st = rk::check_desc(pruned_mean, 4))) return st;
    if (pruned_mean->dtype != k_pruned->dtype) return RK_ERR_DTYPE;
    if (!same_bhs(pruned_mean, B, H, Sv) || pruned_mean->shape[3] != 1) return RK_ERR_SHAPE;
    a.pm = (const uint16_t*)pruned_mean->data;
    a.p_sb = pruned_mean->stride[0];
    a.p_sh = pruned_mean->stride[1];
    a.p_ss = pruned_mean->stride[2];
  }
  if (out->dtype != k_pruned->dtype) return RK_ERR_DTYPE;
  a.rows = a.pr.S + Sv + a.tx.S;
  if (!same_bhs(out, B, H, a.rows)) return RK_ERR_SHAPE;
  if (!launch) return RK_OK;
  if (B * H == 0 || a.rows == 0) return RK_OK;
  if (!out->data || (Sv > 0 && !mask->data) || (Sv > 0 && a.kc.C > 0 && !k_pruned->data) ||
      (spark && Sv > 0 && !pruned_mean->data) || (a.pr.S > 0 && !a.pr.data) || (a.tx.S > 0 && !a.tx.data) ||
      (!spark && !mask->data))
    return RK_ERR_NULL;
  const int cus = resolve_cus(num_cus, &st);
  if (st) return st;
  a.out = out_of(out);
  a.H = (int)H;
  a.D = (int)D;
  int splits = token_splits(B * H, a.rows, cus, 8, kTile);
  a.chunk = cdiv(cdiv(a.rows, splits), kTile) * kTile;
  splits = (int)cdiv(a.rows, a.chunk);
  const dim3 grid((unsigned)splits, (unsigned)(B * H));
  hipStream_t s = (hipStream_t)stream;
  // 16-byte rows everywhere (whole 8-channel groups), 8-byte mask rows (SparK)
  bool fast = D % 8 == 0 && rows16(out) && (!k_prompt || rows16(k_prompt)) && (!k_text || rows16(k_text)) &&
              a.kc.C % 8 == 0 && (a.kc.C == 0 || rows16(k_pruned));
  if (spark)
    fast = fast && mask->stride[3] == 1 && mask->stride[0] % 8 == 0 && mask->stride[1] % 8 == 0 &&
           mask->stride[2] % 8 == 0 && (((uintptr_t)mask->data) & 7) == 0;
  const bool full = D == kD;
  auto go = [&](auto kernel) { hipLaunchKernelGGL(kernel, grid, dim3(kThreads), 0, s, a); };
  if (spark) {
    if (fast)
      full ? go(recover_kernel<true, true, true>) : go(recover_kernel<true, true, false>);
    else
      full ? go(recover_kernel<true, false, true>) : go(recover_kernel<true, false, false>);
  } else {
    if (fast)
      full ? go(recover_kernel<false, true, true>) : go(recover_kernel<false, true, false>);
    else
      full ? go(recover_kernel<false, false, true>) : go(recover_kernel<false, false, false>);
  }
  return hipGetLastError() == hipSuccess ? RK_OK : RK_ERR_HIP;
}

}  // namespace

extern "C" int rk_think_score_and_compact_check(const rk_tensor* keys_vision, const rk_tensor* queries_recent,
                                                int64_t num_kv_heads, int64_t prune_count,
                                                const rk_tensor* k_compact_out, const rk_tensor* keep_mask_out,
                                                int32_t num_cus, size_t* workspace_bytes) {
  View kv, qv;
  MaskView mv;
  int64_t keep;
  int st = think_check(keys_vision, queries_recent, num_kv_heads, prune_count, k_compact_out, keep_mask_out, &kv,
                       &qv, &mv, &keep);
  if (st) return st;
  const int cus = resolve_cus(num_cus, &st);
  if (st) return st;
  if (workspace_bytes) *workspace_bytes = think_plan(keys_vision->shape[0] * kv.H, kv.S, cus).total;
  return RK_OK;
}

extern "C" int rk_think_score_and_compact(const rk_tensor* keys_vision, const rk_tensor* queries_recent,
                                          int64_t num_kv_heads, int64_t prune_count,
                                          const rk_tensor* k_compact_out, const rk_tensor* keep_mask_out,
                                          void* workspace, size_t workspace_bytes, void* stream) {
  View kv, qv;
  MaskView mv;
  int64_t keep;
  int st = think_check(keys_vision, queries_recent, num_kv_heads, prune_count, k_compact_out, keep_mask_out, &kv,
                       &qv, &mv, &keep);
  if (st) return st;
  const int64_t B = keys_vision->shape[0], H = kv.H, Hq = queries_recent->shape[1];
  const int cus = resolve_cus(0, &st);
  if (st) return st;
  const ThinkPlan p = think_plan(B * H, kv.S, cus);
  if (!workspace || (((uintptr_t)workspace) & 255) || workspace_bytes < p.total) return RK_ERR_WORKSPACE;
  if (B * H == 0) return RK_OK;
  if ((kv.S > 0 && !kv.data) || (qv.S > 0 && !qv.data) || !mv.data || (keep > 0 && kv.S > 0 && !k_compact_out->data))
    return RK_ERR_NULL;
  const int G = (int)(Hq / H);
  const int64_t D = kv.C;
  const float f_keys = mean_factor(B * H * D, B * H * kv.S * D);
  const float f_win = mean_factor(B * Hq * D, B * Hq * qv.S * D);
  const float f_grp = mean_factor(B * H * D, B * Hq * D);
  const bool kvec = rows16(keys_vision) && D % 8 == 0;
  hipStream_t s = (hipStream_t)stream;
  const hipError_t e = keys_vision->dtype == RK_F16
                           ? launch_think<rk::F16>(kv, kvec, qv, G, (int)keep, p, B, f_keys, f_win, f_grp, mv,
                                                   k_compact_out, workspace, s)
                           : launch_think<rk::BF16>(kv, kvec, qv, G, (int)keep, p, B, f_keys, f_win, f_grp, mv,
                                                    k_compact_out, workspace, s);
  return e == hipSuccess ? RK_OK : RK_ERR_HIP;
}

extern "C" int rk_spark_prune_check(const rk_tensor* keys_vision, const rk_tensor* queries, int64_t num_kv_groups,
                                    int64_t prune_count, const rk_tensor* k_compact_out,
                                    const rk_tensor* keep_mask_out, const rk_tensor* pruned_mean_out,
                                    int32_t num_cus, size_t* workspace_bytes) {
  View kv, qv;
  MaskView mv;
  int64_t keep;
  int st = spark_check(keys_vision, queries, num_kv_groups, prune_count, k_compact_out, keep_mask_out,
                       pruned_mean_out, &kv, &qv, &mv, &keep);
  if (st) return st;
  const int cus = resolve_cus(num_cus, &st);
  if (st) return st;
  if (workspace_bytes) *workspace_bytes = spark_plan(keys_vision->shape[0] * kv.H, kv.S, cus).total;
  return RK_OK;
}

extern "C" int rk_spark_prune(const rk_tensor* keys_vision, const rk_tensor* queries, int64_t num_kv_groups,
                              int64_t prune_count, const rk_tensor* k_compact_out, const rk_tensor* keep_mask_out,
                              const rk_tensor* pruned_mean_out, void* workspace, size_t workspace_bytes,
                              void* stream) {
  View kv, qv;
  MaskView mv;
  int64_t keep;
  int st = spark_check(keys_vision, queries, num_kv_groups, prune_count, k_compact_out, keep_mask_out,
                       pruned_mean_out, &kv, &qv, &mv, &keep);
  if (st) return st;
  const int64_t B = keys_vision->shape[0], H = kv.H;
  const int cus = resolve_cus(0, &st);
  if (st) return st;
  const SparkPlan p = spark_plan(B * H, kv.S, cus);
  if (!workspace || (((uintptr_t)workspace) & 255) || workspace_bytes < p.total) return RK_ERR_WORKSPACE;
  if (B * H == 0) return RK_OK;
  if ((kv.S > 0 && (!kv.data || !mv.data || !pruned_mean_out->data || (keep > 0 && !k_compact_out->data))) ||
      (qv.S > 0 && !qv.data))
    return RK_ERR_NULL;
  const int64_t W = qv.S, D = kv.C;
  const float f_grp = mean_factor(B * H * W * D, B * H * num_kv_groups * W * D);
  const float f_pruned = mean_factor(B * H * kv.S, B * H * kv.S * prune_count);
  const bool kvec = rows16(keys_vision) && D % 8 == 0;
  const bool mvec = D % 8 == 0 && keep_mask_out->stride[3] == 1 && keep_mask_out->stride[0] % 8 == 0 &&
                    keep_mask_out->stride[1] % 8 == 0 && keep_mask_out->stride[2] % 8 == 0 &&
                    (((uintptr_t)keep_mask_out->data) & 7) == 0;
  hipStream_t s = (hipStream_t)stream;
  const hipError_t e =
      keys_vision->dtype == RK_F16
          ? launch_spark<rk::F16>(kv, kvec, mvec, qv, (int)num_kv_groups, (int)keep, p, B, f_grp, f_pruned, mv,
                                  k_compact_out, pruned_mean_out, workspace, s)
          : launch_spark<rk::BF16>(kv, kvec, mvec, qv, (int)num_kv_groups, (int)keep, p, B, f_grp, f_pruned, mv,
                                   k_compact_out, pruned_mean_out, workspace, s);
  return e == hipSuccess ? RK_OK : RK_ERR_HIP;
}

extern "C" int rk_think_recover_check(const rk_tensor* k_prompt, const rk_tensor* k_pruned,
                                      const rk_tensor* k_text, const rk_tensor* think_mask,
                                      const rk_tensor* out) {
  return recover(false, k_prompt, k_pruned, k_text, think_mask, nullptr, out, 1, nullptr, false);
}

extern "C" int rk_think_recover(const rk_tensor* k_prompt, const rk_tensor* k_pruned, const rk_tensor* k_text,
                                const rk_tensor* think_mask, const rk_tensor* out, void* stream) {
  return recover(false, k_prompt, k_pruned, k_text, think_mask, nullptr, out, 0, stream, true);
}

extern "C" int rk_spark_recover_check(const rk_tensor* k_prompt, const rk_tensor* k_pruned,
                                      const rk_tensor* k_text, const rk_tensor* spark_mask,
                                      const rk_tensor* pruned_mean, const rk_tensor* out) {
  return recover(true, k_prompt, k_pruned, k_text, spark_mask, pruned_mean, out, 1, nullptr, false);
}

extern "C" int rk_spark_recover(const rk_tensor* k_prompt, const rk_tensor* k_pruned, const rk_tensor* k_text,
                                const rk_tensor* spark_mask, const rk_tensor* pruned_mean, const rk_tensor* out,
                                void* stream) {
  return recover(true, k_prompt, k_pruned, k_text, spark_mask, pruned_mean, out, 0, stream, true);
}

extern "C" int rk_channel_selection(const rk_tensor* keep_mask, const rk_tensor* R_out, void* stream) {
  if (!keep_mask || !R_out) return RK_ERR_NULL;
  int st = rk::check_desc(R_out, 4);
  if (st) return st;
  if (!rk::is_float_param(R_out->dtype)) return RK_ERR_DTYPE;
  const int64_t B = R_out->shape[0], H = R_out->shape[1], D = R_out->shape[2], Dk = R_out->shape[3];
  if (D < 1 || D > 128) return RK_ERR_HEAD_DIM;
  if (Dk < 1 || Dk > D) return RK_ERR_KEEP_DIM;
  if (H > (INT64_C(1) << 30) || B * H > (INT64_C(1) << 30)) return RK_ERR_SHAPE;
  MaskView m;
  if ((st = mask_of(keep_mask, B, H, 0, D, false, &m))) return st;
  if (B * H == 0) return RK_OK;
  if (!m.data || !R_out->data) return RK_ERR_NULL;
  hipStream_t s = (hipStream_t)stream;
  const dim3 grid((unsigned)(B * H));
  const int64_t* rs = R_out->stride;
  if (R_out->dtype == RK_F32) {
    hipLaunchKernelGGL((selection_kernel<float>), grid, dim3(kD), 0, s, m, (int)H, (int)D, (int)Dk,
                       (float*)R_out->data, rs[0], rs[1], rs[2], rs[3], 1.0f);
  } else {
    const uint16_t one = R_out->dtype == RK_F16 ? (uint16_t)0x3C00 : (uint16_t)0x3F80;
    hipLaunchKernelGGL((selection_kernel<uint16_t>), grid, dim3(kD), 0, s, m, (int)H, (int)D, (int)Dk,
                       (uint16_t*)R_out->data, rs[0], rs[1], rs[2], rs[3], one);
  }
  return hipGetLastError() == hipSuccess ? RK_OK : RK_ERR_HIP;
}
