// rk_decode.hip -- fused split-K RotateK decode for MI355X (gfx950).
//
// One launch computes a whole decode step (fused_decode.py:303-420,
// gqa_decode.py:280-321, and the dense baseline of
// full_channel_flash_decoding.py:162-229 when the visual span is empty),
// over a grid of work units x workgroups per unit:
//
//   work units = (b, kv head, block of <= 16 query heads) under the GQA
//                policy, (b, query head) under the paper policy;
//   workgroups = wg_vis chunks of the rotated visual span followed by
//                wg_full chunks of the full-width prompt+text span;
//
// unit-major (grid (np, units)), or chunk-major (grid (units, np)) for one
// round of short workgroups (rk_plan_decode).
//
// A workgroup is 4 independent waves that walk interleaved 32-token blocks
// of its chunk.  Each wave keeps a ring of NBUF blocks of K/V in registers:
// the loads of block i + NBUF are issued before block i is computed, so a
// wave always has NBUF-1..NBUF blocks (10-16 KB) in flight.  Loads are
// unconditional 16-byte loads at 32-bit offsets from wave-uniform head
// bases, with rows clamped into the chunk (clamped rows get probability 0).
// Rows read whole by one 16-lane group (V, compact visual K) are loaded
// non-temporally; full-width K rows, split over four groups, are not.
// Per block a wave
//   * scores 16 query heads x 32 tokens with v_mfma_f32_16x16x32 (the visual
//     path feeds q R as an fp16/bf16 hi+lo pair so the score keeps ~fp32
//     precision; the full path feeds q exactly),
//   * runs the online softmax in the log2 domain (q . delta_mu bias and
//     1/sqrt(D) folded into one fused multiply-add per score; the
//     accumulator is rescaled only when some head's running max moved),
//   * accumulates O^T += V^T P^T on the MFMA with P split hi+lo, V^T built
//     by an in-register 8x8 transpose of eight 16-byte row loads.
// Prompt/text validity (chunk range and mask_full) is staged once per
// workgroup as bytes in LDS.  The four wave states are merged through LDS
// into one partial record (m, l, acc) per workgroup and head; the unit's
// records are merged into acc / (l + 1e-6) in the output dtype either by a
// second, small launch (merge_kernel) or, for one round of one-head units,
// by the unit's last workgroup behind a counter (merge_fused).  There the
// records are written through to memory and read with coherent loads and
// the counters are device-scope atomics, with no agent-scope
// release/acquire (which on gfx950 writes back and invalidates the whole
// XCD L2, 2.5x slower at B=32, 16k context); every call leaves the
// counters at zero, so either form is graph-capturable as is.
#include <math.h>
#include <stdlib.h>
#include <string.h>

#include <atomic>
#include <mutex>

#include "rk_common.h"
#include "rotatek_hip.h"

namespace rk {

struct DecodeArgs {
  const uint16_t* q;
  const void* R;
  const void* dm;
  const uint16_t* kf;
  const uint16_t* vf;
  const uint8_t* mask;
  int32_t* len_full;  // optional per-batch valid prompt/text length (device)
  // Prompt/text V rows at or past vf_gap_at live vf_gap rows further on (the
  // visual span sits between them in the span cache); UINT32_MAX = no gap.
  uint32_t vf_gap_at, vf_gap;
  // Fused append (span cache): the token k_new / v_new [B, H_kv, 128] joins
  // at row pos[b] = len_full[b].  Workgroup 0 of each unit folds it into
  // its partial and the first unit of the KV head writes it to kf_w / vf_w;
  // the merge launch advances len_full (nothing else reads it there).
  const uint16_t* k_new;
  const uint16_t* v_new;
  uint16_t* kf_w;
  uint16_t* vf_w;
  int64_t kn_sb, kn_sh, kn_sd, vn_sb, vn_sh, vn_sd;
  const uint16_t* ks;
  const uint16_t* vs;
  uint16_t* out;
  // split partials: one record of kRecFloats per (unit, workgroup, head),
  // acc[0..127], then m, l (each record on cache lines of its own)
  float* part;
  // single-launch merge: per-unit arrival tickets and, with a fused append,
  // per-batch-row unit tickets; both zero between calls
  uint32_t* ticket;
  uint32_t* bticket;
  int32_t fused;
  int64_t q_sb, q_sh, q_sd;
  int64_t R_sb, R_sh, R_sd, R_sk;
  int64_t dm_sb, dm_sh, dm_sd;
  int64_t kf_sb, kf_sh;
  int64_t vf_sb, vf_sh;
  int64_t mf_sb, mf_ss;
  int64_t ks_sb, ks_sh;
  int64_t vs_sb, vs_sh;
  int64_t o_sb, o_sh, o_sd;
  int64_t S_v, S_f, chunk_vis, chunk_full;
  // within-head strides (elements); a head's span is < 2^31 elements
  uint32_t kf_ss, kf_sd, vf_ss, vf_sd, ks_ss, ks_sd, vs_ss, vs_sd;
  int32_t G, Dk, hpu, spk, units_per_b, wg_vis, np, rot_x;
  // cmajor: the grid is (units, np), so workgroup ids run chunk-major
  // (x * units + u) and visual chunks x < nfast hold chunk_fast tokens (the
  // others chunk_vis; see rk_plan_decode)
  int32_t cmajor, nfast;
  int64_t chunk_fast;
  // xgroup > 1 (one unit per query head, G query heads per KV head): the
  // units of a KV head that read the same chunk run in consecutive slots of
  // one XCD (see decode_kernel); units = B * H_q
  int32_t xgroup, units;
  int32_t r_dtype, dm_dtype, has_bias, has_mask;
  // prologue layouts: q rows contiguous and 16-byte aligned (one 16-byte load
  // per thread); R a contiguous, 16-byte aligned [128][Dk] 16-bit block
  // with Dk <= 64, or up to 128 in the compute type (staged through LDS
  // with 16-byte loads)
  int32_t q_vec, r_vec;
  int32_t qr_mfma;  // q R on the MFMA also for rows of <= 32 kept channels
  float scale_log2;
};

constexpr int kThreads = 256;
constexpr int kWaves = 4;
constexpr int kBlk = 32;
constexpr int kMaskChunk = 4096;  // max prompt+text tokens per workgroup
constexpr int kRecFloats = 160;   // partial record: acc[128], m, l; 640 B = five 128-byte lines

// Eight 16-bit elements of one row: channels chan..chan+7 (element index,
// not yet scaled by the channel stride) at element offset `row_off` from a
// wave-uniform head base.  VEC: one 16-byte load at a 32-bit byte offset
// (unit channel stride, 16-byte aligned rows).  Otherwise element loads of
// the first `nvalid` channels only, zeros for the rest.
//
// NT: non-temporal load (the "nt" bit), for rows that are streamed once and
// read whole by one instruction (every V row; compact visual K rows of up to
// 32 channels), so they do not displace reused lines in L2 / MALL: +5 % at
// config 2, +10 % at config 3.  Full 128-channel K rows are read in 64-byte
// quarters by four instructions; NT there makes the second half of each
// 128-byte line miss again (the dense sweep slowed by 14 %), so those loads
// are ordinary.
template <bool VEC, bool NT = true>
__device__ __forceinline__ uint4 load_row8(const uint16_t* base, uint32_t row_off, uint32_t chan,
                                           uint32_t sd, int nvalid) {
  if constexpr (VEC) {
    const uint32_t boff = (row_off + chan) * 2u;
    if constexpr (NT) {
      const u32x4 v = __builtin_nontemporal_load((const u32x4*)((const char*)base + boff));
      return make_uint4(v.x, v.y, v.z, v.w);
    } else {
      return *(const uint4*)((const char*)base + boff);
    }
  } else {
    uint32_t w[4] = {0, 0, 0, 0};
#pragma unroll
    for (int e = 0; e < 8; ++e)
      if (e < nvalid) w[e >> 1] |= (uint32_t)base[row_off + (chan + e) * sd] << ((e & 1) * 16);
    return make_uint4(w[0], w[1], w[2], w[3]);
  }
}

// load_row8 with the row given as a byte offset `row_b` (a multiple of 2):
// VEC, one 16-byte load at row_b + 2 chan; otherwise element loads of
// channels chan.. at stride sd from element row_b / 2.
template <bool VEC, bool NT = true>
__device__ __forceinline__ uint4 load_row8b(const uint16_t* base, uint32_t row_b, uint32_t chan, uint32_t sd,
                                            int nvalid) {
  if constexpr (VEC) {
    const uint32_t boff = row_b + 2u * chan;
    if constexpr (NT) {
      const u32x4 v = __builtin_nontemporal_load((const u32x4*)((const char*)base + boff));
      return make_uint4(v.x, v.y, v.z, v.w);
    } else {
      return *(const uint4*)((const char*)base + boff);
    }
  } else {
    return load_row8<false, NT>(base, row_b >> 1, chan, sd, nvalid);
  }
}

__device__ __forceinline__ uint4 zero_if(bool keep, uint4 v) {
  return keep ? v : make_uint4(0, 0, 0, 0);
}

__device__ __forceinline__ uint4 pack8(const uint16_t (&h)[8]) {
  return make_uint4(h[0] | ((uint32_t)h[1] << 16), h[2] | ((uint32_t)h[3] << 16),
                    h[4] | ((uint32_t)h[5] << 16), h[6] | ((uint32_t)h[7] << 16));
}

// Online-softmax update of one 32-token block for the lane's head n.
// s[r] = log2-domain score of token 8g + r (-inf when invalid); vr[r] = the
// lane's 16-byte slice (channels 8n..8n+7) of V row 8g + r.
template <class TT>
__device__ __forceinline__ void softmax_pv(const float (&s)[8], const uint4 (&vr)[8], float& m,
                                           float& l, f32x4 (&acc)[8]) {
  float mx = s[0];
#pragma unroll
  for (int r = 1; r < 8; ++r) mx = fmaxf(mx, s[r]);
  mx = fmaxf(mx, shfl_xor(mx, 16));
  mx = fmaxf(mx, shfl_xor(mx, 32));
  const float m_new = fmaxf(m, mx);
  const float alpha = fast_exp2(m - m_new);
  if (__any(m_new != m)) {
#pragma unroll
    for (int j = 0; j < 8; ++j) acc[j] *= alpha;
  }
  m = m_new;
  float p[8], ps = 0.f;
#pragma unroll
  for (int r = 0; r < 8; ++r) {
    p[r] = fast_exp2(s[r] - m_new);
    ps += p[r];
  }
  l = l * alpha + ps;
  // P^T operand: tokens 8g..8g+7 of head n, hi + lo parts
  uint4 ph, pl;
  TT::split8(p, ph, pl);
  // V^T operand for channel slot j: element r = V[8g + r][8n + j]
  uint4 av[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const int wi = j >> 1;
    if (j & 1) {
      av[j].x = pack_hi(word(vr[0], wi), word(vr[1], wi));
      av[j].y = pack_hi(word(vr[2], wi), word(vr[3], wi));
      av[j].z = pack_hi(word(vr[4], wi), word(vr[5], wi));
      av[j].w = pack_hi(word(vr[6], wi), word(vr[7], wi));
    } else {
      av[j].x = pack_lo(word(vr[0], wi), word(vr[1], wi));
      av[j].y = pack_lo(word(vr[2], wi), word(vr[3], wi));
      av[j].z = pack_lo(word(vr[4], wi), word(vr[5], wi));
      av[j].w = pack_lo(word(vr[6], wi), word(vr[7], wi));
    }
  }
#pragma unroll
  for (int j = 0; j < 8; ++j) acc[j] = TT::mfma(av[j], ph, acc[j]);
#pragma unroll
  for (int j = 0; j < 8; ++j) acc[j] = TT::mfma(av[j], pl, acc[j]);
}

// Register ring over this wave's blocks wave, wave+4, ... < nblk, visited
// in a rotated order (workgroups start at different points of their chunks,
// so the many chunks that begin at the same offset inside equally strided
// heads do not all hit the same memory channels at once).  prime() issues
// the first NBUF blocks; run() consumes block j and then loads block
// j + NBUF into the freed slot, so NBUF-1..NBUF blocks are always in
// flight.  Loads past the wave's last block stay unconditional (a load
// under a branch costs the ring its overlap: 862 -> 1239 us at B=32/16k)
// but name the block just past the chunk, whose rows all clamp to the
// chunk's last row: one K row and one V row per load instead of a whole
// block, which non-temporal loads would fetch from HBM again.  The loop has
// no exits other than its trip count; the last nw % NBUF blocks are
// consumed after it.
template <int NBUF, class Buf>
struct Ring {
  Buf buf[NBUF];
  int64_t nw, rot;
  int wave;

  __device__ __forceinline__ Ring(int64_t nblk, int wave_, uint32_t seed) : wave(wave_) {
    nw = wave_ < nblk ? (nblk - 1 - wave_) / kWaves + 1 : 0;
    rot = (int64_t)__umulhi(seed, (uint32_t)nw);  // floor(seed * nw / 2^32) < nw
  }
  __device__ __forceinline__ int64_t blk_of(int64_t j) const {
    int64_t r = j + rot;
    r = r >= nw ? r - nw : r;
    // j >= nw: block wave + 4 nw >= nblk, past the chunk (rows clamp)
    return (int64_t)wave + (int64_t)kWaves * (j < nw ? r : nw);
  }
  template <class Load>
  __device__ __forceinline__ void prime(const Load& load) {
    if (nw == 0) return;
#pragma unroll
    for (int i = 0; i < NBUF; ++i) load(buf[i], blk_of(i));
  }
  template <class Load, class Compute>
  __device__ __forceinline__ void run(const Load& load, const Compute& compute) {
    if (nw == 0) return;
    int64_t j = 0;
    for (; j + NBUF <= nw; j += NBUF) {
#pragma unroll
      for (int i = 0; i < NBUF; ++i) {
        compute(buf[i], blk_of(j + i));
        load(buf[i], blk_of(j + i + NBUF));
      }
    }
#pragma unroll
    for (int i = 0; i < NBUF - 1; ++i)
      if (j + i < nw) compute(buf[i], blk_of(j + i));
  }
};

template <int DKB>
struct VisBuf {
  uint4 k[2][DKB];
  uint4 v[8];
};

struct FullBuf {
  uint4 k[2][4];
  uint4 v[8];
};

// ---- partial records and their merge
//   out = sum_p acc_p 2^(m_p - M) / (sum_p l_p 2^(m_p - M) + 1e-6),
//   M = max_p m_p                                  (fused_decode.py:275-296)
// Record (u, x, h) of a unit's workgroup x and head h sits at
// part + ((u * np + x) * hpu + h) * kRecFloats.

// Channels 8 c8 .. 8 c8 + 7 of a record's acc, and its (m, l).  COH: relaxed
// agent-scope atomic loads, which the single-launch merge uses to read
// records written by workgroups on other XCDs in the same launch (each XCD
// has its own L2; these loads are coherent across them).
template <bool COH>
__device__ __forceinline__ void load_rec(const float* rec, int c8, float (&v)[8], float& m, float& l) {
  if constexpr (COH) {
    const uint64_t* p = (const uint64_t*)(rec + 8 * c8);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const uint64_t w = __hip_atomic_load(p + i, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      v[2 * i] = __builtin_bit_cast(float, (uint32_t)w);
      v[2 * i + 1] = __builtin_bit_cast(float, (uint32_t)(w >> 32));
    }
    const uint64_t w = __hip_atomic_load((const uint64_t*)(rec + 128), __ATOMIC_RELAXED,
                                         __HIP_MEMORY_SCOPE_AGENT);
    m = __builtin_bit_cast(float, (uint32_t)w);
    l = __builtin_bit_cast(float, (uint32_t)(w >> 32));
  } else {
    const float4 s0 = ((const float4*)(rec + 8 * c8))[0], s1 = ((const float4*)(rec + 8 * c8))[1];
    const float2 ml = *(const float2*)(rec + 128);
    v[0] = s0.x; v[1] = s0.y; v[2] = s0.z; v[3] = s0.w;
    v[4] = s1.x; v[5] = s1.y; v[6] = s1.z; v[7] = s1.w;
    m = ml.x;
    l = ml.y;
  }
}

// Store of a workgroup's record slice (the lane's eight acc channels; m, l
// by the c8 == 0 lane).  COH: relaxed agent-scope atomic stores, which
// write through to memory, so that after the storing thread's wait for
// their completion any XCD reads them.
template <bool COH>
__device__ __forceinline__ void store_rec(float* rec, int c8, const float (&A)[8], float M, float L) {
  if constexpr (COH) {
    uint64_t* p = (uint64_t*)(rec + 8 * c8);
#pragma unroll
    for (int i = 0; i < 4; ++i)
      __hip_atomic_store(p + i,
                         (uint64_t)__builtin_bit_cast(uint32_t, A[2 * i]) |
                             ((uint64_t)__builtin_bit_cast(uint32_t, A[2 * i + 1]) << 32),
                         __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if (c8 == 0)
      __hip_atomic_store((uint64_t*)(rec + 128),
                         (uint64_t)__builtin_bit_cast(uint32_t, M) |
                             ((uint64_t)__builtin_bit_cast(uint32_t, L) << 32),
                         __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  } else {
    float4* dst = (float4*)(rec + 8 * c8);
    dst[0] = make_float4(A[0], A[1], A[2], A[3]);
    dst[1] = make_float4(A[4], A[5], A[6], A[7]);
    if (c8 == 0) *(float2*)(rec + 128) = make_float2(M, L);
  }
}

// Folds the records x = p0, p0 + step, ... < np of one (unit, head) into
// (M, L, A) for channels 8 c8 .. 8 c8 + 7; `rec0` is the record of x = 0
// and `rstride` the floats between consecutive x.  NB records' loads are
// issued together; entries past np are clamped in-bounds loads with weight
// zero (a batch's first entry is always valid, so its max is finite).
template <bool COH, int NB = 8>
__device__ __forceinline__ void fold_records(const float* rec0, int64_t rstride, int np, int p0, int step,
                                             int c8, float& M, float& L, float (&A)[8]) {
  for (int p = p0; p < np; p += NB * step) {
    float mm[NB], ll[NB], vv[NB][8];
#pragma unroll
    for (int i = 0; i < NB; ++i) {
      const int q = p + step * i;
      const bool ok = q < np;
      load_rec<COH>(rec0 + (int64_t)(ok ? q : p) * rstride, c8, vv[i], mm[i], ll[i]);
      if (!ok) {
        mm[i] = -INFINITY;
        ll[i] = 0.f;
      }
    }
    float mx = M;
#pragma unroll
    for (int i = 0; i < NB; ++i) mx = fmaxf(mx, mm[i]);
    const float sc = fast_exp2(M - mx);
    L *= sc;
#pragma unroll
    for (int e = 0; e < 8; ++e) A[e] *= sc;
#pragma unroll
    for (int i = 0; i < NB; ++i) {
      const float w = fast_exp2(mm[i] - mx);
      L += ll[i] * w;
#pragma unroll
      for (int e = 0; e < 8; ++e) A[e] += vv[i][e] * w;
    }
    M = mx;
  }
}

// (M, L, A) += (Mo, Lo, Ao) rescaled to the common max (either side may be
// empty, M = -inf).
__device__ __forceinline__ void combine(float& M, float& L, float (&A)[8], float Mo, float Lo,
                                        const float (&Ao)[8]) {
  const float Mx = fmaxf(M, Mo);
  const float ws = M == -INFINITY ? 0.f : fast_exp2(M - Mx);
  const float wo = Mo == -INFINITY ? 0.f : fast_exp2(Mo - Mx);
  L = L * ws + Lo * wo;
#pragma unroll
  for (int e = 0; e < 8; ++e) A[e] = A[e] * ws + Ao[e] * wo;
  M = Mx;
}

// acc / (l + 1e-6) in the output dtype, channels 8 c8 .. 8 c8 + 7 of (b, hq).
template <class TT>
__device__ __forceinline__ void write_out(const DecodeArgs& a, int b, int hq, int c8, float L,
                                          const float (&A)[8]) {
  const float den = L + kDenomEps;
  if constexpr (TT::kBytes == 4) {
    float* dst = (float*)a.out + b * a.o_sb + (int64_t)hq * a.o_sh + 8 * c8 * a.o_sd;
    if (a.o_sd == 1 && (((uintptr_t)dst) & 15) == 0) {
      ((float4*)dst)[0] = make_float4(A[0] / den, A[1] / den, A[2] / den, A[3] / den);
      ((float4*)dst)[1] = make_float4(A[4] / den, A[5] / den, A[6] / den, A[7] / den);
    } else {
#pragma unroll
      for (int e = 0; e < 8; ++e) dst[e * a.o_sd] = A[e] / den;
    }
  } else {
    uint16_t o[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) o[e] = TT::from_f32(A[e] / den);
    uint16_t* dst = a.out + b * a.o_sb + (int64_t)hq * a.o_sh + 8 * c8 * a.o_sd;
    if (a.o_sd == 1 && (((uintptr_t)dst) & 15) == 0) {
      *(uint4*)dst = pack8(o);
    } else {
#pragma unroll
      for (int e = 0; e < 8; ++e) dst[e * a.o_sd] = o[e];
    }
  }
}

// Merge of one unit's records by one 256-thread workgroup (both merges run
// this, so their results are bit-identical).  The 16 slices of 16 lanes
// (s = tid >> 4) are shared out S = 16 / nh (a power of two) per head;
// slice j of head h folds records x = j, j + S, ... (eight records' loads
// in flight at a time, so one or two memory round trips cover a unit), and
// the S slices of a head are combined pairwise, lower slice first: within a
// wave by lane exchange, across waves through LDS (s_mrg, 16 x kRecFloats
// floats).  COH: the records were written in this launch (coherent loads).
template <class TT, bool COH>
__device__ __forceinline__ void merge_unit(const DecodeArgs& a, int64_t u, int b, int h0, int nh, int tid,
                                           float* s_mrg) {
  int S = 16;
  while (S * nh > 16) S >>= 1;
  const int s = tid >> 4, c8 = tid & 15, h = s / S, j = s - (s / S) * S;
  const bool act = h < nh;
  float M = -INFINITY, L = 0.f, A[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
  if (act) {
    const float* rec0 = a.part + (u * a.np * a.hpu + h) * kRecFloats;
    fold_records<COH>(rec0, (int64_t)a.hpu * kRecFloats, a.np, j, S, c8, M, L, A);
  }
#pragma unroll
  for (int d = 1; d <= 2; d <<= 1) {  // lane exchange: slices s ^ 1, s ^ 2 share a wave
    if (d < S) {
      float Ao[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) Ao[e] = shfl_xor(A[e], 16 * d);
      const float Mo = shfl_xor(M, 16 * d), Lo = shfl_xor(L, 16 * d);
      if ((j & d) == 0) combine(M, L, A, Mo, Lo, Ao);
    }
  }
  for (int d = 4; d < S; d <<= 1) {  // across waves (S = 8, 16: one or two heads)
    float* mine = s_mrg + s * kRecFloats;
    if (act && (j & (2 * d - 1)) == d) {
#pragma unroll
      for (int e = 0; e < 8; ++e) mine[8 * c8 + e] = A[e];
      if (c8 == 0) {
        mine[128] = M;
        mine[129] = L;
      }
    }
    __syncthreads();
    if (act && (j & (2 * d - 1)) == 0) {
      const float* o = s_mrg + (s + d) * kRecFloats;
      float Ao[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) Ao[e] = o[8 * c8 + e];
      combine(M, L, A, o[128], o[129], Ao);
    }
    __syncthreads();
  }
  if (act && j == 0) write_out<TT>(a, b, h0 + h, c8, L, A);
}

// Merge of one unit of one query head (hpu == 1) by the 16 lanes of one
// slice: the records x = 0 .. np - 1 in order, eight loads in flight, no
// cross-slice combine.  Both merges run this for such units (bit-identical
// results); the merge kernel gives each slice of a workgroup its own unit.
template <class TT, bool COH>
__device__ __forceinline__ void merge_slice(const DecodeArgs& a, int64_t u, int b, int hq, int c8) {
  float M = -INFINITY, L = 0.f, A[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
  fold_records<COH>(a.part + u * a.np * kRecFloats, kRecFloats, a.np, 0, 1, c8, M, L, A);
  write_out<TT>(a, b, hq, c8, L, A);
}

// Single-launch merge, run by every workgroup after it has stored its
// record.  The workgroup waits until its record stores have completed
// (they write through to memory), then takes a ticket on the unit's
// counter; the last of the unit's np workgroups resets the counter and
// merges the unit's records, read with coherent loads, in the order of
// the merge kernel (merge_unit; the result is bit-identical to the
// two-launch merge).  No
// agent-scope release or acquire fence is needed, so no XCD L2 is written
// back or invalidated.  With a fused append, the last unit of a batch row
// to finish advances len_full[b] behind a second ticket: by then every
// workgroup of the row has read it.  Both counters are left at zero.
template <class TT, bool APPEND>
__device__ __forceinline__ void merge_fused(const DecodeArgs& a, int u, int b, int h0, int nh, int tid,
                                            float* s_mrg) {
  __shared__ uint32_t s_ticket;
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
  __builtin_amdgcn_s_waitcnt(0);  // this thread's record stores have completed
  __syncthreads();                // ... and so have every thread's
  if (tid == 0)
    s_ticket = __hip_atomic_fetch_add(a.ticket + u, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  __syncthreads();
  if (s_ticket != (uint32_t)(a.np - 1)) return;
  if (tid == 0) __hip_atomic_store(a.ticket + u, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  if (a.hpu == 1) {
    if (tid < 16) merge_slice<TT, true>(a, u, b, h0, tid);
  } else {
    merge_unit<TT, true>(a, u, b, h0, nh, tid, s_mrg);
  }
  if constexpr (APPEND) {
    if (tid == 0) {
      const uint32_t t = __hip_atomic_fetch_add(a.bticket + b, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      if (t == (uint32_t)(a.units_per_b - 1)) {
        __hip_atomic_store(a.bticket + b, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        const int32_t pos = (int32_t)min(a.S_f, (int64_t)max(a.len_full[b], 0));
        if (pos < a.S_f) a.len_full[b] = pos + 1;
      }
    }
  }
}

// APPEND: fused append of k_new / v_new (span cache decode step); a
// separate instantiation so the plain decode carries none of its registers.
// NTL: V rows and compact visual Key rows use non-temporal loads (false for
// the grouped one-unit-per-query-head mode, whose G units of a KV head read
// each line through one XCD's L2).
template <class TT, int DKB, bool VEC, int HMAX, bool HAS_VIS, bool APPEND, bool NTL = true>
__global__ void __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(2)))
decode_kernel(const DecodeArgs a) {
  constexpr int DKP = DKB * 32;
  // visual blocks in flight per wave: three for multi-head units of <= 32
  // kept channels, else two (one-head units: measured faster on MI355X, eager
  // / graph us, config 1 34.1 / 33.2 -> 32.5 / 31.9, B=1 at 4000 tokens
  // 17.2 -> 16.2 graph, config 2 814.7 -> 811.4; multi-head units of 7 at
  // 12001 tokens 864 -> 888 us per config 4 step with two)
  constexpr int NBUF_V = DKB == 1 && HMAX > 1 ? 3 : 2;
  constexpr int NBUF_F = 2;
  __shared__ __attribute__((aligned(16))) float s_q[HMAX][128];
  __shared__ __attribute__((aligned(16))) float s_qt[HMAX][DKP];
  __shared__ float s_bias[HMAX];
  __shared__ float s_dm[128];
  __shared__ float s_m[kWaves][HMAX];
  __shared__ float s_l[kWaves][HMAX];
  __shared__ float s_acc[kWaves][HMAX][128];
  __shared__ __attribute__((aligned(16))) uint8_t s_valid[kMaskChunk];
  // raw R [128][Dk] (16 KB for Dk <= 64, 32 KB up to 128): in s_acc when
  // that is large enough (its upper half, the lower one holding the q R
  // partial sums; all of it for 65-128 channels, whose q R runs on the MFMA
  // with no partial sums), else its own
  constexpr int kRawChunks = DKB == 4 ? 2048 : 1024;
  __shared__ uint4 s_rsep[HMAX >= 16 ? 1 : kRawChunks];

  const int tid = threadIdx.x;
  // wave index in a scalar register: the ring's block bookkeeping (block
  // numbers, token offsets, bounds) then runs on the scalar unit, not as
  // per-lane 64-bit arithmetic
  const int lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6), g = lane >> 4, n = lane & 15;
  const int nq = n < HMAX ? n : 0;  // LDS row for this lane's head column
  // Workgroups go to the 8 XCDs round-robin by linear id: u * np + x, or
  // x * units + u in a chunk-major grid (rk_plan_decode); rot_x rotates
  // each unit's chunk numbers by the unit index (see run_decode).
  int u = a.cmajor ? (int)blockIdx.x : (int)blockIdx.y;
  int x = a.cmajor ? (int)blockIdx.y : (int)blockIdx.x + (a.rot_x ? u % a.np : 0);
  x = x >= a.np ? x - a.np : x;
  if (!NTL && a.xgroup > 1) {  // compiled into the grouped mode's instantiation only
    // Workgroup id i = y * np + x runs on XCD i mod 8 as the (i / 8)-th of
    // that XCD.  Each XCD takes a contiguous range of the work items
    // ((b, kv) major, then chunk, then the query head j of the group), so
    // the G units that read one K/V chunk are neighbours on one XCD and
    // share its L2 instead of each fetching the chunk from HBM.
    const int64_t N = (int64_t)a.units * a.np, bid = (int64_t)blockIdx.y * gridDim.x + blockIdx.x;
    const int64_t c = bid & 7, q8 = N >> 3, r8 = N & 7;
    const int64_t item = c * q8 + min(c, r8) + (bid >> 3);
    const int64_t grp = item / a.xgroup;  // (b, kv, chunk)
    const int j = (int)(item - grp * a.xgroup);
    const int64_t ukv = grp / a.np;
    x = (int)(grp - ukv * a.np);
    u = (int)(ukv * a.xgroup + j);
  }
  const int b = u / a.units_per_b;
  const int r_in_b = u - b * a.units_per_b;
  const int kv = r_in_b / a.spk;
  const int jblk = r_in_b - kv * a.spk;
  const int h0 = kv * a.G + jblk * a.hpu;
  const int nh = min(a.hpu, a.G - jblk * a.hpu);
  const bool is_vis = HAS_VIS && x < a.wg_vis;
  const int xf = HAS_VIS ? x - a.wg_vis : x;

  // Fused append: workgroup 0 of the unit stages the new token in LDS
  // behind the ring's prime and folds it into wave 0's state at the end.
  __shared__ float s_new[2][128];  // k_new, v_new of this unit's KV head
  const bool fold_new = APPEND && x == 0;
  int64_t pos_new = 0;
  if (fold_new) pos_new = min(a.S_f, (int64_t)max(a.len_full[b], 0));
  const bool has_new = fold_new && pos_new < a.S_f;  // a full buffer neither attends nor stores
  uint16_t new_raw = 0;
  auto load_new = [&]() {
    if (has_new) {
      const int c = tid & 127;
      new_raw = tid < 128 ? a.k_new[b * a.kn_sb + (int64_t)kv * a.kn_sh + (int64_t)c * a.kn_sd]
                          : a.v_new[b * a.vn_sb + (int64_t)kv * a.vn_sh + (int64_t)c * a.vn_sd];
    }
  };
  // after the staging barrier: the first unit of the KV head stores the row
  auto store_new = [&]() {
    if (has_new) {
      s_new[tid >> 7][tid & 127] = TT::to_f32(new_raw);
      if (jblk == 0) {
        const int64_t c = tid & 127;
        if (tid < 128) {
          a.kf_w[b * a.kf_sb + (int64_t)kv * a.kf_sh + pos_new * a.kf_ss + c * a.kf_sd] = new_raw;
        } else {
          const uint32_t row = (uint32_t)pos_new + ((uint32_t)pos_new >= a.vf_gap_at ? a.vf_gap : 0u);
          a.vf_w[b * a.vf_sb + (int64_t)kv * a.vf_sh + (int64_t)row * a.vf_ss + c * a.vf_sd] = new_raw;
        }
      }
    }
  };

  float m = kNegInit, l = 0.f;
  f32x4 acc[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) acc[j] = f32x4{0.f, 0.f, 0.f, 0.f};
  // A-operand token row of this lane inside a block, per score sub-block
  const uint32_t krow0 = 8 * (n >> 2) + (n & 3), krow1 = krow0 + 4;
  // the units of one KV head visit a chunk's blocks in the same order
  const uint32_t useed = !NTL && a.xgroup > 1 ? (uint32_t)(u / a.xgroup) : (uint32_t)u;
  const uint32_t rot_seed = (useed * 0x9E3779B1u) ^ ((uint32_t)x * 0x85EBCA77u);

  // Prologue order: the first NBUF K/V blocks are requested, then the
  // prologue's own loads (q rows; R / delta_mu or the mask bytes), and only
  // then does anything wait, so one memory latency covers them all.  Loads
  // are unconditional from clamped (in-bounds) addresses and masked after:
  // a load under a divergent branch compiles to its own wait.
  constexpr int kQPer = (HMAX * 128 + kThreads - 1) / kThreads;
  float qv[kQPer];
  // q rows, fast layout: thread t loads channels 8 (t & 15) .. + 7 of head
  // t >> 4 (clamped to a valid head) with one 16-byte load.
  uint16_t qraw[kQPer];
  uint4 q16 = make_uint4(0u, 0u, 0u, 0u);
  // load_q issues the fast-layout load before the first K/V blocks; the
  // element-wise fallback loads inside store_q, after them.
  auto load_q = [&]() {
    if (a.q_vec) {
      const int h = min(tid >> 4, nh - 1);
      q16 = *(const uint4*)(a.q + b * a.q_sb + (int64_t)(h0 + h) * a.q_sh + 8 * (tid & 15));
    }
  };
  auto store_q = [&]() {
    if (!a.q_vec) {
#pragma unroll
      for (int k = 0; k < kQPer; ++k) {
        const int i = tid + k * kThreads;
        const int h = min(i >> 7, nh - 1), d = i & 127;
        qraw[k] = a.q[b * a.q_sb + (int64_t)(h0 + h) * a.q_sh + d * a.q_sd];
      }
    }
    if (a.q_vec) {
      const int h = tid >> 4;
      if (h < HMAX) {
        float f[8];
#pragma unroll
        for (int e = 0; e < 8; ++e)
          f[e] = h < nh ? TT::to_f32((uint16_t)(word(q16, e >> 1) >> ((e & 1) * 16))) : 0.f;
        float4* dst = (float4*)&s_q[h][8 * (tid & 15)];
        dst[0] = make_float4(f[0], f[1], f[2], f[3]);
        dst[1] = make_float4(f[4], f[5], f[6], f[7]);
      }
    } else {
#pragma unroll
      for (int k = 0; k < kQPer; ++k) {
        const int i = tid + k * kThreads;
        qv[k] = (i < HMAX * 128 && (i >> 7) < nh) ? TT::to_f32(qraw[k]) : 0.f;
        if (i < HMAX * 128) s_q[i >> 7][i & 127] = qv[k];
      }
    }
  };

  if (is_vis) {
    // ---- visual span: rotated, truncated Keys (Dk channels)
    const int64_t t_begin = x < a.nfast ? (int64_t)x * a.chunk_fast
                                        : (int64_t)a.nfast * a.chunk_fast + (int64_t)(x - a.nfast) * a.chunk_vis;
    const int64_t t_end = min(a.S_v, t_begin + (x < a.nfast ? a.chunk_fast : a.chunk_vis));
    const uint32_t t_last = (uint32_t)(t_end - 1);
    const uint16_t* ksb = a.ks + b * a.ks_sb + kv * a.ks_sh;
    const uint16_t* vsb = a.vs + b * a.vs_sb + kv * a.vs_sh;
    bool kval[DKB];
    uint32_t kch[DKB];
    int knv[DKB];
#pragma unroll
    for (int kb = 0; kb < DKB; ++kb) {
      const int c0 = kb * 32 + 8 * g;
      kval[kb] = c0 < a.Dk;
      kch[kb] = kval[kb] ? (uint32_t)c0 : 0u;
      knv[kb] = kval[kb] ? min(a.Dk - c0, 8) : 0;
    }
    const uint32_t vch = 8u * n;
    const int64_t nblk = (t_end - t_begin + kBlk - 1) / kBlk;
    // Row addresses are byte offsets from the head base: a per-lane part (the
    // lane's row inside the block, and with 16-byte loads its channel slot)
    // plus the block's first token times the token stride (a scalar), clamped
    // to the chunk's last row, so a row costs two vector adds/mins and no
    // multiply.  Every sum stays below 2^32: the host bounds a head's span
    // plus 32 rows below 2^31 elements (set_head).
    constexpr bool kFoldK = VEC && DKB == 1;
    const uint32_t kss2 = 2u * a.ks_ss, vss2 = 2u * a.vs_ss;
    const uint32_t kfold = kFoldK ? 2u * kch[0] : 0u, vfold = VEC ? 2u * vch : 0u;
    const uint32_t kro0 = krow0 * kss2 + kfold, kro1 = krow1 * kss2 + kfold, klast = t_last * kss2 + kfold;
    const uint32_t vro = 8u * g * vss2 + vfold, vlast = t_last * vss2 + vfold;
    auto load = [&](VisBuf<DKB>& B, int64_t blk) {
      // blocks past the chunk start at (and clamp to) its last row
      const uint32_t t0 = min((uint32_t)(t_begin + blk * kBlk), t_last);
      const uint32_t kb0 = t0 * kss2, vb0 = t0 * vss2;
      const uint32_t r0 = min(kro0 + kb0, klast), r1 = min(kro1 + kb0, klast);
#pragma unroll
      for (int kb = 0; kb < DKB; ++kb) {
        const uint32_t ch = kFoldK ? 0u : kch[kb];
        B.k[0][kb] = load_row8b<VEC, NTL && DKB == 1>(ksb, r0, ch, a.ks_sd, knv[kb]);
        B.k[1][kb] = load_row8b<VEC, NTL && DKB == 1>(ksb, r1, ch, a.ks_sd, knv[kb]);
      }
#pragma unroll
      for (int r = 0; r < 8; ++r)
        B.v[r] = load_row8b<VEC, NTL>(vsb, min(vro + vb0 + (uint32_t)r * vss2, vlast), VEC ? 0u : vch, a.vs_sd, 8);
    };

    // q R: thread (c, part) loads R[part*L .. part*L+L-1][c], forms partial
    // dot products for every head, and the parts are summed in LDS.
    constexpr int kParts = kThreads / DKP, kL = 128 / kParts;
    const int c = tid % DKP, part = tid / DKP;
    // The first K/V blocks, then the prologue's own loads (q; R straight
    // into LDS in the fast layout; delta_mu) are issued back to back, so one
    // memory latency covers them all.
    uint4* s_r = HMAX >= 16 ? (uint4*)&s_acc[0][0][0] + (DKB == 4 ? 0 : kRawChunks) : s_rsep;
    constexpr int kRPer = kRawChunks / kThreads;
    const int nchunks = 16 * a.Dk;  // [128][Dk] 16-bit elements in 16-byte chunks
    Ring<NBUF_V, VisBuf<DKB>> ring(nblk, wave, rot_seed);
    ring.prime(load);
    load_q();
    load_new();
    if (a.r_vec) {
      // LDS DMA (global_load_lds_dwordx4): wave w copies 1 KB blocks
      // r * 4 + w of R straight into s_r, holding no registers across the
      // K/V prime; lanes past the end re-read the last chunk into unused slots
      const uint4* rsrc = (const uint4*)((const uint16_t*)a.R + b * a.R_sb + kv * a.R_sh);
#pragma unroll
      for (int r = 0; r < kRPer; ++r) {
        const int j0 = (r * kWaves + wave) * 64;
        if (j0 < nchunks)
          __builtin_amdgcn_global_load_lds(
              (__attribute__((address_space(1))) void*)(rsrc + min(j0 + lane, nchunks - 1)),
              (__attribute__((address_space(3))) void*)(s_r + j0), 16, 0, 0);
      }
    }
    uint32_t dmraw = 0u;
    if (a.has_bias) {
      const int64_t di = b * a.dm_sb + kv * a.dm_sh + (int64_t)(tid & 127) * a.dm_sd;
      dmraw = a.dm_dtype == 2 ? ((const uint32_t*)a.dm)[di] : (uint32_t)((const uint16_t*)a.dm)[di];
    }

    const float dmv = (tid < 128 && a.has_bias) ? raw_to_f32(dmraw, a.dm_dtype) : 0.f;
    store_q();
    store_new();
    if (tid < 128) s_dm[tid] = dmv;
    __syncthreads();
    // q . delta_mu: 16 lanes per head, eight channels each (needs only s_q
    // and s_dm, complete at the barrier above)
    auto q_dot_dm = [&]() {
      const int hb = tid >> 4, j = tid & 15, hs = min(hb, HMAX - 1);
      float bsum = 0.f;
#pragma unroll
      for (int e = 0; e < 8; ++e) bsum = fmaf(s_q[hs][8 * j + e], s_dm[8 * j + e], bsum);
#pragma unroll
      for (int off = 1; off < 16; off <<= 1) bsum += shfl_xor(bsum, off);
      if (hb < HMAX && j == 0) s_bias[hb] = bsum;
    };
    if ((DKB >= 2 || a.qr_mfma) && a.r_vec && a.r_dtype == TT::kRk) {
      // q R on the MFMA: wave w forms the 16-column tiles w, w + 4, .. of
      // q R (16 head rows x DKP columns) over the four 32-channel steps.
      // A = q (16-bit values, exact), B = R columns read from LDS (columns
      // past Dk zero); the products are exact and summed in fp32.  Taken
      // for 33-128 kept channels (config 4 at keep 64: 664 -> 618 us per
      // step at 4097 visual tokens, 1035 -> 990 at 12001); with one block of
      // 32 (only waves 0 and 1 busy) it measured 2-3 % slower at 12001
      // tokens, so those keep the FMA form below except in one-per-CU
      // plans (qr_mfma, set by the host).
      const uint16_t* rl = (const uint16_t*)s_r;
      const int dk1 = max(a.Dk - 1, 0);
      const bool hrow = n < HMAX;  // HMAX = 1: the other A rows are zero
      for (int t = wave; t < DKP / 16; t += kWaves) {  // uniform
        const int col = 16 * t + n;
        const uint16_t* rc = rl + min(col, dk1);
        f32x4 d = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int kk = 0; kk < 4; ++kk) {
          const int k0 = 32 * kk + 8 * g;
          uint16_t rb[8];
#pragma unroll
          for (int e = 0; e < 8; ++e) rb[e] = rc[(k0 + e) * a.Dk];
          const float4 f0 = *(const float4*)&s_q[nq][k0], f1 = *(const float4*)&s_q[nq][k0 + 4];
          const uint4 av = hrow ? make_uint4(TT::pack2(f0.x, f0.y), TT::pack2(f0.z, f0.w), TT::pack2(f1.x, f1.y),
                                             TT::pack2(f1.z, f1.w))
                                : make_uint4(0u, 0u, 0u, 0u);
          const uint4 bv = col < a.Dk ? pack8(rb) : make_uint4(0u, 0u, 0u, 0u);
          d = TT::mfma(av, bv, d);
        }
        // lane (g, n) holds rows 4g .. 4g + 3 of column 16t + n
#pragma unroll
        for (int i = 0; i < 4; ++i)
          if (4 * g + i < HMAX) s_qt[4 * g + i][col] = d[i];
      }
      q_dot_dm();
      __syncthreads();
    } else {  // q R by FMAs: partial sums over 8 (..2) channel slices, then summed
      float rv[kL];
      if (DKB < 4 && a.r_vec) {  // (65-128 channels stage R only for the MFMA form)
        // the thread's kL reads of column c issued back to back, then one
        // branch on R's (launch-uniform) 16-bit dtype; lanes past Dk read the
        // last column and are zeroed after (a per-element dtype and column
        // test put each read in its own branch, each waiting for its data)
        const uint16_t* rl = (const uint16_t*)s_r + min(c, max(a.Dk - 1, 0)) + part * kL * a.Dk;
        uint16_t raw[kL];
#pragma unroll
        for (int i = 0; i < kL; ++i) raw[i] = rl[i * a.Dk];
        if (a.r_dtype == RK_F16) {
#pragma unroll
          for (int i = 0; i < kL; ++i) rv[i] = F16::to_f32(raw[i]);
        } else {
#pragma unroll
          for (int i = 0; i < kL; ++i) rv[i] = BF16::to_f32(raw[i]);
        }
#pragma unroll
        for (int i = 0; i < kL; ++i) rv[i] = c < a.Dk ? rv[i] : 0.f;
      } else {  // element-wise fallback (column c, clamped in-bounds; no load
                // at all when Dk == 0, where R_partial has no storage)
#pragma unroll
        for (int i = 0; i < kL; ++i) rv[i] = 0.f;
        if (a.Dk > 0) {
          const int64_t rb = b * a.R_sb + kv * a.R_sh + (int64_t)min(c, a.Dk - 1) * a.R_sk;
          load_any_n(a.R, rb + (int64_t)(part * kL) * a.R_sd, a.R_sd, a.r_dtype, rv);
#pragma unroll
          for (int i = 0; i < kL; ++i) rv[i] = c < a.Dk ? rv[i] : 0.f;
        }
      }
      float* s_part = &s_acc[0][0][0];  // [kParts][HMAX][DKP], free until the epilogue
      // two heads per (uniform) branch, so their q reads share one LDS round
      // trip; rows of absent heads hold zeros and are never read back
      constexpr int kHS = HMAX >= 2 ? 2 : 1;
#pragma unroll
      for (int h = 0; h < HMAX; h += kHS) {
        if (h < nh) {
          float acc_h[kHS];
#pragma unroll
          for (int j = 0; j < kHS; ++j) {
            acc_h[j] = 0.f;
#pragma unroll
            for (int i = 0; i < kL; ++i) acc_h[j] += s_q[h + j][part * kL + i] * rv[i];
          }
#pragma unroll
          for (int j = 0; j < kHS; ++j) s_part[(part * HMAX + h + j) * DKP + c] = acc_h[j];
        }
      }
      __syncthreads();
      for (int i = tid; i < HMAX * DKP; i += kThreads) {
        const int h = i / DKP, cc = i % DKP;
        float sum = 0.f;
        if (h < nh) {
#pragma unroll
          for (int pp = 0; pp < kParts; ++pp) sum += s_part[(pp * HMAX + h) * DKP + cc];
        }
        s_qt[h][cc] = sum;
      }
      q_dot_dm();
      __syncthreads();
    }

    uint4 qh[DKB], ql[DKB];
#pragma unroll
    for (int kb = 0; kb < DKB; ++kb) {
      uint16_t hv[8], lv[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const float v = (n < HMAX) ? s_qt[nq][kb * 32 + 8 * g + e] : 0.f;
        TT::split(v, hv[e], lv[e]);
      }
      qh[kb] = pack8(hv);
      ql[kb] = pack8(lv);
    }
    const float bias2 = (n < HMAX ? s_bias[nq] : 0.f) * a.scale_log2;
    auto compute = [&](VisBuf<DKB>& B, int64_t blk) {
      // rows 8g + 4sb + i of the block at or past `lim` lie beyond the chunk
      const int lim = (int)min(t_end - (t_begin + blk * kBlk), (int64_t)kBlk);
      float s[8];
#pragma unroll
      for (int sb = 0; sb < 2; ++sb) {
        f32x4 cc = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int kb = 0; kb < DKB; ++kb) cc = TT::mfma(zero_if(kval[kb], B.k[sb][kb]), qh[kb], cc);
#pragma unroll
        for (int kb = 0; kb < DKB; ++kb) cc = TT::mfma(zero_if(kval[kb], B.k[sb][kb]), ql[kb], cc);
#pragma unroll
        for (int i = 0; i < 4; ++i)
          s[4 * sb + i] = (8 * g + 4 * sb + i < lim) ? fmaf(cc[i], a.scale_log2, bias2) : -INFINITY;
      }
      softmax_pv<TT>(s, B.v, m, l, acc);
    };
    ring.run(load, compute);
  } else {
    // ---- prompt + text span: full-width Keys
    const int64_t t_begin = (int64_t)xf * a.chunk_full;
    const int64_t s_f = a.len_full ? min(a.S_f, (int64_t)max(a.len_full[b], 0)) : a.S_f;
    const int64_t t_end = max(t_begin, min(s_f, t_begin + a.chunk_full));
    const uint32_t t_last = (uint32_t)max(t_begin, t_end - 1);
    const uint16_t* kfb = a.kf + b * a.kf_sb + kv * a.kf_sh;
    const uint16_t* vfb = a.vf + b * a.vf_sb + kv * a.vf_sh;
    const uint32_t vch = 8u * n;
    const int64_t nblk = (t_end - t_begin + kBlk - 1) / kBlk;
    auto load = [&](FullBuf& B, int64_t blk) {
      const uint32_t t0 = (uint32_t)(t_begin + blk * kBlk);
      const uint32_t r0 = min(t0 + krow0, t_last) * a.kf_ss, r1 = min(t0 + krow1, t_last) * a.kf_ss;
#pragma unroll
      for (int kb = 0; kb < 4; ++kb) {
        B.k[0][kb] = load_row8<VEC, false>(kfb, r0, (uint32_t)(kb * 32 + 8 * g), a.kf_sd, 8);
        B.k[1][kb] = load_row8<VEC, false>(kfb, r1, (uint32_t)(kb * 32 + 8 * g), a.kf_sd, 8);
      }
#pragma unroll
      for (int r = 0; r < 8; ++r) {
        uint32_t row = min(t0 + 8u * g + r, t_last);
        row += row >= a.vf_gap_at ? a.vf_gap : 0u;
        B.v[r] = load_row8<VEC, NTL>(vfb, row * a.vf_ss, vch, a.vf_sd, 8);
      }
    };

    // first K/V blocks, then q and the mask bytes (see the visual path)
    Ring<NBUF_F, FullBuf> ring(nblk, wave, rot_seed);
    ring.prime(load);
    load_q();
    load_new();
    const uint8_t* mb = a.mask ? a.mask + b * a.mf_sb : nullptr;
    uint32_t mv[kMaskChunk / kThreads];  // one register each: no byte packing between loads
    if (mb && t_end > t_begin) {  // uniform: all mask loads issued together
#pragma unroll
      for (int k = 0; k < kMaskChunk / kThreads; ++k)
        mv[k] = mb[min(t_begin + tid + k * kThreads, t_end - 1) * a.mf_ss];
    } else {
#pragma unroll
      for (int k = 0; k < kMaskChunk / kThreads; ++k) mv[k] = 1;
    }
    // keep the compares on the mask below this point (the compiler would
    // otherwise test each byte as it arrives, one memory latency per byte)
#pragma unroll
    for (int k = 0; k < kMaskChunk / kThreads; ++k) asm volatile("" : "+v"(mv[k]));

    store_q();
    store_new();
#pragma unroll
    for (int k = 0; k < kMaskChunk / kThreads; ++k) {
      const int i = tid + k * kThreads;
      s_valid[i] = (t_begin + i < t_end) && mv[k] != 0;
    }
    __syncthreads();

    uint4 qf[4];
#pragma unroll
    for (int kb = 0; kb < 4; ++kb) {
      uint16_t hv[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) hv[e] = TT::from_f32((n < HMAX) ? s_q[nq][kb * 32 + 8 * g + e] : 0.f);
      qf[kb] = pack8(hv);
    }
    auto compute = [&](FullBuf& B, int64_t blk) {
      const uint2 vb = *(const uint2*)&s_valid[blk * kBlk + 8 * g];
      float s[8];
#pragma unroll
      for (int sb = 0; sb < 2; ++sb) {
        f32x4 cc = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int kb = 0; kb < 4; ++kb) cc = TT::mfma(B.k[sb][kb], qf[kb], cc);
        const uint32_t w = sb ? vb.y : vb.x;
#pragma unroll
        for (int i = 0; i < 4; ++i)
          s[4 * sb + i] = ((w >> (8 * i)) & 0xffu) ? cc[i] * a.scale_log2 : -INFINITY;
      }
      softmax_pv<TT>(s, B.v, m, l, acc);
    };
    ring.run(load, compute);
  }

  // ---- fused append: wave 0 attends the new token (score q . k_new, a
  // full-width token without bias) as one more row of its online softmax
  if (has_new && wave == 0) {
    float d = 0.f;
#pragma unroll
    for (int c = 0; c < 32; ++c) d = fmaf(s_q[nq][32 * g + c], s_new[0][32 * g + c], d);
    d += shfl_xor(d, 16);
    d += shfl_xor(d, 32);
    const float sn = d * a.scale_log2;
    const float m_new = fmaxf(m, sn);
    const float alpha = fast_exp2(m - m_new), w = fast_exp2(sn - m_new);
#pragma unroll
    for (int j = 0; j < 8; ++j)
#pragma unroll
      for (int i = 0; i < 4; ++i) acc[j][i] = acc[j][i] * alpha + w * s_new[1][32 * g + 8 * i + j];
    l = l * alpha + (g == 0 ? w : 0.f);
    m = m_new;
  }

  // ---- merge the four wave states into this workgroup's partial
  float lt = l + shfl_xor(l, 16);
  lt += shfl_xor(lt, 32);
  if (n < HMAX) {
    if (g == 0) {
      s_m[wave][nq] = m;
      s_l[wave][nq] = lt;
    }
#pragma unroll
    for (int j = 0; j < 8; ++j)
#pragma unroll
      for (int i = 0; i < 4; ++i) s_acc[wave][nq][32 * g + 8 * i + j] = acc[j][i];
  }
  __syncthreads();
  {
    const int h = tid >> 4, c8 = tid & 15;
    if (h < nh) {
      float M = -INFINITY;
#pragma unroll
      for (int w = 0; w < kWaves; ++w) M = fmaxf(M, s_m[w][h]);
      float L = 0.f, A[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int w = 0; w < kWaves; ++w) {
        const float wt = fast_exp2(s_m[w][h] - M);
        L += s_l[w][h] * wt;
#pragma unroll
        for (int e = 0; e < 8; ++e) A[e] += s_acc[w][h][8 * c8 + e] * wt;
      }
      float* rec = a.part + (((int64_t)u * a.np + x) * a.hpu + h) * kRecFloats;
      if (a.fused)
        store_rec<true>(rec, c8, A, M, L);
      else
        store_rec<false>(rec, c8, A, M, L);
    }
  }
  if (a.fused) merge_fused<TT, APPEND>(a, u, b, h0, nh, tid, HMAX >= 16 ? &s_acc[0][0][0] : (float*)s_rsep);
}

// ---- fp32 decode (q, K, V and out in F32; R_partial and delta_mu F16,
// BF16 or F32), the dtype of the reference's CPU-scale configuration.  The
// reference kernels load any float input as fp32 and compute in fp32
// (fused_decode.py:133,166,174; full_channel_flash_decoding.py:65,84,92);
// so does this kernel, on the VALU: fp32 has no MFMA path that keeps its
// precision at this arithmetic intensity.  One unit per query head (hpu 1),
// the plan's grid and records as the 16-bit kernel, so both merges apply.
// Each wave walks 64-token blocks of its workgroup's chunk (blocks wave,
// wave + 4, ...): lane t scores token t0 + t as a dot product over its
// row, the wave runs the online softmax (log2 domain), and lane j
// accumulates channels 2j, 2j + 1 of P V over the block's rows, with the
// block's probabilities broadcast from LDS.
constexpr int kBlk32 = 64;

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v = fmaxf(v, shfl_xor(v, off));
  return v;
}
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v += shfl_xor(v, off);
  return v;
}

// sum_c w[c] * row[c * sd], c < n <= KMAX; w in LDS.  VEC: unit stride,
// 16-byte aligned row, n a multiple of 4: all KMAX / 4 16-byte loads are
// issued before any is used (those past n re-read the row's last four
// floats, in bounds, and are not used), so the row costs one memory round
// trip; float4 i accumulates into s0 (i even) or s1 (i odd).
template <bool VEC, int KMAX>
__device__ __forceinline__ float dot_row32(const float* row, uint32_t sd, const float* w, int n) {
  float s0 = 0.f, s1 = 0.f;
  if constexpr (VEC) {
    if (n <= 0) return 0.f;
    float4 r[KMAX / 4];
#pragma unroll
    for (int i = 0; i < KMAX / 4; ++i) r[i] = *(const float4*)(row + min(4 * i, n - 4));
#pragma unroll
    for (int i = 0; i < KMAX / 4; ++i) {
      if (4 * i < n) {
        const float4 w4 = *(const float4*)(w + 4 * i);
        float& acc = (i & 1) ? s1 : s0;
        acc = fmaf(w4.x, r[i].x, acc);
        acc = fmaf(w4.y, r[i].y, acc);
        acc = fmaf(w4.z, r[i].z, acc);
        acc = fmaf(w4.w, r[i].w, acc);
      }
    }
  } else {
    for (int c = 0; c < n; ++c) s0 = fmaf(w[c], row[(int64_t)c * sd], s0);
  }
  return s0 + s1;
}

template <bool HAS_VIS, bool VEC>
__global__ void __launch_bounds__(kThreads) decode32_kernel(const DecodeArgs a) {
  __shared__ __attribute__((aligned(16))) float s_q[128];
  __shared__ __attribute__((aligned(16))) float s_qt[128];
  __shared__ float s_bias[2];
  __shared__ float s_p[kWaves][kBlk32];
  __shared__ float s_m[kWaves], s_l[kWaves];
  __shared__ float s_acc[kWaves][128];
  __shared__ float s_mrg[16 * kRecFloats];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int u = blockIdx.y, x = blockIdx.x;
  const int b = u / a.units_per_b;
  const int r_in_b = u - b * a.units_per_b;
  const int kv = r_in_b / a.spk;
  const int h0 = kv * a.G + (r_in_b - kv * a.spk) * a.hpu;
  const bool is_vis = HAS_VIS && x < a.wg_vis;
  const int xf = HAS_VIS ? x - a.wg_vis : x;
  const float* q = (const float*)a.q;

  if (tid < 128) s_q[tid] = q[b * a.q_sb + (int64_t)h0 * a.q_sh + (int64_t)tid * a.q_sd];
  __syncthreads();

  float m = kNegInit, l = 0.f, acc0 = 0.f, acc1 = 0.f;
  // online-softmax step over one block: s = log2-domain score of token
  // t0 + lane (-inf when invalid), V rows clamped to t_last
  auto step = [&](float s, const float* vb, uint32_t vss, uint32_t vsd, int64_t t0, int64_t t_last,
                  uint32_t gap_at, uint32_t gap) {
    const float m_new = fmaxf(m, wave_max(s));
    const float alpha = fast_exp2(m - m_new);
    const float p = fast_exp2(s - m_new);
    l = l * alpha + wave_sum(p);
    acc0 *= alpha;
    acc1 *= alpha;
    m = m_new;
    s_p[wave][lane] = p;
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    // the block's V rows in two batches of 32 loads in flight (one memory
    // round trip each), then their fused multiply-adds in token order
    constexpr int kVB = 32;
#pragma unroll
    for (int j0 = 0; j0 < kBlk32; j0 += kVB) {
      float v0[kVB], v1[kVB];
#pragma unroll
      for (int jj = 0; jj < kVB; ++jj) {
        uint32_t row = (uint32_t)min(t0 + j0 + jj, t_last);
        row += row >= gap_at ? gap : 0u;
        const float* vr = vb + (int64_t)row * vss;
        if constexpr (VEC) {
          const float2 v = *(const float2*)(vr + 2 * lane);
          v0[jj] = v.x;
          v1[jj] = v.y;
        } else {
          v0[jj] = vr[(int64_t)(2 * lane) * vsd];
          v1[jj] = vr[(int64_t)(2 * lane + 1) * vsd];
        }
      }
#pragma unroll
      for (int jj = 0; jj < kVB; ++jj) {
        const float pj = s_p[wave][j0 + jj];
        acc0 = fmaf(pj, v0[jj], acc0);
        acc1 = fmaf(pj, v1[jj], acc1);
      }
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  };

  if (is_vis) {
    {  // q R_partial: thread (half, c) sums rows 64 half .. 64 half + 63 of
       // column c, all 64 loads in flight; the halves meet in LDS
      const int c = tid & 127, half = tid >> 7;
      const int cc = min(c, max(a.Dk - 1, 0));
      const int64_t rb = b * a.R_sb + kv * a.R_sh + (int64_t)cc * a.R_sk;
      float sum = 0.f;
      if (a.Dk > 0) {
        float rv[64];
        load_any_n(a.R, rb + (int64_t)(64 * half) * a.R_sd, a.R_sd, a.r_dtype, rv);
#pragma unroll
        for (int i = 0; i < 64; ++i) sum = fmaf(s_q[64 * half + i], rv[i], sum);
      }
      s_acc[half][c] = sum;  // s_acc is free until the epilogue
      __syncthreads();
      if (tid < 128) s_qt[tid] = tid < a.Dk ? s_acc[0][tid] + s_acc[1][tid] : 0.f;
    }
    if (wave < 2) {  // q . delta_mu
      const int d = tid;
      const float t = a.has_bias ? s_q[d] * load_any(a.dm, b * a.dm_sb + kv * a.dm_sh + (int64_t)d * a.dm_sd,
                                                    a.dm_dtype)
                                 : 0.f;
      const float w = wave_sum(t);
      if (lane == 0) s_bias[wave] = w;
    }
    __syncthreads();
    const float bias2 = (s_bias[0] + s_bias[1]) * a.scale_log2;
    const int64_t t_begin = (int64_t)x * a.chunk_vis;
    const int64_t t_end = min(a.S_v, t_begin + a.chunk_vis);
    const float* ksb = (const float*)a.ks + b * a.ks_sb + kv * a.ks_sh;
    const float* vsb = (const float*)a.vs + b * a.vs_sb + kv * a.vs_sh;
    for (int64_t t0 = t_begin + (int64_t)wave * kBlk32; t0 < t_end; t0 += kWaves * kBlk32) {
      const int64_t t = t0 + lane;
      const float* kr = ksb + (int64_t)min(t, t_end - 1) * a.ks_ss;
      const float d = a.Dk <= 32   ? dot_row32<VEC, 32>(kr, a.ks_sd, s_qt, a.Dk)
                      : a.Dk <= 64 ? dot_row32<VEC, 64>(kr, a.ks_sd, s_qt, a.Dk)
                                   : dot_row32<VEC, 128>(kr, a.ks_sd, s_qt, a.Dk);
      const float s = t < t_end ? fmaf(d, a.scale_log2, bias2) : -INFINITY;
      step(s, vsb, a.vs_ss, a.vs_sd, t0, t_end - 1, UINT32_MAX, 0u);
    }
  } else {
    const int64_t t_begin = (int64_t)xf * a.chunk_full;
    const int64_t t_end = min(a.S_f, t_begin + a.chunk_full);
    const float* kfb = (const float*)a.kf + b * a.kf_sb + kv * a.kf_sh;
    const float* vfb = (const float*)a.vf + b * a.vf_sb + kv * a.vf_sh;
    for (int64_t t0 = t_begin + (int64_t)wave * kBlk32; t0 < t_end; t0 += kWaves * kBlk32) {
      const int64_t t = t0 + lane;
      const int64_t tc = min(t, t_end - 1);
      const float d = dot_row32<VEC, 128>(kfb + tc * a.kf_ss, a.kf_sd, s_q, 128);
      const bool ok = t < t_end && (!a.mask || a.mask[b * a.mf_sb + tc * a.mf_ss] != 0);
      step(ok ? d * a.scale_log2 : -INFINITY, vfb, a.vf_ss, a.vf_sd, t0, t_end - 1, a.vf_gap_at, a.vf_gap);
    }
  }

  // the four wave states -> this workgroup's record
  if (lane == 0) {
    s_m[wave] = m;
    s_l[wave] = l;
  }
  s_acc[wave][2 * lane] = acc0;
  s_acc[wave][2 * lane + 1] = acc1;
  __syncthreads();
  if (tid < 16) {
    const int c8 = tid;
    float M = -INFINITY;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) M = fmaxf(M, s_m[w]);
    float L = 0.f, A[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int w = 0; w < kWaves; ++w) {
      const float wt = fast_exp2(s_m[w] - M);
      L += s_l[w] * wt;
#pragma unroll
      for (int e = 0; e < 8; ++e) A[e] += s_acc[w][8 * c8 + e] * wt;
    }
    float* rec = a.part + ((int64_t)u * a.np + x) * kRecFloats;
    if (a.fused)
      store_rec<true>(rec, c8, A, M, L);
    else
      store_rec<false>(rec, c8, A, M, L);
  }
  if (a.fused) merge_fused<F32, false>(a, u, b, h0, 1, tid, s_mrg);
}

// Second launch: one workgroup per unit runs merge_unit, or with one query
// head per unit (hpu == 1) one workgroup per 16 units, a slice each
// (merge_slice).  With a fused append the unit holding query head 0 of row
// b advances len_full[b]; the split launch that read it has completed.
template <class TT>
__global__ void __launch_bounds__(kThreads) merge_kernel(const DecodeArgs a) {
  __shared__ float s_mrg[16 * kRecFloats];
  const int tid = threadIdx.x;
  const bool sliced = a.hpu == 1;
  const int64_t u = sliced ? (int64_t)blockIdx.x * 16 + (tid >> 4) : (int64_t)blockIdx.x;
  if (u >= a.units) return;  // sliced: the last workgroup's spare slices
  const int b = (int)(u / a.units_per_b);
  const int r_in_b = (int)(u - (int64_t)b * a.units_per_b);
  const int kv = r_in_b / a.spk;
  const int jblk = r_in_b - kv * a.spk;
  const int h0 = kv * a.G + jblk * a.hpu;
  if (sliced)
    merge_slice<TT, false>(a, u, b, h0, tid & 15);
  else
    merge_unit<TT, false>(a, u, b, h0, min(a.hpu, a.G - jblk * a.hpu), tid, s_mrg);
  if (a.k_new && r_in_b == 0 && (tid & (sliced ? 15 : 255)) == 0) {
    const int32_t pos = (int32_t)min(a.S_f, (int64_t)max(a.len_full[b], 0));
    if (pos < a.S_f) a.len_full[b] = pos + 1;
  }
}

}  // namespace rk

// =====================================================================
// host side
// =====================================================================
#include "rk_host.h"

namespace {

// Planner knobs (rk_set_decode_*): process-wide, atomic, and read once per
// plan (Knobs), so a plan never mixes values of a concurrent change.
//
// Bytes of K/V a workgroup streams: total / (2 * CUs), clamped to
// [64 KB, 512 KB].  Measured on MI355X: 512 KB chunks are within 2-5% of the
// best split at B=32/16k (MHA), B=16/32k (GQA) and B=1/16k; small problems
// get at least ~2 workgroups per CU.
std::atomic<int64_t> g_min_wg_bytes{INT64_C(64) << 10};
std::atomic<int64_t> g_max_wg_bytes{INT64_C(512) << 10};
// Workgroups planned per CU: 0 (default) plans two (the kernel's register
// budget holds two per CU), or one for a single round of small workgroups
// (rk_plan_decode); n > 0 plans n.
std::atomic<int32_t> g_wgs_per_cu{0};
// Visual chunks are whole multiples of this many tokens (a 32-token block
// or the 128 tokens of one block per wave); 0: 32 in a chunk-major grid,
// else 128.
std::atomic<int64_t> g_chunk_align{0};
// One-round grids of short workgroups (see rk_plan_decode): 0 keeps the
// unit-major launch, 1000 launches chunk-major with equal chunks, more
// gives the first-dispatched chunks of the smallest workgroups this many
// thousandths of the others' tokens.
std::atomic<int32_t> g_skew_permille{1300};

int64_t cdiv(int64_t a, int64_t b) { return (a + b - 1) / b; }
int64_t round_up(int64_t a, int64_t b) { return cdiv(a, b) * b; }
size_t align256(size_t x) { return (x + 255) & ~size_t(255); }

constexpr int64_t kWgTokens = rk::kWaves * rk::kBlk;  // 128
// Bytes one resident workgroup slot streams during a workgroup's fixed
// latency (prologue + epilogue, ~8 us at ~14 GB/s per slot on MI355X).
constexpr int64_t kSlotLatencyBytes = INT64_C(128) << 10;
constexpr int64_t kMinWgsPerUnit = 8;
constexpr int64_t kSkewMaxBytes = INT64_C(128) << 10;
// Two-slot visual workgroups of at most this many bytes in a one-round
// chunk-major grid are planned one per CU instead (rk_plan_decode); units
// of one query head (a lighter prologue, and a single-launch merge that
// then folds half the records) gain up to larger workgroups.
constexpr int64_t kOneSlotMaxBytes = INT64_C(128) << 10;
constexpr int64_t kOneSlotMaxBytesOneHead = INT64_C(192) << 10;
constexpr int64_t kOneSlotMaxBytesOneHeadNarrow = INT64_C(256) << 10;  // <= 32 kept channels

// Merge mode (rk_set_decode_merge): 0 (default) = per shape (below),
// 1 = two launches,
// 2 = single launch where the ticket region holds the counters.
std::atomic<int32_t> g_merge_mode{0};

// One plan's snapshot of the knobs above (a byte cap below the floor reads
// as the floor).
struct Knobs {
  int64_t min_wg, max_wg, chunk_align;
  int32_t wgs_per_cu, skew_permille, merge_mode;
  int64_t resident() const { return wgs_per_cu > 0 ? wgs_per_cu : 2; }
};

Knobs knobs() {
  constexpr auto r = std::memory_order_relaxed;
  Knobs k;
  k.min_wg = g_min_wg_bytes.load(r);
  k.max_wg = g_max_wg_bytes.load(r);
  k.chunk_align = g_chunk_align.load(r);
  k.wgs_per_cu = g_wgs_per_cu.load(r);
  k.skew_permille = g_skew_permille.load(r);
  k.merge_mode = g_merge_mode.load(r);
  if (k.max_wg < k.min_wg) k.max_wg = k.min_wg;
  return k;
}

struct WsLayout {
  size_t ticket, bticket, part, total;
};

// The ticket region (fixed size, at offset 0, so that every shape finds its
// counters at zero whatever earlier calls wrote past it), then one partial
// record per (unit, workgroup, head).
WsLayout ws_layout(const rk_decode_plan& p) {
  const int64_t np = p.wg_vis + p.wg_full;
  const size_t parts = (size_t)p.units * np * p.heads_per_unit;
  WsLayout w;
  w.ticket = 0;
  w.bticket = (size_t)p.units * sizeof(uint32_t);
  w.part = RK_DECODE_TICKET_BYTES;
  w.total = w.part + align256(parts * rk::kRecFloats * sizeof(float));
  return w;
}

// Single-launch merge where the counters fit: on request (mode 2), or by
// default for one round of units of one query head each, where the unit's
// last workgroup merges with one 16-lane slice (merge_slice).  Measured on
// MI355X (eager / graph us per step, two launches -> one): B=1, 32 heads,
// 16k context 35.9 / 35.3 -> 33.8 / 33.4; the same at 2.4k tokens in fp32
// 32.4-33.2 / 26.9 -> 29.3-30.1 / 25.8.  Elsewhere one launch ends no
// earlier than two: its tail (record stores written through and waited
// for, ~2 us under load; the ticket, ~0.5 us; a multi-head unit's merge,
// ~3.5 us) is as long as the kernel boundary plus the merge kernel, and the
// split phase's slowest workgroup finishes 1-2 us later (B=8 with 4 KV heads
// of 7 query heads, 12001 + 61 tokens: both end at 34 us; over 28 layers in
// one graph, one launch 938 us against 891 us per step).  On grids of many
// rounds it is worse still: every workgroup holds its slot through its own
// wait (B=32, 16k context: 935 against 815 us; B=4, 32 heads, 4.6k tokens,
// two rounds: 44.2 -> 44.8 us).
bool use_single_launch(const rk_decode_plan& p, int64_t B, int cus, const Knobs& k) {
  if (p.units + B > (int64_t)(RK_DECODE_TICKET_BYTES / sizeof(uint32_t))) return false;
  if (k.merge_mode != 0) return k.merge_mode == 2;
  return p.heads_per_unit == 1 && p.grid <= (int64_t)cus * k.resident();
}

}  // namespace

namespace {

__global__ void __launch_bounds__(256) zero_words_kernel(uint32_t* p, int64_t n) {
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x)
    p[i] = 0u;
}

}  // namespace

extern "C" int rk_decode_workspace_init(void* workspace, size_t workspace_bytes, void* stream) {
  if (!workspace) return RK_ERR_NULL;
  if ((((uintptr_t)workspace) & 255) != 0) return RK_ERR_WORKSPACE;
  const size_t n = (workspace_bytes < RK_DECODE_TICKET_BYTES ? workspace_bytes : RK_DECODE_TICKET_BYTES) / 4;
  if (n == 0) return RK_OK;
  hipLaunchKernelGGL(zero_words_kernel, dim3(64), dim3(256), 0, (hipStream_t)stream, (uint32_t*)workspace,
                     (int64_t)n);
  return hipGetLastError() == hipSuccess ? RK_OK : RK_ERR_HIP;
}

extern "C" void rk_set_decode_merge(int32_t mode) {
  if (mode >= 0 && mode <= 2) g_merge_mode.store(mode, std::memory_order_relaxed);
}

extern "C" void rk_set_decode_chunk_align(int32_t tokens) {
  if (tokens == 0 || tokens == rk::kBlk || tokens == 2 * rk::kBlk || tokens == kWgTokens)
    g_chunk_align.store(tokens, std::memory_order_relaxed);
}

extern "C" void rk_set_decode_skew(int32_t permille) {
  if (permille == 0 || (permille >= 1000 && permille <= 4000))
    g_skew_permille.store(permille, std::memory_order_relaxed);
}

extern "C" void rk_set_decode_tuning(int64_t min_bytes, int64_t max_bytes, int32_t wgs_per_cu) {
  constexpr auto r = std::memory_order_relaxed;
  if (min_bytes > 0) g_min_wg_bytes.store(min_bytes, r);
  if (max_bytes > 0) g_max_wg_bytes.store(max_bytes, r);
  if (wgs_per_cu > 0) g_wgs_per_cu.store(wgs_per_cu, r);
  if (wgs_per_cu < 0) g_wgs_per_cu.store(0, r);
}

namespace {

// The chunking of a plan whose unit fields are set, for rounds of `slots`
// resident workgroups on `num_cus` CUs.
int split_plan(rk_decode_plan& p, int64_t Dk, int64_t S_v, int64_t S_f, int32_t elem_bytes, int64_t slots,
               int32_t num_cus, const Knobs& k) {
  // Workgroups run in rounds of `slots` resident workgroups (two per CU at
  // the kernel's register budget).  A partial last round costs as much as a
  // full one, so the grid is sized to whole rounds: the fewest rounds that
  // keep a workgroup at <= the byte cap, then as many workgroups per unit
  // as those rounds hold (but none below the byte floor), split between the
  // visual and prompt/text spans in proportion to their bytes.
  const int64_t unit_vis = S_v * (Dk + 128) * elem_bytes;
  const int64_t unit_full = S_f * 256 * elem_bytes;
  const int64_t unit_bytes = unit_vis + unit_full;
  const int64_t total = p.units * unit_bytes;
  // A unit with several query heads pays more per workgroup (q R for every
  // head, one merge row each), so it takes larger chunks: measured on MI355X,
  // a GQA group of 7 runs best in a single round of up to 4 MB workgroups,
  // one query head per unit at 512 KB.
  const int64_t max_wg = p.heads_per_unit > 1 ? 8 * k.max_wg : k.max_wg;
  int64_t rounds = cdiv(total, slots * max_wg);
  // ... and enough rounds for kMinWgsPerUnit workgroups per unit: with many
  // units a single round leaves each unit one or two workgroups of several
  // MB (measured on MI355X, B=32 with 8 KV heads of 4 query heads: 228 us
  // at 2-3 workgroups per unit, 216 us at 7; a floor of 12 or 16 instead of
  // 8 measured slower: that shape 210 -> 218-220 us, config 3 110 -> 114,
  // config 2 811 -> 817)
  const int64_t by_units = cdiv(kMinWgsPerUnit * p.units, slots);
  if (rounds < by_units && total / (by_units * slots) >= k.min_wg) rounds = by_units;
  if (rounds < 1) rounds = 1;
  int64_t budget = p.units > 0 ? rounds * slots / p.units : 1;
  const int64_t by_min = unit_bytes / k.min_wg;
  if (budget > by_min) budget = by_min;
  if (budget < 1) budget = 1;
  // Each span gets its byte share of the budget, rounded, at least one
  // workgroup.  A prompt/text span too small for a workgroup of its own
  // still gets one; the visual span then keeps its full share (and the grid
  // overflows the rounds) only if that shortens each visual workgroup by
  // more than a slot streams during a workgroup's fixed latency, since the
  // overflow waits that long for the small workgroups' slots.  80
  // prompt/text tokens beside 16000 visual ones at two slots per unit keep
  // two visual workgroups (not one); 60 beside 12001 at sixteen slots give
  // the slot back.
  int64_t w_full = 0, w_vis = 0;
  if (S_f > 0) {
    w_full = (budget * unit_full + unit_bytes / 2) / unit_bytes;
    if (w_full < 1) w_full = 1;
  }
  if (S_v > 0) {
    w_vis = (budget * unit_vis + unit_bytes / 2) / unit_bytes;
    if (w_vis < 1) w_vis = 1;
    const int64_t fit = budget - w_full > 1 ? budget - w_full : 1;
    if (w_vis > fit && p.units * (w_vis + w_full) > rounds * slots &&
        unit_vis / fit - unit_vis / w_vis < kSlotLatencyBytes)
      w_vis = fit;
  }
  // One round of workgroups of at most the byte cap (a grid of short
  // workgroups, whose fixed costs show) launches chunk-major (below) with
  // 32-token chunks, so that the round's slots fill.
  const bool short_round = k.skew_permille > 0 && elem_bytes == 2 && S_v > 0 && rounds == 1 &&
                           unit_bytes <= (w_vis + w_full) * k.max_wg;
  const int64_t align = k.chunk_align > 0 ? k.chunk_align : short_round ? rk::kBlk : kWgTokens;
  if (S_v > 0) {
    p.chunk_vis = round_up(cdiv(S_v, w_vis), align);
    p.wg_vis = (int32_t)cdiv(S_v, p.chunk_vis);
  }
  if (S_f > 0) {
    p.chunk_full = round_up(cdiv(S_f, w_full), kWgTokens);
    if (p.chunk_full > rk::kMaskChunk) p.chunk_full = rk::kMaskChunk;
    p.wg_full = (int32_t)cdiv(S_f, p.chunk_full);
  }
  if (p.wg_vis + p.wg_full == 0) {  // nothing to attend: one empty chunk writes zeros
    p.wg_full = 1;
    p.chunk_full = kWgTokens;
  }
  p.grid = p.units * (p.wg_vis + p.wg_full);
  if (p.units > 65535 * 1024 || p.wg_vis + p.wg_full > (1 << 30)) return RK_ERR_SHAPE;
  // Chunk-major launch (workgroup id x * units + u) of a short round: with
  // units a multiple of 8, all chunks of a unit run on one XCD (ids go to
  // the XCDs round-robin), which then fetches the unit's q, R_partial and
  // delta_mu once into its L2 instead of every XCD fetching every unit's.
  // Measured on MI355X over 28 graph-replayed layers of B=8, 4 KV heads of
  // 7 query heads: 945 -> 894 us per step at 12001 visual tokens, 740 ->
  // 665 us at 4097 (keep 32); B=1, 32 heads, 16k: 35.2 -> 35.0 us.  Rounds
  // of larger workgroups keep the unit-major launch (B=16, 32k, G=7: 1.4 MB
  // workgroups, 111.8 us unit-major, 113.5 us chunk-major).
  if (short_round && p.grid <= slots && p.grid <= 65535) p.chunk_major = 1;
  // The CUs take the first num_cus workgroup ids one each, then the rest.
  // Both workgroups of a CU start together, but the first-dispatched one
  // streams faster (per-workgroup timestamps on MI355X: 76 against 103 us
  // at B=16, 32k context, G=7; 17 against 21 us on a B=8, 12001-token
  // layer).  In a chunk-major grid the first num_cus ids are the chunks
  // x < n_fast = num_cus / units of every unit.  Where workgroups stream
  // <= 128 KB (fixed latency dominates), those chunks take chunk_fast
  // tokens, skew_permille / 1000 times the others' (whole 32-token
  // blocks): B=8, 4097 visual tokens, keep 32, 665 -> 648 us per step; at
  // 12001 tokens (256 KB workgroups) the skew measured 894 -> 903 us.
  if (p.chunk_major && k.skew_permille > 1000 && p.wg_vis >= 2 && p.grid > num_cus &&
      unit_vis <= p.wg_vis * kSkewMaxBytes) {
    const int64_t nf = num_cus / p.units, ns = p.wg_vis - nf;
    const int64_t nb = cdiv(S_v, rk::kBlk);
    if (nf >= 1 && ns >= 1) {
      const double rho = k.skew_permille / 1000.0;
      const int64_t bf = (int64_t)(rho * (double)nb / ((double)nf * rho + (double)ns) + 0.5);
      const int64_t bs = nb - nf * bf > 0 ? cdiv(nb - nf * bf, ns) : 0;
      if (bs >= 1 && bf > bs && nf * bf + (ns - 1) * bs < nb) {
        p.n_fast = (int32_t)nf;
        p.chunk_fast = bf * rk::kBlk;
        p.chunk_vis = bs * rk::kBlk;
      }
    }
  }
  return RK_OK;
}

}  // namespace

extern "C" int rk_plan_decode(int64_t B, int64_t H_q, int64_t H_kv, int64_t Dk, int64_t S_v,
                              int64_t S_f, int32_t elem_bytes, int32_t policy, int32_t num_cus,
                              rk_decode_plan* plan) {
  if (!plan) return RK_ERR_NULL;
  if (B < 0 || H_q <= 0 || H_kv <= 0 || S_v < 0 || S_f < 0 || elem_bytes <= 0 || num_cus <= 0)
    return RK_ERR_ARG;
  if (H_q % H_kv != 0) return RK_ERR_HEADS;
  if (policy != RK_POLICY_PAPER && policy != RK_POLICY_GQA) return RK_ERR_ARG;
  const int64_t G = H_q / H_kv;
  rk_decode_plan p;
  memset(&p, 0, sizeof(p));
  if (policy == RK_POLICY_GQA) {
    p.heads_per_unit = (int32_t)(G < 16 ? G : 16);
    p.head_blocks = (int32_t)cdiv(G, 16);
    p.units = B * H_kv * p.head_blocks;
  } else {
    p.heads_per_unit = 1;
    p.head_blocks = 1;
    p.units = B * H_q;
  }
  const rk_decode_plan units_only = p;
  const Knobs k = knobs();
  int st = split_plan(p, Dk, S_v, S_f, elem_bytes, (int64_t)num_cus * k.resident(), num_cus, k);
  if (st) return st;
  // A single round of small workgroups (two-slot visual chunks of <= 128 KB)
  // runs faster as one workgroup per CU of twice the tokens, where that is
  // still one chunk-major round: the fixed costs of a workgroup (prologue,
  // the merge of its waves, its record) are paid once per CU, the unit's
  // merge folds half the records, and no CU holds a later-dispatched,
  // slower-streaming second workgroup.  Graph-replayed layers on MI355X (us,
  // two slots -> one): B=8, 4 KV heads of 7 query heads, keep 32, 2049 /
  // 4097 / 6001 visual tokens 17.2 -> 16.3, 19.7 -> 18.8, 22.1 -> 21.3;
  // B=1, 32 heads, 4000 + 640 tokens 20.1 -> 18.2.  At 143-160 KB the two
  // slots are 1-2 % faster (8001 tokens: 23.8 against 24.1), and where one
  // slot per CU needs a second round they are faster still (B=16, 2049
  // tokens: 21.2 against 22.5).  Units of one query head gain up to
  // 256 KB at <= 32 kept channels (B=1, 32 heads, 640 prompt/text tokens,
  // 6000 / 8000 visual tokens: 22.2 -> 20.4, 23.9 -> 22.8 us; with the
  // one-per-CU MFMA q R, 10000 / 11000 / 12000: 26.6 -> 24.9, 27.2 ->
  // 26.4, 28.2 -> 27.7 us; 13000, 277 KB, loses: 29.5 against 31.6) but
  // lose at 209 KB with 64 (24.7 against 25.2), so theirs is 192 KB.
  const int64_t one_slot_max = p.heads_per_unit > 1 ? kOneSlotMaxBytes
                               : Dk <= 32            ? kOneSlotMaxBytesOneHeadNarrow
                                                     : kOneSlotMaxBytesOneHead;
  if (k.wgs_per_cu == 0 && p.chunk_major && S_v * (Dk + 128) * elem_bytes <= p.wg_vis * one_slot_max) {
    rk_decode_plan one = units_only;
    if (split_plan(one, Dk, S_v, S_f, elem_bytes, num_cus, num_cus, k) == RK_OK && one.chunk_major &&
        one.grid <= num_cus)
      p = one;
  }
  // fp32 (the VALU kernel, unit-major): one workgroup per CU whenever that
  // is still one round, at any workgroup size up to the cap.  With two
  // slots a grid of a little over num_cus leaves some CUs two workgroups,
  // which finish last.  Graph-replayed decodes on MI355X (us, two slots ->
  // one), B=1, 32 heads, 128 prompt/text tokens: 1024 / 2304 / 4608 / 6000
  // visual tokens 20.9 -> 14.7, 25.9 -> 19.2, 35.2 -> 26.4, 38.6 -> 32.0;
  // 4 KV heads of 7 query heads at 4096 tokens 28.5 -> 20.4.  Where one
  // slot per CU needs a second round (B=1 at 8192 tokens, B=2 or 4), the
  // two-slot plan is as fast or faster and is kept.
  if (k.wgs_per_cu == 0 && elem_bytes == 4 && p.grid > num_cus) {
    rk_decode_plan one = units_only;
    if (split_plan(one, Dk, S_v, S_f, elem_bytes, num_cus, num_cus, k) == RK_OK && one.grid <= num_cus) p = one;
  }
  p.workspace_bytes = ws_layout(p).total;
  p.single_launch = use_single_launch(p, B, num_cus, k) ? 1 : 0;
  *plan = p;
  return RK_OK;
}

namespace {

struct Checked {
  int64_t B, H_q, H_kv, G, Dk, S_v, S_f;
  int dtype;
};

int check_out(const rk_tensor* out, const Checked& c) {
  int st = rk::check_desc(out, 3);
  if (st) return st;
  if (out->dtype != c.dtype) return RK_ERR_DTYPE;
  if (out->shape[0] != c.B || out->shape[1] != c.H_q || out->shape[2] != 128) return RK_ERR_SHAPE;
  return RK_OK;
}

int check_kv4(const rk_tensor* t, const Checked& c, int64_t S, int64_t last, bool dtype_must_match) {
  int st = rk::check_desc(t, 4);
  if (st) return st;
  if (dtype_must_match && t->dtype != c.dtype) return RK_ERR_DTYPE;
  if (t->shape[0] != c.B || t->shape[1] != c.H_kv || t->shape[2] != S || t->shape[3] != last)
    return RK_ERR_SHAPE;
  return RK_OK;
}

// Validation mirroring fused_decode.py:323-338 (plus the shape agreement
// the Triton kernels assume but do not check).
int check_rotatek(const rk_tensor* q, const rk_tensor* R, const rk_tensor* dm,
                  const rk_tensor* kf, const rk_tensor* vf, const rk_tensor* mask,
                  const rk_tensor* ks, const rk_tensor* vs, int64_t G, Checked* c) {
  if (!q || !R || !kf || !vf || !ks || !vs) return RK_ERR_NULL;
  if (q->ndim != 3) return RK_ERR_RANK;
  if (R->ndim != 4) return RK_ERR_RANK;
  if (mask && mask->dtype != RK_U8) return RK_ERR_DTYPE;
  int st = rk::check_desc(q, 3);
  if (st) return st;
  st = rk::check_desc(R, 4);
  if (st) return st;
  if (G <= 0) return RK_ERR_ARG;
  c->B = q->shape[0];
  c->H_q = q->shape[1];
  c->H_kv = R->shape[1];
  c->G = G;
  c->Dk = R->shape[3];
  c->dtype = q->dtype;
  if (c->H_q / G != c->H_kv || c->H_q % G != 0) return RK_ERR_HEADS;
  if (!rk::is_half(q->dtype) && q->dtype != RK_F32) return RK_ERR_DTYPE;
  if (q->shape[2] != 128) return RK_ERR_HEAD_DIM;
  if (!rk::is_float_param(R->dtype)) return RK_ERR_DTYPE;
  if (R->shape[0] != c->B || R->shape[2] != 128) return RK_ERR_SHAPE;
  // Dk = 0 (channel_ratio >= 1, every channel pruned): visual logits are the
  // bias q . delta_mu alone, as the reference's kernels give with no kept
  // channel (its masked BLOCK_DK loads, fused_decode.py:131-148)
  if (c->Dk < 0 || c->Dk > 128) return RK_ERR_KEEP_DIM;
  if (dm) {
    st = rk::check_desc(dm, 3);
    if (st) return st;
    if (!rk::is_float_param(dm->dtype)) return RK_ERR_DTYPE;
    if (dm->shape[0] != c->B || dm->shape[1] != c->H_kv || dm->shape[2] != 128) return RK_ERR_SHAPE;
  }
  st = rk::check_desc(kf, 4);
  if (st) return st;
  c->S_f = kf->shape[2];
  st = rk::check_desc(ks, 4);
  if (st) return st;
  c->S_v = ks->shape[2];
  if ((st = check_kv4(kf, *c, c->S_f, 128, true))) return st;
  if ((st = check_kv4(vf, *c, c->S_f, 128, true))) return st;
  if ((st = check_kv4(ks, *c, c->S_v, c->Dk, true))) return st;
  if ((st = check_kv4(vs, *c, c->S_v, 128, true))) return st;
  if (mask) {
    st = rk::check_desc(mask, 2);
    if (st) return st;
    if (mask->shape[0] != c->B || mask->shape[1] != c->S_f) return RK_ERR_SHAPE;
  }
  return RK_OK;
}

// The RotateK entry points run the paper family (ROTATEK_KERNEL=paper, one
// unit per query head, fused_decode.py:370) with the grouped decomposition
// when query heads share a KV head: the G heads of a group then read each
// K/V tile once instead of G times (measured on MI355X, B=32 with 8 KV heads
// of 4 query heads: 429 -> 208 us).  Every head's scores, softmax and P V
// are computed as in the per-head decomposition, in fp32 with the same
// hi + lo operand splits, so the two differ only in fp32 summation order.
// The dense baseline keeps the per-head decomposition (the reference's
// structure, full_channel_flash_decoding.py:197-203).
int32_t rotatek_policy(int32_t policy, int64_t G) {
  return policy == RK_POLICY_PAPER && G > 1 ? RK_POLICY_GQA : policy;
}

// The plan of a checked call.  fp32 runs one unit per query head (the
// VALU kernel has no grouped form) over 4-byte elements.
int plan_for(const Checked& c, bool has_vis, int32_t policy, int cus, rk_decode_plan* p) {
  const bool f32 = c.dtype == RK_F32;
  return rk_plan_decode(c.B, c.H_q, c.H_kv, has_vis ? c.Dk : 0, has_vis ? c.S_v : 0, c.S_f, f32 ? 4 : 2,
                        f32 ? RK_POLICY_PAPER : policy, cus, p);
}

int resolve_cus(int32_t num_cus, int* st) {
  *st = RK_OK;
  if (num_cus > 0) return num_cus;
  int dev = 0;
  const int cus = rk::current_device_cus(&dev);
  if (cus <= 0) *st = RK_ERR_NO_DEVICE;
  return cus;
}

// Workgroups of the merge kernel: one per unit, or one per 16 units of one
// query head each (merge_kernel's sliced form).
unsigned merge_grid(const rk::DecodeArgs& a) {
  return (unsigned)(a.hpu == 1 ? (a.units + 15) / 16 : a.units);
}

template <class TT, int DKB, bool VEC, int HMAX, bool HAS_VIS>
hipError_t launch_one(const rk::DecodeArgs& a, dim3 grid, hipStream_t s) {
  bool launched = false;
  // grouped one-unit-per-query-head mode (temporal loads): the dense
  // baseline's paper family at G > 1 only (the RotateK entries run that
  // family grouped, see rotatek_policy)
  if constexpr (VEC && HMAX == 1 && !HAS_VIS) {
    if (a.xgroup > 1) {
      hipLaunchKernelGGL((rk::decode_kernel<TT, DKB, VEC, HMAX, HAS_VIS, false, false>), grid,
                         dim3(rk::kThreads), 0, s, a);
      launched = true;
    }
  }
  if constexpr (HAS_VIS) {  // the span cache's step always carries the visual span
    if (!launched && a.k_new) {
      hipLaunchKernelGGL((rk::decode_kernel<TT, DKB, VEC, HMAX, true, true>), grid, dim3(rk::kThreads), 0,
                         s, a);
      launched = true;
    }
  }
  if (!launched)
    hipLaunchKernelGGL((rk::decode_kernel<TT, DKB, VEC, HMAX, HAS_VIS, false>), grid, dim3(rk::kThreads), 0,
                       s, a);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess || a.fused) return e;
  hipLaunchKernelGGL((rk::merge_kernel<TT>), dim3(merge_grid(a)), dim3(rk::kThreads), 0, s, a);
  return hipGetLastError();
}

template <class TT, int DKB, bool VEC, int HMAX>
hipError_t launch_vis(bool has_vis, const rk::DecodeArgs& a, dim3 grid, hipStream_t s) {
  return has_vis ? launch_one<TT, DKB, VEC, HMAX, true>(a, grid, s)
                 : launch_one<TT, 1, VEC, HMAX, false>(a, grid, s);
}

template <class TT, int DKB, bool VEC>
hipError_t launch_h(int hmax, bool has_vis, const rk::DecodeArgs& a, dim3 grid, hipStream_t s) {
  return hmax > 1 ? launch_vis<TT, DKB, VEC, 16>(has_vis, a, grid, s)
                  : launch_vis<TT, DKB, VEC, 1>(has_vis, a, grid, s);
}

template <class TT, int DKB>
hipError_t launch_v(bool vec, int hmax, bool has_vis, const rk::DecodeArgs& a, dim3 grid,
                    hipStream_t s) {
  return vec ? launch_h<TT, DKB, true>(hmax, has_vis, a, grid, s)
             : launch_h<TT, DKB, false>(hmax, has_vis, a, grid, s);
}

template <class TT>
hipError_t launch_dk(int dkb, bool vec, int hmax, bool has_vis, const rk::DecodeArgs& a, dim3 grid,
                     hipStream_t s) {
  switch (dkb) {
    case 1: return launch_v<TT, 1>(vec, hmax, has_vis, a, grid, s);
    case 2: return launch_v<TT, 2>(vec, hmax, has_vis, a, grid, s);
    default: return launch_v<TT, 4>(vec, hmax, has_vis, a, grid, s);
  }
}

// fp32 rows read as float4 / float2: unit channel stride, every other
// stride a multiple of 4 elements, 16-byte aligned base.
bool vec32_ok(const rk_tensor* t) {
  if (!t || !t->data) return true;
  if (t->stride[t->ndim - 1] != 1 && t->shape[t->ndim - 1] > 1) return false;
  for (int i = 0; i < t->ndim - 1; ++i)
    if (t->shape[i] > 1 && (t->stride[i] % 4) != 0) return false;
  return (((uintptr_t)t->data) & 15) == 0;
}

hipError_t launch32(bool has_vis, bool vec, const rk::DecodeArgs& a, dim3 grid, hipStream_t s) {
  if (has_vis) {
    if (vec)
      hipLaunchKernelGGL((rk::decode32_kernel<true, true>), grid, dim3(rk::kThreads), 0, s, a);
    else
      hipLaunchKernelGGL((rk::decode32_kernel<true, false>), grid, dim3(rk::kThreads), 0, s, a);
  } else {
    if (vec)
      hipLaunchKernelGGL((rk::decode32_kernel<false, true>), grid, dim3(rk::kThreads), 0, s, a);
    else
      hipLaunchKernelGGL((rk::decode32_kernel<false, false>), grid, dim3(rk::kThreads), 0, s, a);
  }
  hipError_t e = hipGetLastError();
  if (e != hipSuccess || a.fused) return e;
  hipLaunchKernelGGL((rk::merge_kernel<rk::F32>), dim3(merge_grid(a)), dim3(rk::kThreads), 0, s, a);
  return hipGetLastError();
}

void set4(const rk_tensor* t, int64_t& s0, int64_t& s1, int64_t& s2, int64_t& s3) {
  s0 = t->stride[0];
  s1 = t->stride[1];
  s2 = t->stride[2];
  s3 = t->stride[3];
}

// Head strides (b, h) as int64; token/channel strides as uint32 with the
// whole within-head span, plus 32 rows, below 2^31 elements (kernel offsets
// are 32-bit byte offsets) and the token stride below 2^26.
bool set_head(const rk_tensor* t, int64_t& sb, int64_t& sh, uint32_t& ss, uint32_t& sd) {
  sb = t->stride[0];
  sh = t->stride[1];
  // (32 rows of slack: the visual ring adds a block's row offsets to its
  // first row before clamping to the chunk's last row)
  const int64_t span = (t->shape[2] > 0 ? (t->shape[2] - 1 + 32) * t->stride[2] : 0) +
                       (t->shape[3] > 0 ? (t->shape[3] - 1) * t->stride[3] : 0) + 8;
  if (span >= (INT64_C(1) << 31) || t->stride[2] >= (INT64_C(1) << 26) ||
      t->stride[3] >= (INT64_C(1) << 31))
    return false;
  ss = (uint32_t)t->stride[2];
  sd = (uint32_t)t->stride[3];
  return true;
}

int run_decode(const Checked& c, const rk_tensor* q, const rk_tensor* R, const rk_tensor* dm,
               const rk_tensor* kf, const rk_tensor* vf, const rk_tensor* mask,
               const rk_tensor* ks, const rk_tensor* vs, const rk_tensor* out, int32_t policy,
               void* ws, size_t ws_bytes, void* stream, bool has_vis,
               int32_t* len_full = nullptr, int64_t v_gap_at = -1, int64_t v_gap = 0,
               const rk_tensor* k_new = nullptr, const rk_tensor* v_new = nullptr) {
  int st = RK_OK;
  const int cus = resolve_cus(0, &st);
  if (st) return st;
  rk_decode_plan p;
  st = plan_for(c, has_vis, policy, cus, &p);
  if (st) return st;
  if (!ws || (((uintptr_t)ws) & 255) != 0 || ws_bytes < p.workspace_bytes) return RK_ERR_WORKSPACE;
  if (c.B == 0) return RK_OK;
  const bool vis_work = has_vis && c.S_v > 0;
  if (!q->data || !out->data || (vis_work && ((c.Dk > 0 && (!R->data || !ks->data)) || !vs->data)) ||
      (c.S_f > 0 && (!kf->data || !vf->data)))
    return RK_ERR_NULL;
  const WsLayout w = ws_layout(p);
  rk::DecodeArgs a;
  memset(&a, 0, sizeof(a));
  a.q = (const uint16_t*)q->data;
  a.out = (uint16_t*)out->data;
  a.kf = (const uint16_t*)kf->data;
  a.vf = (const uint16_t*)vf->data;
  a.part = (float*)((char*)ws + w.part);
  a.ticket = (uint32_t*)((char*)ws + w.ticket);
  a.bticket = (uint32_t*)((char*)ws + w.bticket);
  a.fused = p.single_launch;
  a.q_sb = q->stride[0];
  a.q_sh = q->stride[1];
  a.q_sd = q->stride[2];
  a.o_sb = out->stride[0];
  a.o_sh = out->stride[1];
  a.o_sd = out->stride[2];
  if (!set_head(kf, a.kf_sb, a.kf_sh, a.kf_ss, a.kf_sd) ||
      !set_head(vf, a.vf_sb, a.vf_sh, a.vf_ss, a.vf_sd))
    return RK_ERR_STRIDE;
  if (mask && mask->data) {
    a.mask = (const uint8_t*)mask->data;
    a.mf_sb = mask->stride[0];
    a.mf_ss = mask->stride[1];
    a.has_mask = 1;
  }
  bool vec = rk::vec_ok(kf) && rk::vec_ok(vf);
  a.q_vec = q->stride[2] == 1 && q->stride[1] % 8 == 0 && q->stride[0] % 8 == 0 &&
            (((uintptr_t)q->data) & 15) == 0;
  int dkb = 1;
  if (has_vis) {
    a.R = R->data;
    a.r_dtype = R->dtype;
    set4(R, a.R_sb, a.R_sh, a.R_sd, a.R_sk);
    if (dm && dm->data) {
      a.dm = dm->data;
      a.dm_dtype = dm->dtype;
      a.dm_sb = dm->stride[0];
      a.dm_sh = dm->stride[1];
      a.dm_sd = dm->stride[2];
      a.has_bias = 1;
    }
    // R staged into LDS (16-byte DMA): up to 64 channels in either 16-bit
    // type; 65-128 only in the compute type (their q R is an MFMA product
    // read straight from the staged rows, and R fills the kernel's s_acc)
    a.r_vec = rk::is_half(R->dtype) && (c.Dk <= 64 || (c.Dk <= 128 && R->dtype == c.dtype)) &&
              R->stride[3] == 1 && R->stride[2] == c.Dk &&
              R->stride[1] % 8 == 0 && R->stride[0] % 8 == 0 && (((uintptr_t)R->data) & 15) == 0;
    a.ks = (const uint16_t*)ks->data;
    a.vs = (const uint16_t*)vs->data;
    if (!set_head(vs, a.vs_sb, a.vs_sh, a.vs_ss, a.vs_sd)) return RK_ERR_STRIDE;
    if (c.Dk > 0) {
      if (!set_head(ks, a.ks_sb, a.ks_sh, a.ks_ss, a.ks_sd)) return RK_ERR_STRIDE;
    } else {
      // no kept channel: the (unconditional, masked-out) Key loads read the
      // visual Value rows instead, so no address depends on an empty tensor
      a.ks = a.vs;
      a.ks_sb = a.vs_sb;
      a.ks_sh = a.vs_sh;
      a.ks_ss = a.vs_ss;
      a.ks_sd = a.vs_sd;
    }
    a.S_v = c.S_v;
    a.Dk = (int32_t)c.Dk;
    vec = vec && (c.Dk == 0 || rk::vec_ok(ks)) && rk::vec_ok(vs) && (c.Dk % 8 == 0);
    dkb = c.Dk <= 32 ? 1 : c.Dk <= 64 ? 2 : 4;
  }
  a.S_f = c.S_f;
  a.len_full = len_full;
  if (k_new) {
    a.k_new = (const uint16_t*)k_new->data;
    a.v_new = (const uint16_t*)v_new->data;
    a.kf_w = (uint16_t*)kf->data;
    a.vf_w = (uint16_t*)vf->data;
    a.kn_sb = k_new->stride[0];
    a.kn_sh = k_new->stride[1];
    a.kn_sd = k_new->stride[3];
    a.vn_sb = v_new->stride[0];
    a.vn_sh = v_new->stride[1];
    a.vn_sd = v_new->stride[3];
  }
  a.vf_gap_at = v_gap_at < 0 ? UINT32_MAX : (uint32_t)v_gap_at;
  a.vf_gap = (uint32_t)v_gap;
  a.chunk_vis = p.chunk_vis;
  a.chunk_full = p.chunk_full;
  a.G = (int32_t)c.G;
  a.hpu = p.heads_per_unit;
  a.spk = policy == RK_POLICY_GQA ? p.head_blocks : (int32_t)c.G;
  a.units_per_b = (int32_t)(p.units / c.B);
  a.wg_vis = p.wg_vis;
  a.np = p.wg_vis + p.wg_full;
  // XCD balance.  Workgroup u * np + x runs on XCD (u * np + x) mod 8, so
  // with g = gcd(np, 8) > 1 chunk x of every unit lands on the XCDs
  // congruent to x mod g.  When the visual chunks do not split evenly over
  // those classes, some XCDs get the small prompt/text chunks and less of
  // the visual stream (np = 8: all prompt/text chunks on XCD 7).  Rotating
  // each unit's chunk numbers by u spreads them.  Measured on MI355X:
  // B=32 with 8 KV heads of 4 query heads 219.8 -> 208.7 us, config 3
  // 112.7 -> 110.0 us.  The rotation is not applied where nothing aliases:
  // there it measured 0.6-2.4 % slower (configs 2 and 4).
  {
    int gx = 8;
    while (a.np % gx != 0) gx >>= 1;
    a.rot_x = gx > 1 && p.wg_vis % gx != 0 ? 1 : 0;
  }
  a.units = (int32_t)p.units;
  a.xgroup = policy == RK_POLICY_PAPER && c.G > 1 && c.dtype != RK_F32 ? (int32_t)c.G : 0;
  if (a.xgroup || c.dtype == RK_F32) a.rot_x = 0;
  if (c.dtype == RK_F32) a.spk = (int32_t)c.G;  // one unit per query head
  a.scale_log2 = (float)(rk::kLog2e / sqrt(128.0));
  a.cmajor = has_vis && c.dtype != RK_F32 && !a.xgroup ? p.chunk_major : 0;
  a.nfast = a.cmajor ? p.n_fast : 0;
  a.chunk_fast = p.chunk_fast;
  if (a.cmajor) a.rot_x = 0;
  const dim3 grid = a.cmajor ? dim3((unsigned)p.units, (unsigned)a.np) : dim3((unsigned)a.np, (unsigned)p.units);
  const int hmax = p.heads_per_unit > 1 ? 16 : 1;
  // Rows of <= 32 kept channels form q R on the MFMA too where each CU runs
  // one workgroup (the one-per-CU plans): nothing streams during that
  // workgroup's prologue, so the shorter MFMA prologue pays.  In two-slot
  // rounds the CU's other workgroup hides the FMA prologue and the MFMA
  // form measured slower.  Graph-replayed config 4 steps on MI355X (28
  // layers, us): 4097 visual tokens keep 32 / 16 576.5 -> 558.9 / 545.8 ->
  // 535.2; at 12001 tokens (two slots) 864.1 -> 875.9 with the MFMA form.
  a.qr_mfma = dkb == 1 && a.cmajor && p.grid <= cus ? 1 : 0;
  hipStream_t s = (hipStream_t)stream;
  if (c.dtype == RK_F32) {
    const bool v32 = vec32_ok(kf) && vec32_ok(vf) &&
                     (!has_vis || ((c.Dk == 0 || vec32_ok(ks)) && vec32_ok(vs) && c.Dk % 4 == 0));
    return launch32(has_vis, v32, a, grid, s) == hipSuccess ? RK_OK : RK_ERR_HIP;
  }
  hipError_t e = c.dtype == RK_F16 ? launch_dk<rk::F16>(dkb, vec, hmax, has_vis, a, grid, s)
                                   : launch_dk<rk::BF16>(dkb, vec, hmax, has_vis, a, grid, s);
  return e == hipSuccess ? RK_OK : RK_ERR_HIP;
}

}  // namespace

extern "C" int rk_rotatek_decode_check(const rk_tensor* q_full, const rk_tensor* R_partial,
                                       const rk_tensor* delta_mu, const rk_tensor* k_full,
                                       const rk_tensor* v_full, const rk_tensor* mask_full,
                                       const rk_tensor* k_sparse, const rk_tensor* v_sparse,
                                       int64_t num_kv_groups, const rk_tensor* out,
                                       int32_t policy, int32_t num_cus, size_t* workspace_bytes) {
  Checked c;
  int st = check_rotatek(q_full, R_partial, delta_mu, k_full, v_full, mask_full, k_sparse, v_sparse,
                         num_kv_groups, &c);
  if (st) return st;
  if (out && (st = check_out(out, c))) return st;
  const int cus = resolve_cus(num_cus, &st);
  if (st) return st;
  if (policy != RK_POLICY_PAPER && policy != RK_POLICY_GQA) return RK_ERR_ARG;
  rk_decode_plan p;
  st = plan_for(c, true, rotatek_policy(policy, c.G), cus, &p);
  if (st) return st;
  if (workspace_bytes) *workspace_bytes = p.workspace_bytes;
  return RK_OK;
}

extern "C" int rk_rotatek_decode(const rk_tensor* q_full, const rk_tensor* R_partial,
                                 const rk_tensor* delta_mu, const rk_tensor* k_full,
                                 const rk_tensor* v_full, const rk_tensor* mask_full,
                                 const rk_tensor* k_sparse, const rk_tensor* v_sparse,
                                 int64_t num_kv_groups, const rk_tensor* out, int32_t policy,
                                 void* workspace, size_t workspace_bytes, void* stream) {
  Checked c;
  int st = check_rotatek(q_full, R_partial, delta_mu, k_full, v_full, mask_full, k_sparse, v_sparse,
                         num_kv_groups, &c);
  if (st) return st;
  if (!out) return RK_ERR_NULL;
  if ((st = check_out(out, c))) return st;
  if (policy != RK_POLICY_PAPER && policy != RK_POLICY_GQA) return RK_ERR_ARG;
  return run_decode(c, q_full, R_partial, delta_mu, k_full, v_full, mask_full, k_sparse, v_sparse,
                    out, rotatek_policy(policy, c.G), workspace, workspace_bytes, stream, true);
}

extern "C" int rk_rotatek_decode_varlen(const rk_tensor* q_full, const rk_tensor* R_partial,
                                        const rk_tensor* delta_mu, const rk_tensor* k_full,
                                        const rk_tensor* v_buf, int64_t v_gap_at, int64_t v_gap,
                                        const rk_tensor* mask_full, const rk_tensor* k_sparse,
                                        const rk_tensor* v_sparse, int64_t num_kv_groups,
                                        const rk_tensor* k_new, const rk_tensor* v_new,
                                        int32_t* len_full, const rk_tensor* out, int32_t policy,
                                        void* workspace, size_t workspace_bytes, void* stream) {
  if (!k_full || !v_buf) return RK_ERR_NULL;
  int st = rk::check_desc(v_buf, 4);
  if (st) return st;
  if ((st = rk::check_desc(k_full, 4))) return st;
  const int64_t S_f = k_full->shape[2];
  if (v_gap < 0 || v_gap_at < 0 || v_gap_at > S_f || v_gap >= (INT64_C(1) << 31)) return RK_ERR_ARG;
  if (v_buf->shape[2] != S_f + v_gap) return RK_ERR_SHAPE;
  rk_tensor v_logical = *v_buf;  // prompt/text rows only, for the shape checks
  v_logical.shape[2] = S_f;
  Checked c;
  st = check_rotatek(q_full, R_partial, delta_mu, k_full, &v_logical, mask_full, k_sparse, v_sparse,
                     num_kv_groups, &c);
  if (st) return st;
  if (!out || !len_full) return RK_ERR_NULL;
  if (c.dtype == RK_F32) return RK_ERR_DTYPE;  // the span cache holds 16-bit Keys and Values
  if ((st = check_out(out, c))) return st;
  if (policy != RK_POLICY_PAPER && policy != RK_POLICY_GQA) return RK_ERR_ARG;
  if ((k_new == nullptr) != (v_new == nullptr)) return RK_ERR_NULL;
  if (k_new) {
    for (const rk_tensor* t : {k_new, v_new}) {
      if ((st = rk::check_desc(t, 4))) return st;
      if (t->dtype != c.dtype) return RK_ERR_DTYPE;
      if (t->shape[0] != c.B || t->shape[1] != c.H_kv || t->shape[2] != 1 || t->shape[3] != 128)
        return RK_ERR_SHAPE;
      if (c.B > 0 && !t->data) return RK_ERR_NULL;
    }
  }
  return run_decode(c, q_full, R_partial, delta_mu, k_full, v_buf, mask_full, k_sparse, v_sparse,
                    out, rotatek_policy(policy, c.G), workspace, workspace_bytes, stream, true, len_full,
                    v_gap > 0 ? v_gap_at : -1, v_gap, k_new, v_new);
}

namespace {

// One workgroup per batch row: copy the new token's K (and V) of every head
// into slot len[b] of the span buffers, then advance len[b].  A full buffer
// (len[b] >= capacity) is left untouched.
__global__ void __launch_bounds__(256) append_kernel(const uint16_t* kn, int64_t kn_b, int64_t kn_h,
                                                     int64_t kn_d, const uint16_t* vn, int64_t vn_b,
                                                     int64_t vn_h, int64_t vn_d, uint16_t* kb,
                                                     int64_t kb_b, int64_t kb_h, int64_t kb_s,
                                                     int64_t kb_d, uint16_t* vb, int64_t vb_b,
                                                     int64_t vb_h, int64_t vb_s, int64_t vb_d,
                                                     int32_t* len, int H, int64_t cap) {
  const int b = blockIdx.x;
  const int32_t pos = len[b];
  __syncthreads();
  if (pos >= 0 && pos < cap) {
    for (int i = threadIdx.x; i < H * 128; i += blockDim.x) {
      const int h = i >> 7, d = i & 127;
      kb[b * kb_b + h * kb_h + pos * kb_s + d * kb_d] = kn[b * kn_b + h * kn_h + d * kn_d];
      if (vn) vb[b * vb_b + h * vb_h + pos * vb_s + d * vb_d] = vn[b * vn_b + h * vn_h + d * vn_d];
    }
    __syncthreads();
    if (threadIdx.x == 0) len[b] = pos + 1;
  }
}

}  // namespace

extern "C" int rk_append_kv(const rk_tensor* k_new, const rk_tensor* v_new, const rk_tensor* k_buf,
                            const rk_tensor* v_buf, int32_t* len_full, void* stream) {
  if (!k_new || !k_buf || !len_full) return RK_ERR_NULL;
  int st = rk::check_desc(k_new, 4);
  if (st) return st;
  if ((st = rk::check_desc(k_buf, 4))) return st;
  if (!rk::is_half(k_new->dtype) || k_buf->dtype != k_new->dtype) return RK_ERR_DTYPE;
  const int64_t B = k_new->shape[0], H = k_new->shape[1];
  if (k_new->shape[2] != 1 || k_new->shape[3] != 128) return RK_ERR_SHAPE;
  if (k_buf->shape[0] != B || k_buf->shape[1] != H || k_buf->shape[3] != 128) return RK_ERR_SHAPE;
  if ((v_new == nullptr) != (v_buf == nullptr)) return RK_ERR_NULL;
  if (v_new) {
    if ((st = rk::check_desc(v_new, 4)) || (st = rk::check_desc(v_buf, 4))) return st;
    if (v_new->dtype != k_new->dtype || v_buf->dtype != k_new->dtype) return RK_ERR_DTYPE;
    for (int i = 0; i < 4; ++i)
      if (v_new->shape[i] != k_new->shape[i] || v_buf->shape[i] != k_buf->shape[i]) return RK_ERR_SHAPE;
  }
  if (B == 0 || H == 0) return RK_OK;
  if (!k_new->data || !k_buf->data || (v_new && (!v_new->data || !v_buf->data))) return RK_ERR_NULL;
  if (B > (INT64_C(1) << 30) || H * 128 > (INT64_C(1) << 30)) return RK_ERR_SHAPE;
  hipLaunchKernelGGL(append_kernel, dim3((unsigned)B), dim3(256), 0, (hipStream_t)stream,
                     (const uint16_t*)k_new->data, k_new->stride[0], k_new->stride[1], k_new->stride[3],
                     v_new ? (const uint16_t*)v_new->data : nullptr, v_new ? v_new->stride[0] : 0,
                     v_new ? v_new->stride[1] : 0, v_new ? v_new->stride[3] : 0, (uint16_t*)k_buf->data,
                     k_buf->stride[0], k_buf->stride[1], k_buf->stride[2], k_buf->stride[3],
                     v_buf ? (uint16_t*)v_buf->data : nullptr, v_buf ? v_buf->stride[0] : 0,
                     v_buf ? v_buf->stride[1] : 0, v_buf ? v_buf->stride[2] : 0, v_buf ? v_buf->stride[3] : 0,
                     len_full, (int)H, k_buf->shape[2]);
  return hipGetLastError() == hipSuccess ? RK_OK : RK_ERR_HIP;
}

namespace {

// Validation mirroring full_channel_flash_decoding.py:173-178.
int check_dense(const rk_tensor* q, const rk_tensor* k, const rk_tensor* v, int64_t G, Checked* c) {
  if (!q || !k || !v) return RK_ERR_NULL;
  if (q->ndim != 3) return RK_ERR_RANK;
  int st = rk::check_desc(q, 3);
  if (st) return st;
  if ((st = rk::check_desc(k, 4))) return st;
  if (G <= 0) return RK_ERR_ARG;
  c->B = q->shape[0];
  c->H_q = q->shape[1];
  c->H_kv = k->shape[1];
  c->G = G;
  c->Dk = 0;
  c->S_v = 0;
  c->S_f = k->shape[2];
  c->dtype = q->dtype;
  if (k->shape[3] != q->shape[2] || v->ndim < 1 || v->shape[v->ndim - 1] != q->shape[2])
    return RK_ERR_SHAPE;
  if (c->H_kv <= 0 || c->H_q / G != c->H_kv || c->H_q % G != 0) return RK_ERR_HEADS;
  if (!rk::is_half(q->dtype) && q->dtype != RK_F32) return RK_ERR_DTYPE;
  if (q->shape[2] != 128) return RK_ERR_HEAD_DIM;
  if ((st = check_kv4(k, *c, c->S_f, 128, true))) return st;
  if ((st = check_kv4(v, *c, c->S_f, 128, true))) return st;
  return RK_OK;
}

}  // namespace

extern "C" int rk_full_channel_decode_check(const rk_tensor* q, const rk_tensor* k,
                                            const rk_tensor* v, int64_t num_kv_groups,
                                            const rk_tensor* out, int32_t policy, int32_t num_cus,
                                            size_t* workspace_bytes) {
  Checked c;
  int st = check_dense(q, k, v, num_kv_groups, &c);
  if (st) return st;
  if (out && (st = check_out(out, c))) return st;
  const int cus = resolve_cus(num_cus, &st);
  if (st) return st;
  rk_decode_plan p;
  st = plan_for(c, false, policy, cus, &p);
  if (st) return st;
  if (workspace_bytes) *workspace_bytes = p.workspace_bytes;
  return RK_OK;
}

extern "C" int rk_full_channel_decode(const rk_tensor* q, const rk_tensor* k, const rk_tensor* v,
                                      int64_t num_kv_groups, const rk_tensor* out, int32_t policy,
                                      void* workspace, size_t workspace_bytes, void* stream) {
  Checked c;
  int st = check_dense(q, k, v, num_kv_groups, &c);
  if (st) return st;
  if (!out) return RK_ERR_NULL;
  if ((st = check_out(out, c))) return st;
  if (policy != RK_POLICY_PAPER && policy != RK_POLICY_GQA) return RK_ERR_ARG;
  return run_decode(c, q, nullptr, nullptr, k, v, nullptr, nullptr, nullptr, out, policy, workspace,
                    workspace_bytes, stream, false);
}

// ---- allocation-free decode (rk_rotatek_decode_noalloc)
// The workspace of the other entry points, as a file-scope device array:
// each GPU the library runs on holds its own copy until the process ends.
// Host code never uses the array's name as a device address (on the host
// it is only a stand-in): hipGetSymbolAddress gives each device's address,
// once per device, and that pointer is what the kernels receive.
static __device__ __align__(256) unsigned char scratch[RK_NOALLOC_SCRATCH_BYTES];

namespace {

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices];

// This device's `scratch`: on the first call on a device, its address
// (checked) and a cleared ticket region (a fill kernel on `stream`, ahead
// of the decode that follows on the same stream).
int device_scratch(hipStream_t stream, void** ptr) {
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0) return RK_ERR_NO_DEVICE;
  if (dev >= kMaxDevices) return RK_ERR_ARG;
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void* p = nullptr;
    if (hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)) != hipSuccess || !p) return RK_ERR_HIP;
    const int st = rk_decode_workspace_init(p, RK_DECODE_TICKET_BYTES, stream);
    if (st) return st;
    g_scratch_ptr[dev] = p;
  }
  *ptr = g_scratch_ptr[dev];
  return RK_OK;
}

}  // namespace

extern "C" int rk_rotatek_decode_noalloc(const rk_tensor* q_full, const rk_tensor* R_partial,
                                         const rk_tensor* delta_mu, const rk_tensor* k_full,
                                         const rk_tensor* v_full, const rk_tensor* mask_full,
                                         const rk_tensor* k_sparse, const rk_tensor* v_sparse,
                                         int64_t num_kv_groups, const rk_tensor* out, int32_t policy,
                                         void* stream) {
  Checked c;
  int st = check_rotatek(q_full, R_partial, delta_mu, k_full, v_full, mask_full, k_sparse, v_sparse,
                         num_kv_groups, &c);
  if (st) return st;
  if (!out) return RK_ERR_NULL;
  if ((st = check_out(out, c))) return st;
  if (policy != RK_POLICY_PAPER && policy != RK_POLICY_GQA) return RK_ERR_ARG;
  const int32_t pol = rotatek_policy(policy, c.G);
  const int cus = resolve_cus(0, &st);
  if (st) return st;
  rk_decode_plan p;
  if ((st = plan_for(c, true, pol, cus, &p))) return st;
  if (p.workspace_bytes > RK_NOALLOC_SCRATCH_BYTES) return RK_ERR_SCRATCH;
  void* ws = nullptr;
  if ((st = device_scratch((hipStream_t)stream, &ws))) return st;
  return run_decode(c, q_full, R_partial, delta_mu, k_full, v_full, mask_full, k_sparse, v_sparse, out, pol,
                    ws, RK_NOALLOC_SCRATCH_BYTES, stream, true);
}
