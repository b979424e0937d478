// rk_decode_dev.h -- fused split-K RotateK decode kernels for MI355X (gfx950),
// included by the per-dtype launch units (rk_decode_{f16,bf16,f32}.hip).
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
#pragma once

#include <math.h>

#include "rk_common.h"
#include "rk_decode.h"
#include "rotatek_hip.h"

namespace rk {


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

// Records are written and read back either with ordinary stores and loads
// (COH false: the merge kernel reads what the split launch wrote) or, for
// the single-launch merge, with relaxed agent-scope atomic stores and loads
// (COH true): the stores write through the XCD's L2 to memory and the
// loads read from there, so the unit's last workgroup, on any XCD, sees
// every other workgroup's record (each XCD has its own L2).
__device__ __forceinline__ uint64_t pack_f2(float a, float b) {
  return (uint64_t)__builtin_bit_cast(uint32_t, a) | ((uint64_t)__builtin_bit_cast(uint32_t, b) << 32);
}
__device__ __forceinline__ float lo_f(uint64_t w) { return __builtin_bit_cast(float, (uint32_t)w); }
__device__ __forceinline__ float hi_f(uint64_t w) { return __builtin_bit_cast(float, (uint32_t)(w >> 32)); }

// Channels 8 c8 .. 8 c8 + 7 of a record's acc, and its (m, l).
template <bool COH>
__device__ __forceinline__ void load_rec(const float* rec, int c8, float (&v)[8], float& m, float& l) {
  if constexpr (COH) {
    const uint64_t* p = (const uint64_t*)(rec + 8 * c8);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const uint64_t w = __hip_atomic_load(p + i, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      v[2 * i] = lo_f(w);
      v[2 * i + 1] = hi_f(w);
    }
    const uint64_t w = __hip_atomic_load((const uint64_t*)(rec + 128), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    m = lo_f(w);
    l = hi_f(w);
  } else {
    const float4 s0 = ((const float4*)(rec + 8 * c8))[0], s1 = ((const float4*)(rec + 8 * c8))[1];
    const float2 ml = *(const float2*)(rec + 128);
    v[0] = s0.x; v[1] = s0.y; v[2] = s0.z; v[3] = s0.w;
    v[4] = s1.x; v[5] = s1.y; v[6] = s1.z; v[7] = s1.w;
    m = ml.x;
    l = ml.y;
  }
}

// Store of a workgroup's record slice (the lane's eight acc channels; m and
// l by the c8 == 0 lane).
template <bool COH>
__device__ __forceinline__ void store_rec(float* rec, int c8, const float (&A)[8], float M, float L) {
  if constexpr (COH) {
    uint64_t* p = (uint64_t*)(rec + 8 * c8);
#pragma unroll
    for (int i = 0; i < 4; ++i)
      __hip_atomic_store(p + i, pack_f2(A[2 * i], A[2 * i + 1]), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if (c8 == 0)
      __hip_atomic_store((uint64_t*)(rec + 128), pack_f2(M, L), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
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
// Only the first D channels exist (a slice of eight past D writes nothing,
// one straddling D writes its first D - 8 c8 elements).
template <class TT>
__device__ __forceinline__ void write_out(const DecodeArgs& a, int b, int hq, int c8, float L,
                                          const float (&A)[8]) {
  const int nv = min(a.D - 8 * c8, 8);
  if (nv <= 0) return;
  const float den = L + kDenomEps;
  if constexpr (TT::kBytes == 4) {
    float* dst = (float*)a.out + b * a.o_sb + (int64_t)hq * a.o_sh + 8 * c8 * a.o_sd;
    if (nv == 8 && a.o_sd == 1 && (((uintptr_t)dst) & 15) == 0) {
      ((float4*)dst)[0] = make_float4(A[0] / den, A[1] / den, A[2] / den, A[3] / den);
      ((float4*)dst)[1] = make_float4(A[4] / den, A[5] / den, A[6] / den, A[7] / den);
    } else {
#pragma unroll
      for (int e = 0; e < 8; ++e)
        if (e < nv) dst[e * a.o_sd] = A[e] / den;
    }
  } else {
    uint16_t o[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) o[e] = TT::from_f32(A[e] / den);
    uint16_t* dst = a.out + b * a.o_sb + (int64_t)hq * a.o_sh + 8 * c8 * a.o_sd;
    if (nv == 8 && a.o_sd == 1 && (((uintptr_t)dst) & 15) == 0) {
      *(uint4*)dst = pack8(o);
    } else {
#pragma unroll
      for (int e = 0; e < 8; ++e)
        if (e < nv) dst[e * a.o_sd] = o[e];
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
// record.  The workgroup waits until its record stores have completed,
// then takes a ticket on the unit's counter; the last of the unit's np
// workgroups merges the unit's records in the order of the merge kernel
// (merge_unit / merge_slice; the result is bit-identical to the two-launch
// merge).  No agent-scope release or acquire fence is needed, so no XCD L2
// is written back or invalidated.  With a fused append, the last unit of a
// batch row to finish advances len_full[b] behind a second ticket: by then
// every workgroup of the row has read it.
//
// Tickets are atomic increments that wrap to zero at n - 1 (the hardware's
// inc: old >= n - 1 ? 0 : old + 1), so the last arrival's increment is also
// the reset and every call leaves both counters at zero with no second
// store.  A counter holding anything else (a workspace that was never
// initialised) would misplace the merge, which is why the host initialises
// every workspace it has not seen before its first use.
//
// Records are written through to memory and read with coherent loads
// (COH), so the unit's workgroups may run on any XCDs.  What this relies
// on, on gfx942 / gfx950 (the only targets that compile it; the host never
// selects it elsewhere):
//   * relaxed agent-scope atomic stores compile to global stores with the
//     sc1 bit, which write through the XCD's L2 to the memory-side
//     coherence point, and relaxed agent-scope atomic loads to sc1 loads,
//     which read from that point, not from a possibly stale L2 line;
//   * vmcnt counts stores on these targets (there is no separate store
//     counter), so s_waitcnt vmcnt(0) returns only once the thread's
//     stores are acknowledged; the workgroup barrier then orders every
//     thread's completed stores before the ticket;
//   * agent-scope atomics on the ticket are performed at the coherence
//     point, so the workgroup that sees n - 1 is the last of the unit, and
//     its record loads, issued after the ticket returns (a dependency
//     through LDS and a barrier), see every other record;
//   * the signal fence keeps the compiler from moving the record stores
//     past the wait.
template <class TT, bool APPEND, int HMAX>
__device__ __forceinline__ void merge_fused(const DecodeArgs& a, int u, int b, int h0, int nh, int tid,
                                            float* s_mrg) {
#if defined(__gfx942__) || defined(__gfx950__) || !defined(__HIP_DEVICE_COMPILE__)
  __shared__ uint32_t s_ticket;
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
  __builtin_amdgcn_s_waitcnt(0);  // this thread's record stores have completed
  __syncthreads();                // ... and so have every thread's
  if (tid == 0) s_ticket = __builtin_amdgcn_atomic_inc32(a.ticket + u, (uint32_t)(a.np - 1), __ATOMIC_RELAXED, "agent");
  __syncthreads();
  if (s_ticket != (uint32_t)(a.np - 1)) return;
  // one query head per unit: one 16-lane slice (HMAX 1); else the unit's
  // heads over the workgroup
  if constexpr (HMAX == 1) {
    if (tid < 16) merge_slice<TT, true>(a, u, b, h0, tid);
  } else {
    merge_unit<TT, true>(a, u, b, h0, nh, tid, s_mrg);
  }
  if constexpr (APPEND) {
    if (tid == 0) {
      const uint32_t last = (uint32_t)(a.units_per_b - 1);
      if (__builtin_amdgcn_atomic_inc32(a.bticket + b, last, __ATOMIC_RELAXED, "agent") == last) {
        const int32_t pos = (int32_t)min(a.S_f, (int64_t)max(a.len_full[b], 0));
        if (pos < a.S_f) a.len_full[b] = pos + 1;
      }
    }
  }
#endif
}

// APPEND: fused append of k_new / v_new (span cache decode step); a
// separate instantiation so the plain decode carries none of its registers.
// NTL: V rows and compact visual Key rows use non-temporal loads (false for
// the grouped one-unit-per-query-head mode, whose G units of a KV head read
// each line through one XCD's L2).
// DPART (16-byte loads only): head_dim a.D < 128, a multiple of 8.  The
// lanes of channels past D load an in-bounds duplicate of channels D-8..D-1
// (V: only output channels past D see it, and those are not written; full
// K: zeroed before the score product), and q, R_partial's rows and
// delta_mu past D are zeros.  The element-wise kernels (VEC false) take any
// D: their loads past D are not issued and read as zeros.  With VEC and
// not DPART, D is 128 and none of this is compiled.
// FUSED (16-byte loads at head_dim 128 only): the single-launch merge
// (a.fused set).  A separate instantiation: inlined into every
// kernel, the merge's code raised the split pass's register pressure
// enough to spill scalar registers in its loops.
template <class TT, int DKB, bool VEC, int HMAX, bool HAS_VIS, bool APPEND, bool NTL = true, bool DPART = false,
          bool FUSED = false>
__global__ void __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(2)))
decode_kernel(const DecodeArgs a) {
  static_assert(!DPART || VEC, "the element-wise kernels mask head_dim at run time");
  static_assert(!FUSED || (VEC && !DPART), "the single-launch merge runs at head_dim 128 with 16-byte loads");
  constexpr bool kMaskD = DPART || !VEC;  // channels past a.D possible
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
  // channel tid & 127 of k_new (tid < 128) or v_new; past head_dim: zero, not stored
  const bool new_ch = !kMaskD || (tid & 127) < a.D;
  auto load_new = [&]() {
    if (has_new) {
      const int c = kMaskD ? min(tid & 127, a.D - 1) : tid & 127;
      new_raw = tid < 128 ? a.k_new[b * a.kn_sb + (int64_t)kv * a.kn_sh + (int64_t)c * a.kn_sd]
                          : a.v_new[b * a.vn_sb + (int64_t)kv * a.vn_sh + (int64_t)c * a.vn_sd];
    }
  };
  // after the staging barrier: the first unit of the KV head stores the row
  auto store_new = [&]() {
    if (has_new) {
      s_new[tid >> 7][tid & 127] = new_ch ? TT::to_f32(new_raw) : 0.f;
      if (jblk == 0 && new_ch) {
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
  // (fast layout with head_dim < 128: D is a multiple of 8, and the lanes of
  // channels past D re-read the row's last eight and are zeroed in store_q)
  const bool q_ch = !kMaskD || 8 * (tid & 15) < a.D;
  auto load_q = [&]() {
    if (a.q_vec) {
      const int h = min(tid >> 4, nh - 1);
      const int c0 = kMaskD ? min(8 * (tid & 15), a.D - 8) : 8 * (tid & 15);
      q16 = *(const uint4*)(a.q + b * a.q_sb + (int64_t)(h0 + h) * a.q_sh + c0);
    }
  };
  auto store_q = [&]() {
    if (!a.q_vec) {
#pragma unroll
      for (int k = 0; k < kQPer; ++k) {
        const int i = tid + k * kThreads;
        const int h = min(i >> 7, nh - 1), d = kMaskD ? min(i & 127, a.D - 1) : i & 127;
        qraw[k] = a.q[b * a.q_sb + (int64_t)(h0 + h) * a.q_sh + d * a.q_sd];
      }
    }
    if (a.q_vec) {
      const int h = tid >> 4;
      if (h < HMAX) {
        float f[8];
#pragma unroll
        for (int e = 0; e < 8; ++e)
          f[e] = h < nh && q_ch ? TT::to_f32((uint16_t)(word(q16, e >> 1) >> ((e & 1) * 16))) : 0.f;
        float4* dst = (float4*)&s_q[h][8 * (tid & 15)];
        dst[0] = make_float4(f[0], f[1], f[2], f[3]);
        dst[1] = make_float4(f[4], f[5], f[6], f[7]);
      }
    } else {
#pragma unroll
      for (int k = 0; k < kQPer; ++k) {
        const int i = tid + k * kThreads;
        qv[k] = (i < HMAX * 128 && (i >> 7) < nh && (!kMaskD || (i & 127) < a.D)) ? TT::to_f32(qraw[k]) : 0.f;
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
    // V channel slot of this lane: past head_dim, the row's last eight (with
    // 16-byte loads; they feed only output channels that are not written),
    // or no load at all (element-wise)
    const uint32_t vch = DPART ? (uint32_t)min(8 * n, a.D - 8) : 8u * n;
    const int vnv = kMaskD ? max(min(a.D - 8 * n, 8), 0) : 8;
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
        B.v[r] = load_row8b<VEC, NTL>(vsb, min(vro + vb0 + (uint32_t)r * vss2, vlast), VEC ? 0u : vch, a.vs_sd, vnv);
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
    const int nchunks = kMaskD ? (a.D * a.Dk) >> 3 : 16 * a.Dk;  // [D][Dk] 16-bit elements in 16-byte chunks
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
      const int64_t di = b * a.dm_sb + kv * a.dm_sh + (int64_t)(kMaskD ? min(tid & 127, a.D - 1) : tid & 127) * a.dm_sd;
      dmraw = a.dm_dtype == 2 ? ((const uint32_t*)a.dm)[di] : (uint32_t)((const uint16_t*)a.dm)[di];
    }

    const float dmv = (tid < 128 && a.has_bias && (!kMaskD || tid < a.D)) ? raw_to_f32(dmraw, a.dm_dtype) : 0.f;
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
          for (int e = 0; e < 8; ++e) rb[e] = !kMaskD || k0 + e < a.D ? rc[(k0 + e) * a.Dk] : (uint16_t)0;
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
        for (int i = 0; i < kL; ++i) rv[i] = c < a.Dk && (!kMaskD || part * kL + i < a.D) ? rv[i] : 0.f;
      } else {  // element-wise fallback (column c, clamped in-bounds; no load
                // at all when Dk == 0, where R_partial has no storage)
#pragma unroll
        for (int i = 0; i < kL; ++i) rv[i] = 0.f;
        if (a.Dk > 0) {
          const int64_t rb = b * a.R_sb + kv * a.R_sh + (int64_t)min(c, a.Dk - 1) * a.R_sk;
          if constexpr (kMaskD)
            load_any_rows(a.R, rb, a.R_sd, a.r_dtype, part * kL, a.D, rv);
          else  // all 128 rows: addresses stepped on the fly
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

    // q R as a 16-bit hi + lo pair (the score operand).  An entry of 2^15 or
    // more (fp16 ends at 65504; queries of order 10^4) would overflow the
    // hi part: then the pair is formed again from q R scaled by 2^-qsh, and
    // the score multiplier takes 2^qsh.  The scaling is exact, so the scores
    // equal the unsplit fp32 ones the reference's paper kernel computes
    // (fused_decode.py:133-139, 166-167).  The unit's largest entry sets qsh
    // (every wave sees every head and kept channel): one scalar per wave,
    // and one vote on the common path.
    uint4 qh[DKB], ql[DKB];
    float qmax = 0.f;
    auto split_q = [&](float qscale) {
#pragma unroll
      for (int kb = 0; kb < DKB; ++kb) {
        uint16_t hv[8], lv[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const float v = (n < HMAX) ? s_qt[nq][kb * 32 + 8 * g + e] : 0.f;
          qmax = fmaxf(qmax, fabsf(v));
          TT::split(v * qscale, hv[e], lv[e]);
        }
        qh[kb] = pack8(hv);
        ql[kb] = pack8(lv);
      }
    };
    split_q(1.f);
    float sl2 = a.scale_log2;
    if (__builtin_amdgcn_ballot_w64(qmax >= 32768.f) != 0) {  // wave-uniform
#pragma unroll
      for (int off = 1; off < 64; off <<= 1) qmax = fmaxf(qmax, shfl_xor(qmax, off));
      int qexp = 0;
      (void)frexpf(qmax, &qexp);  // qmax < 2^qexp
      const int qsh = __builtin_amdgcn_readfirstlane(qmax < INFINITY && qexp > 15 ? qexp - 15 : 0);
      split_q(ldexpf(1.f, -qsh));
      sl2 = __builtin_bit_cast(float,
                               __builtin_amdgcn_readfirstlane(__builtin_bit_cast(int, ldexpf(a.scale_log2, qsh))));
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
          s[4 * sb + i] = (8 * g + 4 * sb + i < lim) ? fmaf(cc[i], sl2, bias2) : -INFINITY;
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
    // channel slots past head_dim: V as in the visual path; K loads an
    // in-bounds duplicate that is zeroed before the score (16-byte loads),
    // or nothing (element-wise)
    const uint32_t vch = DPART ? (uint32_t)min(8 * n, a.D - 8) : 8u * n;
    const int vnv = kMaskD ? max(min(a.D - 8 * n, 8), 0) : 8;
    uint32_t fch[4];
    int fnv[4];
    bool fval[4];
#pragma unroll
    for (int kb = 0; kb < 4; ++kb) {
      const int c0 = kb * 32 + 8 * g;
      fch[kb] = DPART ? (uint32_t)min(c0, a.D - 8) : (uint32_t)c0;
      fnv[kb] = kMaskD ? max(min(a.D - c0, 8), 0) : 8;
      fval[kb] = c0 < a.D;
    }
    const int64_t nblk = (t_end - t_begin + kBlk - 1) / kBlk;
    auto load = [&](FullBuf& B, int64_t blk) {
      const uint32_t t0 = (uint32_t)(t_begin + blk * kBlk);
      const uint32_t r0 = min(t0 + krow0, t_last) * a.kf_ss, r1 = min(t0 + krow1, t_last) * a.kf_ss;
#pragma unroll
      for (int kb = 0; kb < 4; ++kb) {
        B.k[0][kb] = load_row8<VEC, false>(kfb, r0, fch[kb], a.kf_sd, fnv[kb]);
        B.k[1][kb] = load_row8<VEC, false>(kfb, r1, fch[kb], a.kf_sd, fnv[kb]);
      }
#pragma unroll
      for (int r = 0; r < 8; ++r) {
        uint32_t row = min(t0 + 8u * g + r, t_last);
        row += row >= a.vf_gap_at ? a.vf_gap : 0u;
        B.v[r] = load_row8<VEC, NTL>(vfb, row * a.vf_ss, vch, a.vf_sd, vnv);
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
        for (int kb = 0; kb < 4; ++kb) cc = TT::mfma(DPART ? zero_if(fval[kb], B.k[sb][kb]) : B.k[sb][kb], qf[kb], cc);
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
      store_rec<FUSED>(rec, c8, A, M, L);
    }
  }
  if constexpr (FUSED) merge_fused<TT, APPEND, HMAX>(a, u, b, h0, nh, tid, HMAX >= 16 ? &s_acc[0][0][0] : (float*)s_rsep);
}

// ---- fp32 decode (q, K, V and out in F32; R_partial and delta_mu F16,
// BF16 or F32), the dtype of the reference's CPU-scale configuration.  The
// reference kernels load any float input as fp32 and compute in fp32
// (fused_decode.py:133,166,174; full_channel_flash_decoding.py:65,84,92);
// so do these kernels, on the VALU: fp32 has no MFMA path that keeps its
// precision at this arithmetic intensity.  Plan, grid and records are the
// 16-bit kernel's, so both merges apply.  Each wave walks 64-token blocks
// of its workgroup's chunk (blocks wave, wave + 4, ...): lane t scores
// token t0 + t as a dot product over its row, the wave runs the online
// softmax (log2 domain), and lane j accumulates channels 2j, 2j + 1 of
// P V over the block's rows, with the block's probabilities broadcast
// from LDS.
//   decode32_kernel   one query head per unit (G = 1, or the paper
//                     family's dense baseline);
//   decode32g_kernel  up to HG = 8 query heads of one KV head per unit (the
//                     grouped decomposition, gqa_decode.py:121-210): each
//                     K and V row is loaded once and serves every head (one
//                     online softmax per head).  A separate kernel: folded
//                     into one template with the one-head case, the
//                     one-head instantiations compiled to fewer registers
//                     and fewer loads in flight, and config 0 ran 9 % (the
//                     dense baseline 29 %) slower.
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

// DFULL: head_dim 128, a compile-time constant (the run-time bound cost the
// full-row dot product its loads in flight and spilled scalar registers in
// the loop: config 0 18.8 -> 20.5 us, its dense baseline 20.9 -> 26.8 us).
template <bool HAS_VIS, bool VEC, bool DFULL>
__global__ void __launch_bounds__(kThreads) decode32_kernel(const DecodeArgs a) {
  const int D = DFULL ? 128 : a.D;
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

  // channels past head_dim D are zeros (q, R_partial's rows, delta_mu);
  // V lanes past D read an in-bounds duplicate (16-byte rows: the row's last
  // two channels; else no load) that feeds only output channels not written
  if (tid < 128) s_q[tid] = tid < D ? q[b * a.q_sb + (int64_t)h0 * a.q_sh + (int64_t)tid * a.q_sd] : 0.f;
  __syncthreads();
  const int vc = min(2 * lane, D - 2);  // (VEC: D is a multiple of 4)
  const bool v0ok = 2 * lane < D, v1ok = 2 * lane + 1 < D;

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
          const float2 v = *(const float2*)(vr + vc);
          v0[jj] = v.x;
          v1[jj] = v.y;
        } else {
          v0[jj] = v0ok ? vr[(int64_t)(2 * lane) * vsd] : 0.f;
          v1[jj] = v1ok ? vr[(int64_t)(2 * lane + 1) * vsd] : 0.f;
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
        if constexpr (DFULL)  // all 128 rows: addresses stepped on the fly
          load_any_n(a.R, rb + (int64_t)(64 * half) * a.R_sd, a.R_sd, a.r_dtype, rv);
        else
          load_any_rows(a.R, rb, a.R_sd, a.r_dtype, 64 * half, D, rv);
#pragma unroll
        for (int i = 0; i < 64; ++i) sum = fmaf(s_q[64 * half + i], rv[i], sum);
      }
      s_acc[half][c] = sum;  // s_acc is free until the epilogue
      __syncthreads();
      if (tid < 128) s_qt[tid] = tid < a.Dk ? s_acc[0][tid] + s_acc[1][tid] : 0.f;
    }
    if (wave < 2) {  // q . delta_mu
      const int d = tid;
      const float t = a.has_bias && d < D
                          ? s_q[d] * load_any(a.dm, b * a.dm_sb + kv * a.dm_sh + (int64_t)d * a.dm_sd, a.dm_dtype)
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
      const float d = dot_row32<VEC, 128>(kfb + tc * a.kf_ss, a.kf_sd, s_q, D);
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
  if (a.fused) merge_fused<F32, false, 1>(a, u, b, h0, 1, tid, s_mrg);
}

// d[h] = sum_c w[h * 128 + c] * row[c * sd] for the heads h < nh, c < n <=
// KMAX; w in LDS.  VEC: unit stride, 16-byte aligned row, n a multiple of
// 4: all KMAX / 4 16-byte loads are issued before any is used (those past
// n re-read the row's last four floats, in bounds, and are not used), so
// the row costs one memory round trip; float4 i accumulates into the even
// (i even) or odd partial sum of each head.
template <bool VEC, int KMAX, int HG>
__device__ __forceinline__ void dot_rows32(const float* row, uint32_t sd, const float* w, int n, int nh,
                                           float (&d)[HG]) {
  float s0[HG], s1[HG];
#pragma unroll
  for (int h = 0; h < HG; ++h) s0[h] = s1[h] = 0.f;
  if constexpr (VEC) {
    if (n > 0) {
      float4 r[KMAX / 4];
#pragma unroll
      for (int i = 0; i < KMAX / 4; ++i) r[i] = *(const float4*)(row + min(4 * i, n - 4));
#pragma unroll
      for (int i = 0; i < KMAX / 4; ++i) {
        if (4 * i < n) {
#pragma unroll
          for (int h = 0; h < HG; ++h) {
            if (h < nh) {
              const float4 w4 = *(const float4*)(w + h * 128 + 4 * i);
              float& acc = (i & 1) ? s1[h] : s0[h];
              acc = fmaf(w4.x, r[i].x, acc);
              acc = fmaf(w4.y, r[i].y, acc);
              acc = fmaf(w4.z, r[i].z, acc);
              acc = fmaf(w4.w, r[i].w, acc);
            }
          }
        }
      }
    }
  } else {
    for (int c = 0; c < n; ++c) {
      const float x = row[(int64_t)c * sd];
#pragma unroll
      for (int h = 0; h < HG; ++h)
        if (h < nh) s0[h] = fmaf(w[h * 128 + c], x, s0[h]);
    }
  }
#pragma unroll
  for (int h = 0; h < HG; ++h) d[h] = s0[h] + s1[h];
}

template <bool HAS_VIS, bool VEC, int HG, bool DFULL>
__global__ void __launch_bounds__(kThreads) decode32g_kernel(const DecodeArgs a) {
  const int D = DFULL ? 128 : a.D;  // head_dim (DFULL: 128, as in decode32_kernel)
  __shared__ __attribute__((aligned(16))) float s_q[HG][128];
  __shared__ __attribute__((aligned(16))) float s_qt[HG][128];
  __shared__ float s_bias[HG][2];
  __shared__ float s_p[kWaves][HG][kBlk32];
  __shared__ float s_m[kWaves][HG], s_l[kWaves][HG];
  __shared__ float s_acc[kWaves][HG][128];
  __shared__ float s_mrg[16 * kRecFloats];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int u = blockIdx.y, x = blockIdx.x;
  const int b = u / a.units_per_b;
  const int r_in_b = u - b * a.units_per_b;
  const int kv = r_in_b / a.spk;
  const int jblk = r_in_b - kv * a.spk;
  const int h0 = kv * a.G + jblk * a.hpu;
  const int nh = HG == 1 ? 1 : min(a.hpu, a.G - jblk * a.hpu);  // this unit's query heads
  const bool is_vis = HAS_VIS && x < a.wg_vis;
  const int xf = HAS_VIS ? x - a.wg_vis : x;
  const float* q = (const float*)a.q;

  // channels past head_dim D are zeros (q, R_partial's rows, delta_mu);
  // V lanes past D read an in-bounds duplicate (16-byte rows: the row's last
  // two channels; else no load) that feeds only output channels not written;
  // rows of absent heads (h >= nh) are zeros
  for (int i = tid; i < HG * 128; i += kThreads) {
    const int h = i >> 7, c = i & 127;
    (&s_q[0][0])[i] = h < nh && c < D ? q[b * a.q_sb + (int64_t)(h0 + h) * a.q_sh + (int64_t)c * a.q_sd] : 0.f;
  }
  __syncthreads();
  const int vc = min(2 * lane, D - 2);  // (VEC: D is a multiple of 4)
  const bool v0ok = 2 * lane < D, v1ok = 2 * lane + 1 < D;

  float m[HG], l[HG], acc0[HG], acc1[HG];
#pragma unroll
  for (int h = 0; h < HG; ++h) {
    m[h] = kNegInit;
    l[h] = acc0[h] = acc1[h] = 0.f;
  }
  // online-softmax step over one block: s[h] = log2-domain score of token
  // t0 + lane for head h (-inf when invalid), V rows clamped to t_last
  auto step = [&](const float (&s)[HG], const float* vb, uint32_t vss, uint32_t vsd, int64_t t0, int64_t t_last,
                  uint32_t gap_at, uint32_t gap) {
#pragma unroll
    for (int h = 0; h < HG; ++h) {
      if (h < nh) {
        const float m_new = fmaxf(m[h], wave_max(s[h]));
        const float alpha = fast_exp2(m[h] - m_new);
        const float p = fast_exp2(s[h] - m_new);
        l[h] = l[h] * alpha + wave_sum(p);
        acc0[h] *= alpha;
        acc1[h] *= alpha;
        m[h] = m_new;
        s_p[wave][h][lane] = p;
      }
    }
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
          const float2 v = *(const float2*)(vr + vc);
          v0[jj] = v.x;
          v1[jj] = v.y;
        } else {
          v0[jj] = v0ok ? vr[(int64_t)(2 * lane) * vsd] : 0.f;
          v1[jj] = v1ok ? vr[(int64_t)(2 * lane + 1) * vsd] : 0.f;
        }
      }
#pragma unroll
      for (int h = 0; h < HG; ++h) {
        if (h < nh) {
#pragma unroll
          for (int jj = 0; jj < kVB; ++jj) {
            const float pj = s_p[wave][h][j0 + jj];
            acc0[h] = fmaf(pj, v0[jj], acc0[h]);
            acc1[h] = fmaf(pj, v1[jj], acc1[h]);
          }
        }
      }
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  };

  if (is_vis) {
    {  // q R_partial: thread (half, c) sums rows 64 half .. 64 half + 63 of
       // column c for every head, all 64 loads in flight; the halves meet
       // in LDS
      const int c = tid & 127, half = tid >> 7;
      const int cc = min(c, max(a.Dk - 1, 0));
      const int64_t rb = b * a.R_sb + kv * a.R_sh + (int64_t)cc * a.R_sk;
      float sum[HG];
#pragma unroll
      for (int h = 0; h < HG; ++h) sum[h] = 0.f;
      if (a.Dk > 0) {
        float rv[64];
        if constexpr (DFULL)  // all 128 rows: addresses stepped on the fly
          load_any_n(a.R, rb + (int64_t)(64 * half) * a.R_sd, a.R_sd, a.r_dtype, rv);
        else
          load_any_rows(a.R, rb, a.R_sd, a.r_dtype, 64 * half, D, rv);
#pragma unroll
        for (int h = 0; h < HG; ++h)
          if (h < nh) {
#pragma unroll
            for (int i = 0; i < 64; ++i) sum[h] = fmaf(s_q[h][64 * half + i], rv[i], sum[h]);
          }
      }
#pragma unroll
      for (int h = 0; h < HG; ++h) s_acc[half][h][c] = sum[h];  // s_acc is free until the epilogue
      __syncthreads();
      for (int i = tid; i < HG * 128; i += kThreads) {
        const int h = i >> 7, c2 = i & 127;
        (&s_qt[0][0])[i] = c2 < a.Dk ? s_acc[0][h][c2] + s_acc[1][h][c2] : 0.f;
      }
    }
    if (wave < 2) {  // q . delta_mu, every head of the unit
      const int d = tid;
      const float dm = a.has_bias && d < D
                           ? load_any(a.dm, b * a.dm_sb + kv * a.dm_sh + (int64_t)d * a.dm_sd, a.dm_dtype)
                           : 0.f;
#pragma unroll
      for (int h = 0; h < HG; ++h) {
        if (h < nh) {
          const float w = wave_sum(s_q[h][d] * dm);
          if (lane == 0) s_bias[h][wave] = w;
        }
      }
    }
    __syncthreads();
    float bias2[HG];
#pragma unroll
    for (int h = 0; h < HG; ++h) bias2[h] = h < nh ? (s_bias[h][0] + s_bias[h][1]) * a.scale_log2 : 0.f;
    const int64_t t_begin = (int64_t)x * a.chunk_vis;
    const int64_t t_end = min(a.S_v, t_begin + a.chunk_vis);
    const float* ksb = (const float*)a.ks + b * a.ks_sb + kv * a.ks_sh;
    const float* vsb = (const float*)a.vs + b * a.vs_sb + kv * a.vs_sh;
    for (int64_t t0 = t_begin + (int64_t)wave * kBlk32; t0 < t_end; t0 += kWaves * kBlk32) {
      const int64_t t = t0 + lane;
      const float* kr = ksb + (int64_t)min(t, t_end - 1) * a.ks_ss;
      float d[HG], sc[HG];
      if (a.Dk <= 32)
        dot_rows32<VEC, 32, HG>(kr, a.ks_sd, &s_qt[0][0], a.Dk, nh, d);
      else if (a.Dk <= 64)
        dot_rows32<VEC, 64, HG>(kr, a.ks_sd, &s_qt[0][0], a.Dk, nh, d);
      else
        dot_rows32<VEC, 128, HG>(kr, a.ks_sd, &s_qt[0][0], a.Dk, nh, d);
#pragma unroll
      for (int h = 0; h < HG; ++h) sc[h] = t < t_end ? fmaf(d[h], a.scale_log2, bias2[h]) : -INFINITY;
      step(sc, vsb, a.vs_ss, a.vs_sd, t0, t_end - 1, UINT32_MAX, 0u);
    }
  } else {
    const int64_t t_begin = (int64_t)xf * a.chunk_full;
    const int64_t t_end = min(a.S_f, t_begin + a.chunk_full);
    const float* kfb = (const float*)a.kf + b * a.kf_sb + kv * a.kf_sh;
    const float* vfb = (const float*)a.vf + b * a.vf_sb + kv * a.vf_sh;
    for (int64_t t0 = t_begin + (int64_t)wave * kBlk32; t0 < t_end; t0 += kWaves * kBlk32) {
      const int64_t t = t0 + lane;
      const int64_t tc = min(t, t_end - 1);
      float d[HG], sc[HG];
      dot_rows32<VEC, 128, HG>(kfb + tc * a.kf_ss, a.kf_sd, &s_q[0][0], D, nh, d);
      const bool ok = t < t_end && (!a.mask || a.mask[b * a.mf_sb + tc * a.mf_ss] != 0);
#pragma unroll
      for (int h = 0; h < HG; ++h) sc[h] = ok ? d[h] * a.scale_log2 : -INFINITY;
      step(sc, vfb, a.vf_ss, a.vf_sd, t0, t_end - 1, a.vf_gap_at, a.vf_gap);
    }
  }

  // the four wave states of each head -> this workgroup's records
#pragma unroll
  for (int h = 0; h < HG; ++h) {
    if (h < nh) {
      if (lane == 0) {
        s_m[wave][h] = m[h];
        s_l[wave][h] = l[h];
      }
      s_acc[wave][h][2 * lane] = acc0[h];
      s_acc[wave][h][2 * lane + 1] = acc1[h];
    }
  }
  __syncthreads();
  if (tid < 16 * nh) {
    const int h = tid >> 4, c8 = tid & 15;
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
  if (a.fused) merge_fused<F32, false, HG>(a, u, b, h0, nh, tid, s_mrg);
}

// Second launch: one workgroup per unit runs merge_unit, or with one query
// head per unit (hpu == 1) one workgroup per 16 units, a slice each
// (merge_slice).  With a fused append the unit holding query head 0 of row
// b advances len_full[b]; the split launch that read it has completed.  Its
// read is issued before the merge's loads, so its latency overlaps them
// (nothing else writes len_full[b] during this launch).
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
  // (every thread reads it under the launch-uniform k_new: a read under the
  // per-thread condition below would wait for its data on the spot; the
  // empty asm after the merge keeps any use of the value, and so its wait,
  // behind the merge)
  int32_t len0 = a.k_new ? a.len_full[b] : 0;
  const bool advance = a.k_new && r_in_b == 0 && (tid & (sliced ? 15 : 255)) == 0;
  if (sliced)
    merge_slice<TT, false>(a, u, b, h0, tid & 15);
  else
    merge_unit<TT, false>(a, u, b, h0, min(a.hpu, a.G - jblk * a.hpu), tid, s_mrg);
  asm volatile("" : "+v"(len0));
  if (advance) {
    const int32_t pos = (int32_t)min(a.S_f, (int64_t)max(len0, 0));
    if (pos < a.S_f) a.len_full[b] = pos + 1;
  }
}

// ---- host-side launch templates (instantiated per dtype by the launch units)

template <class TT, int DKB, bool VEC, int HMAX, bool HAS_VIS, bool DPART>
hipError_t launch_one(const DecodeArgs& a, dim3 grid, hipStream_t s) {
  // the single-launch merge is compiled into the 16-byte kernels at head_dim
  // 128 only (the host selects it nowhere else)
  constexpr bool kCanFuse = VEC && !DPART;
  if (a.fused && !kCanFuse) return hipErrorInvalidValue;
  bool launched = false;
  // grouped one-unit-per-query-head mode (temporal loads): the dense
  // baseline's paper family at G > 1 only (the RotateK entries run that
  // family grouped, see rotatek_policy)
  if constexpr (VEC && HMAX == 1 && !HAS_VIS) {
    if (a.xgroup > 1) {
      if (a.fused)
        hipLaunchKernelGGL((decode_kernel<TT, DKB, VEC, HMAX, HAS_VIS, false, false, DPART, kCanFuse>), grid,
                           dim3(kThreads), 0, s, a);
      else
        hipLaunchKernelGGL((decode_kernel<TT, DKB, VEC, HMAX, HAS_VIS, false, false, DPART>), grid,
                           dim3(kThreads), 0, s, a);
      launched = true;
    }
  }
  if constexpr (HAS_VIS) {  // the span cache's step always carries the visual span
    if (!launched && a.k_new) {
      if (a.fused)
        hipLaunchKernelGGL((decode_kernel<TT, DKB, VEC, HMAX, true, true, true, DPART, kCanFuse>), grid,
                           dim3(kThreads), 0, s, a);
      else
        hipLaunchKernelGGL((decode_kernel<TT, DKB, VEC, HMAX, true, true, true, DPART>), grid, dim3(kThreads),
                           0, s, a);
      launched = true;
    }
  }
  if (!launched) {
    if (a.fused)
      hipLaunchKernelGGL((decode_kernel<TT, DKB, VEC, HMAX, HAS_VIS, false, true, DPART, kCanFuse>), grid,
                         dim3(kThreads), 0, s, a);
    else
      hipLaunchKernelGGL((decode_kernel<TT, DKB, VEC, HMAX, HAS_VIS, false, true, DPART>), grid, dim3(kThreads),
                         0, s, a);
  }
  hipError_t e = hipGetLastError();
  if (e != hipSuccess || a.fused) return e;
  hipLaunchKernelGGL((merge_kernel<TT>), dim3(merge_grid(a)), dim3(kThreads), 0, s, a);
  return hipGetLastError();
}

template <class TT, int DKB, bool VEC, int HMAX, bool DPART>
hipError_t launch_vis(bool has_vis, const DecodeArgs& a, dim3 grid, hipStream_t s) {
  return has_vis ? launch_one<TT, DKB, VEC, HMAX, true, DPART>(a, grid, s)
                 : launch_one<TT, 1, VEC, HMAX, false, DPART>(a, grid, s);
}

template <class TT, int DKB, bool VEC, bool DPART>
hipError_t launch_h(int hmax, bool has_vis, const DecodeArgs& a, dim3 grid, hipStream_t s) {
  return hmax > 1 ? launch_vis<TT, DKB, VEC, 16, DPART>(has_vis, a, grid, s)
                  : launch_vis<TT, DKB, VEC, 1, DPART>(has_vis, a, grid, s);
}

// DPART: 16-byte loads at head_dim < 128 (vec must be true)
template <class TT, int DKB, bool DPART>
hipError_t launch_v(bool vec, int hmax, bool has_vis, const DecodeArgs& a, dim3 grid,
                    hipStream_t s) {
  if constexpr (DPART) return launch_h<TT, DKB, true, true>(hmax, has_vis, a, grid, s);
  return vec ? launch_h<TT, DKB, true, false>(hmax, has_vis, a, grid, s)
             : launch_h<TT, DKB, false, false>(hmax, has_vis, a, grid, s);
}

template <class TT, bool DPART = false>
hipError_t launch_dk(int dkb, bool vec, int hmax, bool has_vis, const DecodeArgs& a, dim3 grid,
                     hipStream_t s) {
  switch (dkb) {
    case 1: return launch_v<TT, 1, DPART>(vec, hmax, has_vis, a, grid, s);
    case 2: return launch_v<TT, 2, DPART>(vec, hmax, has_vis, a, grid, s);
    default: return launch_v<TT, 4, DPART>(vec, hmax, has_vis, a, grid, s);
  }
}

}  // namespace rk
