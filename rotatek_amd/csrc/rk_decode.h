// rk_decode.h -- what the decode host code and the per-dtype kernel
// translation units share: the kernel argument block, the launch geometry
// constants and the per-dtype launchers (rk_decode_f16.hip,
// rk_decode_bf16.hip, rk_decode_f32.hip; each compiles its dtype's kernel
// instantiations, so the three build in parallel).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

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
  // 0: merge kernel; 1: single launch (merge_fused)
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
  // head_dim (1..128): channels >= D of q, K, V, R_partial's rows and
  // delta_mu do not exist; the kernels treat them as zeros (the reference's
  // masked BLOCK_D loads) and write only the first D output channels
  int32_t D;
  float scale_log2;  // log2(e) / sqrt(D)
};

constexpr int kThreads = 256;
constexpr int kWaves = 4;
constexpr int kBlk = 32;
constexpr int kMaskChunk = 4096;  // max prompt+text tokens per workgroup
constexpr int kRecFloats = 160;   // partial record: acc[128], m, l; 640 B = five 128-byte lines

// Split launch (and, unless a.fused, the merge launch) of one decode step
// for 16-bit q / K / V: dkb = ceil(Dk / 32) rounded to 1, 2 or 4; vec = 16-byte
// row loads; hmax > 1 = units of up to 16 query heads; has_vis = the visual
// span is present.
hipError_t decode_launch_f16(int dkb, bool vec, int hmax, bool has_vis, const DecodeArgs& a, dim3 grid,
                             hipStream_t s);
hipError_t decode_launch_bf16(int dkb, bool vec, int hmax, bool has_vis, const DecodeArgs& a, dim3 grid,
                              hipStream_t s);
// The same with 16-byte row loads for head_dim < 128 (a multiple of 8): the
// instantiations that mask the channels past D (rk_decode_{f16,bf16}_hd.hip).
// The element-wise kernels (vec false) take any head_dim in the ones above.
hipError_t decode_launch_f16_hd(int dkb, int hmax, bool has_vis, const DecodeArgs& a, dim3 grid, hipStream_t s);
hipError_t decode_launch_bf16_hd(int dkb, int hmax, bool has_vis, const DecodeArgs& a, dim3 grid, hipStream_t s);
// The same for fp32 q / K / V (the VALU kernel, one query head per unit).
hipError_t decode_launch_f32(bool has_vis, bool vec, const DecodeArgs& a, dim3 grid, hipStream_t s);

// Workgroups of the merge kernel: one per unit, or one per 16 units of one
// query head each (merge_kernel's sliced form).
inline unsigned merge_grid(const DecodeArgs& a) {
  return (unsigned)(a.hpu == 1 ? (a.units + 15) / 16 : a.units);
}

}  // namespace rk
