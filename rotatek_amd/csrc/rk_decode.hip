// rk_decode.hip -- host side of the fused split-K RotateK decode (MI355X,
// gfx950): the split planner, argument validation, the C ABI entry points
// (include/rotatek_hip.h), the span-cache append kernel and the
// allocation-free entry point.  The kernels themselves are in
// rk_decode_dev.h, compiled per dtype by rk_decode_{f16,bf16,f32}.hip.
#include <math.h>
#include <stdlib.h>
#include <string.h>

#include <atomic>
#include <mutex>
#include <unordered_set>

#include "rk_common.h"
#include "rk_decode.h"
#include "rk_host.h"
#include "rotatek_hip.h"

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

// The ticket region (fixed size, at offset 0) holds two arrays at fixed
// offsets, whatever the shape: unit tickets, then batch-row tickets (every
// call leaves both at zero).  Then one partial record per (unit, workgroup,
// head).
constexpr int64_t kTicketWords = RK_DECODE_TICKET_BYTES / sizeof(uint32_t);
constexpr int64_t kMaxTicketUnits = kTicketWords * 3 / 4;            // 49152
constexpr int64_t kMaxTicketRows = kTicketWords - kMaxTicketUnits;  // 16384

WsLayout ws_layout(const rk_decode_plan& p) {
  const int64_t np = p.wg_vis + p.wg_full;
  const size_t parts = (size_t)p.units * np * p.heads_per_unit;
  WsLayout w;
  w.ticket = 0;
  w.bticket = (size_t)kMaxTicketUnits * sizeof(uint32_t);
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
// two rounds: 44.2 -> 44.8 us).  Records passed through one XCD's L2
// instead of memory (chunk-major grids put all of a unit's workgroups on
// one XCD when units % 8 == 0; group-scope stores and loads) measured
// slower still: config 1 33.6 against 32.1 us (graph), 28 config 4 layers at
// 4097 visual tokens 562 against 548 us per step (keep 32, two launches).
bool use_single_launch(const rk_decode_plan& p, int64_t B, int cus, const Knobs& k) {
  if (p.units > kMaxTicketUnits || B > kMaxTicketRows) return false;
  if (k.merge_mode != 0) return k.merge_mode == 2;
  return p.heads_per_unit == 1 && p.grid <= (int64_t)cus * k.resident();
}

}  // namespace

namespace {

__global__ void __launch_bounds__(256) zero_words_kernel(uint32_t* p, int64_t n) {
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x)
    p[i] = 0u;
}

// Workspaces whose ticket region has been zeroed (rk_decode_workspace_init,
// or a decode entry's first single-launch use of a workspace it had not
// seen).  Every call leaves the counters at zero, so a registered
// workspace stays ready; rk_decode_workspace_release forgets one.
std::mutex g_ws_mu;
std::unordered_set<uintptr_t> g_ws_ready;

void mark_ready(void* ws, bool ready) {
  std::lock_guard<std::mutex> lock(g_ws_mu);
  if (ready)
    g_ws_ready.insert((uintptr_t)ws);
  else
    g_ws_ready.erase((uintptr_t)ws);
}

bool is_ready(void* ws) {
  std::lock_guard<std::mutex> lock(g_ws_mu);
  return g_ws_ready.count((uintptr_t)ws) != 0;
}

}  // namespace

extern "C" int rk_decode_workspace_init(void* workspace, size_t workspace_bytes, void* stream) {
  if (!workspace) return RK_ERR_NULL;
  if ((((uintptr_t)workspace) & 255) != 0) return RK_ERR_WORKSPACE;
  const size_t n = (workspace_bytes < RK_DECODE_TICKET_BYTES ? workspace_bytes : RK_DECODE_TICKET_BYTES) / 4;
  if (n == 0) return RK_OK;
  hipLaunchKernelGGL(zero_words_kernel, dim3(64), dim3(256), 0, (hipStream_t)stream, (uint32_t*)workspace,
                     (int64_t)n);
  if (hipGetLastError() != hipSuccess) return RK_ERR_HIP;
  // under stream capture the fill only runs when the graph is replayed (and
  // then before every replay's decode), so the address is not marked: the
  // next eager call initialises it again
  hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
  if (hipStreamIsCapturing((hipStream_t)stream, &cs) != hipSuccess) return RK_ERR_HIP;
  if (n * 4 == RK_DECODE_TICKET_BYTES && cs == hipStreamCaptureStatusNone) mark_ready(workspace, true);
  return RK_OK;
}

extern "C" void rk_decode_workspace_release(void* workspace) {
  if (workspace) mark_ready(workspace, false);
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
    // blocks of up to 16 query heads (fp32, the VALU kernel: 8) per unit
    const int64_t hmax = elem_bytes == 4 ? 8 : 16;
    p.heads_per_unit = (int32_t)(G < hmax ? G : hmax);
    p.head_blocks = (int32_t)cdiv(G, hmax);
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
  int64_t B, H_q, H_kv, G, D, Dk, S_v, S_f;
  int dtype;
};

// A [B, H, S, D] K/V descriptor the kernels can address: the whole
// within-head span, plus 32 rows, below 2^31 elements (kernel offsets are
// 32-bit byte offsets; the visual ring adds a block's row offsets to its
// first row before clamping to the chunk's last row) and the token stride
// below 2^26.
bool head_span_ok(const rk_tensor* t) {
  const int64_t span = (t->shape[2] > 0 ? (t->shape[2] - 1 + 32) * t->stride[2] : 0) +
                       (t->shape[3] > 0 ? (t->shape[3] - 1) * t->stride[3] : 0) + 8;
  return span < (INT64_C(1) << 31) && t->stride[2] < (INT64_C(1) << 26) && t->stride[3] < (INT64_C(1) << 31);
}

int check_out(const rk_tensor* out, const Checked& c) {
  int st = rk::check_desc(out, 3);
  if (st) return st;
  if (out->dtype != c.dtype) return RK_ERR_DTYPE;
  if (out->shape[0] != c.B || out->shape[1] != c.H_q || out->shape[2] != c.D) return RK_ERR_SHAPE;
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
  c->D = q->shape[2];
  c->Dk = R->shape[3];
  c->dtype = q->dtype;
  if (c->H_q / G != c->H_kv || c->H_q % G != 0) return RK_ERR_HEADS;
  if (!rk::is_half(q->dtype) && q->dtype != RK_F32) return RK_ERR_DTYPE;
  // any head size up to 128 (the reference pads D to a power-of-two block
  // with a channel mask, fused_decode.py:128, 341-342)
  if (c->D < 1 || c->D > 128) return RK_ERR_HEAD_DIM;
  if (!rk::is_float_param(R->dtype)) return RK_ERR_DTYPE;
  if (R->shape[0] != c->B || R->shape[2] != c->D) return RK_ERR_SHAPE;
  // Dk = 0 (channel_ratio >= 1, every channel pruned): visual logits are the
  // bias q . delta_mu alone, as the reference's kernels give with no kept
  // channel (its masked BLOCK_DK loads, fused_decode.py:131-148)
  if (c->Dk < 0 || c->Dk > 128) return RK_ERR_KEEP_DIM;
  if (dm) {
    st = rk::check_desc(dm, 3);
    if (st) return st;
    if (!rk::is_float_param(dm->dtype)) return RK_ERR_DTYPE;
    if (dm->shape[0] != c->B || dm->shape[1] != c->H_kv || dm->shape[2] != c->D) return RK_ERR_SHAPE;
  }
  st = rk::check_desc(kf, 4);
  if (st) return st;
  c->S_f = kf->shape[2];
  st = rk::check_desc(ks, 4);
  if (st) return st;
  c->S_v = ks->shape[2];
  if ((st = check_kv4(kf, *c, c->S_f, c->D, true))) return st;
  if ((st = check_kv4(vf, *c, c->S_f, c->D, true))) return st;
  if ((st = check_kv4(ks, *c, c->S_v, c->Dk, true))) return st;
  if ((st = check_kv4(vs, *c, c->S_v, c->D, true))) return st;
  if (!head_span_ok(kf) || !head_span_ok(vf) || !head_span_ok(vs) || (c->Dk > 0 && !head_span_ok(ks)))
    return RK_ERR_STRIDE;
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

// The plan of a checked call (fp32 over 4-byte elements).
int plan_for(const Checked& c, bool has_vis, int32_t policy, int cus, rk_decode_plan* p) {
  const bool f32 = c.dtype == RK_F32;
  return rk_plan_decode(c.B, c.H_q, c.H_kv, has_vis ? c.Dk : 0, has_vis ? c.S_v : 0, c.S_f, f32 ? 4 : 2, policy,
                        cus, p);
}

int resolve_cus(int32_t num_cus, int* st) {
  *st = RK_OK;
  if (num_cus > 0) return num_cus;
  int dev = 0;
  const int cus = rk::current_device_cus(&dev);
  if (cus <= 0) *st = RK_ERR_NO_DEVICE;
  return cus;
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

void set4(const rk_tensor* t, int64_t& s0, int64_t& s1, int64_t& s2, int64_t& s3) {
  s0 = t->stride[0];
  s1 = t->stride[1];
  s2 = t->stride[2];
  s3 = t->stride[3];
}

// Head strides (b, h) as int64; token/channel strides as uint32 (bounds
// checked by head_span_ok during validation).
bool set_head(const rk_tensor* t, int64_t& sb, int64_t& sh, uint32_t& ss, uint32_t& sd) {
  if (!head_span_ok(t)) return false;
  sb = t->stride[0];
  sh = t->stride[1];
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
  // the single-launch merge's ordering holds on gfx942 / gfx950 only
  a.fused = p.single_launch && rk::device_has_coherent_tickets() ? 1 : 0;
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
  // 16-byte row loads also need whole 8-channel slots (head_dim % 8 == 0)
  bool vec = rk::vec_ok(kf) && rk::vec_ok(vf) && c.D % 8 == 0;
  a.D = (int32_t)c.D;
  a.q_vec = q->stride[2] == 1 && q->stride[1] % 8 == 0 && q->stride[0] % 8 == 0 &&
            (((uintptr_t)q->data) & 15) == 0 && c.D % 8 == 0;
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
    // (a head's [D][Dk] block is copied as whole 16-byte chunks)
    a.r_vec = rk::is_half(R->dtype) && (c.Dk <= 64 || (c.Dk <= 128 && R->dtype == c.dtype)) &&
              R->stride[3] == 1 && R->stride[2] == c.Dk && (c.D * c.Dk) % 8 == 0 &&
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
  a.scale_log2 = (float)(rk::kLog2e / sqrt((double)c.D));  // 1 / sqrt(D) (fused_decode.py:340)
  a.cmajor = has_vis && c.dtype != RK_F32 && !a.xgroup ? p.chunk_major : 0;
  // the 16-bit kernels carry the single-launch merge at head_dim 128 with
  // 16-byte loads only; elsewhere the merge kernel runs
  if (c.dtype != RK_F32 && !(vec && c.D == 128)) a.fused = 0;
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
  // a workspace this library has not initialised gets zeroed counters first
  // (a fill kernel on the same stream; under graph capture it is recorded
  // with the decode)
  if (a.fused && !is_ready(ws)) {
    const int st0 = rk_decode_workspace_init(ws, RK_DECODE_TICKET_BYTES, stream);
    if (st0) return st0;
  }
  if (c.dtype == RK_F32) {
    const bool v32 = vec32_ok(kf) && vec32_ok(vf) && c.D % 4 == 0 &&
                     (!has_vis || ((c.Dk == 0 || vec32_ok(ks)) && vec32_ok(vs) && c.Dk % 4 == 0));
    return rk::decode_launch_f32(has_vis, v32, a, grid, s) == hipSuccess ? RK_OK : RK_ERR_HIP;
  }
  hipError_t e;
  if (vec && c.D < 128)  // 16-byte loads with the channels past D masked
    e = c.dtype == RK_F16 ? rk::decode_launch_f16_hd(dkb, hmax, has_vis, a, grid, s)
                          : rk::decode_launch_bf16_hd(dkb, hmax, has_vis, a, grid, s);
  else
    e = c.dtype == RK_F16 ? rk::decode_launch_f16(dkb, vec, hmax, has_vis, a, grid, s)
                          : rk::decode_launch_bf16(dkb, vec, hmax, has_vis, a, grid, s);
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
  if (!head_span_ok(v_buf)) return RK_ERR_STRIDE;
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
      if (t->shape[0] != c.B || t->shape[1] != c.H_kv || t->shape[2] != 1 || t->shape[3] != c.D)
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
                                                     int32_t* len, int H, int D, int64_t cap) {
  const int b = blockIdx.x;
  const int32_t pos = len[b];
  __syncthreads();
  if (pos >= 0 && pos < cap) {
    for (int i = threadIdx.x; i < H * D; i += blockDim.x) {
      const int h = i / D, d = i - h * D;
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
  const int64_t B = k_new->shape[0], H = k_new->shape[1], D = k_new->shape[3];
  if (D < 1 || D > 128) return RK_ERR_HEAD_DIM;
  if (k_new->shape[2] != 1) return RK_ERR_SHAPE;
  if (k_buf->shape[0] != B || k_buf->shape[1] != H || k_buf->shape[3] != D) return RK_ERR_SHAPE;
  if ((v_new == nullptr) != (v_buf == nullptr)) return RK_ERR_NULL;
  if (v_new) {
    if ((st = rk::check_desc(v_new, 4)) || (st = rk::check_desc(v_buf, 4))) return st;
    if (v_new->dtype != k_new->dtype || v_buf->dtype != k_new->dtype) return RK_ERR_DTYPE;
    for (int i = 0; i < 4; ++i)
      if (v_new->shape[i] != k_new->shape[i] || v_buf->shape[i] != k_buf->shape[i]) return RK_ERR_SHAPE;
  }
  if (B == 0 || H == 0) return RK_OK;
  if (!k_new->data || !k_buf->data || (v_new && (!v_new->data || !v_buf->data))) return RK_ERR_NULL;
  if (B > (INT64_C(1) << 30) || H * D > (INT64_C(1) << 30)) return RK_ERR_SHAPE;
  hipLaunchKernelGGL(append_kernel, dim3((unsigned)B), dim3(256), 0, (hipStream_t)stream,
                     (const uint16_t*)k_new->data, k_new->stride[0], k_new->stride[1], k_new->stride[3],
                     v_new ? (const uint16_t*)v_new->data : nullptr, v_new ? v_new->stride[0] : 0,
                     v_new ? v_new->stride[1] : 0, v_new ? v_new->stride[3] : 0, (uint16_t*)k_buf->data,
                     k_buf->stride[0], k_buf->stride[1], k_buf->stride[2], k_buf->stride[3],
                     v_buf ? (uint16_t*)v_buf->data : nullptr, v_buf ? v_buf->stride[0] : 0,
                     v_buf ? v_buf->stride[1] : 0, v_buf ? v_buf->stride[2] : 0, v_buf ? v_buf->stride[3] : 0,
                     len_full, (int)H, (int)D, k_buf->shape[2]);
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
  c->D = q->shape[2];
  c->Dk = 0;
  c->S_v = 0;
  c->S_f = k->shape[2];
  c->dtype = q->dtype;
  if (k->shape[3] != q->shape[2] || v->ndim < 1 || v->shape[v->ndim - 1] != q->shape[2])
    return RK_ERR_SHAPE;
  if (c->H_kv <= 0 || c->H_q / G != c->H_kv || c->H_q % G != 0) return RK_ERR_HEADS;
  if (!rk::is_half(q->dtype) && q->dtype != RK_F32) return RK_ERR_DTYPE;
  // any head size up to 128 (full_channel_flash_decoding.py:175-185 pads to
  // a power-of-two block with a mask)
  if (c->D < 1 || c->D > 128) return RK_ERR_HEAD_DIM;
  if ((st = check_kv4(k, *c, c->S_f, c->D, true))) return st;
  if ((st = check_kv4(v, *c, c->S_f, c->D, true))) return st;
  if (!head_span_ok(k) || !head_span_ok(v)) return RK_ERR_STRIDE;
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

// This device's `scratch`: its address, taken (and checked) on the first
// call on the device and kept per device.  Its ticket region is zeroed like
// any workspace the library has not initialised (run_decode).
int device_scratch(void** ptr) {
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0) return RK_ERR_NO_DEVICE;
  if (dev >= kMaxDevices) return RK_ERR_ARG;
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void* p = nullptr;
    if (hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)) != hipSuccess || !p) return RK_ERR_HIP;
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
  if ((st = device_scratch(&ws))) return st;
  return run_decode(c, q_full, R_partial, delta_mu, k_full, v_full, mask_full, k_sparse, v_sparse, out, pol,
                    ws, RK_NOALLOC_SCRATCH_BYTES, stream, true);
}
