/*
 * rotatek_hip.h -- C ABI of librotatek_hip.so, the MI355X (gfx950) library
 * behind the RotateK decode hot path and its prefill producer.
 *
 * Every entry point is plain C: device pointers, element strides, sizes, a
 * dtype code, a caller-owned workspace and a hipStream_t passed as void*.
 * Nothing here allocates device memory, throws, exits or synchronises the
 * host; every function returns an rk_status (0 = success, negative = error)
 * that rk_strerror() turns into text.  Shapes and strides are validated on
 * the host before any HIP call, so the *_check() variants and the error
 * paths of every entry point run without a GPU.
 *
 * Tensors are described by rk_tensor: a device pointer, a dtype, the rank
 * and per-dimension sizes and strides (in elements, any sign-free layout;
 * views such as V[:, :, s_p:s_p+s_v] are accepted as they are).
 *
 * Reference interfaces replaced (beomseokg/rotatek, file:line):
 *   rk_rotatek_decode      rotatek/kernels/fused_decode.py:303-420
 *                          (rotatek_decode_fused_triton, ROTATEK_KERNEL=paper)
 *                          and rotatek/kernels/gqa_decode.py:280-321
 *                          (rotatek_decode_gqa, ROTATEK_KERNEL=gqa)
 *   rk_full_channel_decode rotatek/kernels/full_channel_flash_decoding.py:162-229
 *                          (full_channel_decode_triton) and
 *                          rotatek/kernels/gqa_decode.py:254-277
 *                          (full_channel_decode_gqa)
 *   rk_key_covariance      integrations/lmms_eval/models/model_utils/
 *                          kv_pruning_utils.py:112-115 (mean, centering,
 *                          covariance einsum, symmetrisation)
 *   rk_key_covariance_weighted   kv_pruning_utils.py:112-140 (the above
 *                          plus the query-aware weighting and ridge)
 *   rk_query_weight        kv_pruning_utils.py:116-140 (weighting alone)
 *   rk_rotate_keys         kv_pruning_utils.py:152 (K_vis @ R_partial, the
 *                          truncated visual-Key write)
 *   rk_channel_scores      channel scoring of the head-wise top-k selection
 *                          (mean |K_vis R|), no reference counterpart beyond
 *                          the keep mask of kv_pruning_utils.py:158-159
 *   rk_topk_channels       head-wise channel top-k -> ascending indices + mask
 *                          (kv_pruning_utils.py:158-159 keep_mask)
 *   rk_gather_rotation     R_partial = R_full[..., idx] and
 *                          delta_mu = mu - (mu R) R^T (kv_pruning_utils.py:150-156)
 *   rk_think_score_and_compact   rotatek/baselines/think.py:15-58
 *   rk_spark_prune         rotatek/baselines/spark.py:15-60 (+ the query
 *                          group mean, kv_pruning_utils.py:76-79)
 *   rk_think_recover / rk_spark_recover
 *                          Key recovery + concatenation of the ThinK / SparK
 *                          decode branch (llama_visionzip.py:216-234)
 */
#ifndef ROTATEK_HIP_H
#define ROTATEK_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* 3: any head_dim 1..128 (decode, dense, span cache, prefill, power
 * iteration); fp32 Keys / queries / R_partial in the prefill entries;
 * rk_decode_workspace_release.
 * 2: rk_power_iteration takes eps and a per-matrix info flag; the decode
 * plan carries the chunk-major layout fields; rk_rotatek_decode_noalloc,
 * rk_key_covariance_weighted and the merge / workspace entry points. */
#define RK_ABI_VERSION 3

/* Element types. */
typedef enum rk_dtype {
  RK_F16 = 0,
  RK_BF16 = 1,
  RK_F32 = 2,
  RK_F64 = 3,
  RK_U8 = 4,    /* also used for bool masks */
  RK_I32 = 5,
  RK_I64 = 6
} rk_dtype;

/* Status codes (0 = success). */
typedef enum rk_status {
  RK_OK = 0,
  RK_ERR_NULL = -1,          /* required pointer or descriptor is NULL      */
  RK_ERR_RANK = -2,          /* tensor has the wrong number of dimensions   */
  RK_ERR_DTYPE = -3,         /* unsupported or mismatched element type      */
  RK_ERR_SHAPE = -4,         /* sizes disagree between tensors              */
  RK_ERR_HEADS = -5,         /* H_q / num_kv_groups != H_kv                 */
  RK_ERR_HEAD_DIM = -6,      /* head_dim outside 1..128                     */
  RK_ERR_KEEP_DIM = -7,      /* kept channels out of range (decode 0..128,
                                prefill 1..128, power iteration 1..D)       */
  RK_ERR_STRIDE = -8,        /* negative or overflowing stride              */
  RK_ERR_WORKSPACE = -9,     /* workspace NULL, misaligned or too small     */
  RK_ERR_ARG = -10,          /* other invalid scalar argument               */
  RK_ERR_HIP = -11,          /* a HIP runtime call failed                   */
  RK_ERR_NO_DEVICE = -12,    /* no HIP device visible                       */
  RK_ERR_SCRATCH = -13       /* problem too large for the allocation-free
                                entry point's fixed scratch                 */
} rk_status;

/* Decode launch policy (ROTATEK_KERNEL). */
typedef enum rk_policy {
  RK_POLICY_PAPER = 0,  /* one work unit per query head: K/V re-read per head */
  RK_POLICY_GQA = 1     /* the query heads of a KV group share each K/V tile  */
} rk_policy;

#define RK_MAX_DIMS 4

typedef struct rk_tensor {
  void* data;                  /* device pointer                               */
  int32_t dtype;               /* rk_dtype                                     */
  int32_t ndim;                /* 1..4                                         */
  int64_t shape[RK_MAX_DIMS];  /* sizes; entries >= ndim ignored               */
  int64_t stride[RK_MAX_DIMS]; /* element strides                              */
} rk_tensor;

/* ------------------------------------------------------------------ misc */
const char* rk_strerror(int status);
int rk_abi_version(void);
/* Compute units of HIP device `device` (0 on error, sets *status). */
int rk_device_cu_count(int device, int* status);

/* ------------------------------------------------------------------ decode
 * One RotateK decode step (fused_decode.py:303-420 / gqa_decode.py:280-321):
 *   out[b,h,:] = softmax over {visual, prompt+text} tokens of
 *     visual:      (k_sparse . (q R_partial) + q . delta_mu) / sqrt(D)
 *     prompt+text: (k_full . q) / sqrt(D), tokens with mask_full == 0 skipped
 *   applied to v_sparse / v_full, written as acc / (l + 1e-6).
 * Shapes: q_full [B,H_q,D]; R_partial [B,H_kv,D,Dk]; delta_mu [B,H_kv,D] or
 * NULL; k_full, v_full [B,H_kv,S_f,D]; mask_full [B,S_f] u8 or NULL (= all
 * ones); k_sparse [B,H_kv,S_v,Dk]; v_sparse [B,H_kv,S_v,D]; out [B,H_q,D]
 * (dtype of q_full).  1 <= D <= 128, 0 <= Dk <= 128 (Dk = 0: every channel
 * pruned, visual logits are the bias alone; R_partial and k_sparse may then
 * have no storage).  q, K, V and out share one dtype (F16, BF16 or F32;
 * fp32 runs a VALU kernel, one unit per query head); R_partial and
 * delta_mu may be F16, BF16 or F32.
 * The workspace (size from rk_rotatek_decode_check, 256-byte aligned) holds
 * the split partials and, in its first RK_DECODE_TICKET_BYTES, the
 * counters of the single-launch merge (unit tickets, then batch-row
 * tickets, at fixed offsets).  Every call leaves the counters at zero.  A
 * workspace the library has not seen (by its address) gets them
 * zeroed by a fill kernel on `stream` ahead of its first single-launch
 * decode; rk_decode_workspace_init does the same explicitly, and
 * rk_decode_workspace_release forgets an address (call it before the
 * memory is freed or reused for anything else).  A step is two launches
 * on `stream` (split kernel, merge kernel), or one (see
 * rk_set_decode_merge), and is hipGraph-capturable.  Calls that overlap
 * on one workspace race.  policy RK_POLICY_PAPER with num_kv_groups > 1 runs the
 * grouped decomposition (each K/V tile read once per KV head; the result
 * differs from one unit per query head only in fp32 summation order).
 */
int rk_rotatek_decode_check(const rk_tensor* q_full, const rk_tensor* R_partial,
                            const rk_tensor* delta_mu, const rk_tensor* k_full,
                            const rk_tensor* v_full, const rk_tensor* mask_full,
                            const rk_tensor* k_sparse, const rk_tensor* v_sparse,
                            int64_t num_kv_groups, const rk_tensor* out,
                            int32_t policy, int32_t num_cus,
                            size_t* workspace_bytes);

int rk_rotatek_decode(const rk_tensor* q_full, const rk_tensor* R_partial,
                      const rk_tensor* delta_mu, const rk_tensor* k_full,
                      const rk_tensor* v_full, const rk_tensor* mask_full,
                      const rk_tensor* k_sparse, const rk_tensor* v_sparse,
                      int64_t num_kv_groups, const rk_tensor* out,
                      int32_t policy, void* workspace, size_t workspace_bytes,
                      void* stream);

/* Allocation-free variant of rk_rotatek_decode.  No counterpart in the
 * reference: it is for callers that cannot allocate device memory (code
 * under HIP graph capture, tight serving loops, harnesses that forbid
 * hipMalloc).  Same arguments, results (bit for bit) and errors as
 * rk_rotatek_decode, without the workspace: the split partials and the
 * merge counters live in a fixed device array of RK_NOALLOC_SCRATCH_BYTES
 * that the library holds on every GPU it runs on until the process ends
 * (its address is resolved, and its counters cleared, by the first call
 * on each device).  A shape whose workspace would exceed it returns
 * RK_ERR_SCRATCH (rk_rotatek_decode_check reports the bytes needed).
 * Nothing is allocated by this call.  Calls that overlap on one GPU (other
 * streams, other threads) share the array and race; serialise them. */
#define RK_NOALLOC_SCRATCH_BYTES (16u * 1024u * 1024u)
int rk_rotatek_decode_noalloc(const rk_tensor* q_full, const rk_tensor* R_partial,
                              const rk_tensor* delta_mu, const rk_tensor* k_full,
                              const rk_tensor* v_full, const rk_tensor* mask_full,
                              const rk_tensor* k_sparse, const rk_tensor* v_sparse,
                              int64_t num_kv_groups, const rk_tensor* out,
                              int32_t policy, void* stream);

/* Variable-length variant for a preallocated span cache (no reference
 * counterpart: the reference re-concatenates the spans every decode step,
 * cache_utils.py:52-53, llama_visionzip.py:207-208).
 *   k_full    [B,H_kv,C,D]     prompt then text Keys, capacity C rows.
 *   v_buf     [B,H_kv,C+v_gap,D]  Values; logical prompt/text row t lives
 *             at row t + (t >= v_gap_at ? v_gap : 0), so the cache's
 *             [prompt | visual | text] Value buffer is passed whole with
 *             v_gap_at = S_prompt and v_gap = S_visual (v_gap 0: plain).
 *   mask_full [B,C] or NULL;  v_sparse usually a view of v_buf's visual rows.
 *   len_full  device int32 [B]: only rows t < len_full[b] are attended.
 *   k_new, v_new  [B,H_kv,1,D] or both NULL.  If given, the step appends
 *             them first: the new token is attended, written to row
 *             len_full[b] of k_full / v_buf, and len_full[b] is incremented
 *             (all in the same two launches; a row whose buffer is full,
 *             len_full[b] >= C, neither attends nor stores it).
 * Shapes are fixed by capacity, so one captured HIP graph replays across
 * growing decode steps. */
int rk_rotatek_decode_varlen(const rk_tensor* q_full, const rk_tensor* R_partial,
                             const rk_tensor* delta_mu, const rk_tensor* k_full,
                             const rk_tensor* v_buf, int64_t v_gap_at, int64_t v_gap,
                             const rk_tensor* mask_full, const rk_tensor* k_sparse,
                             const rk_tensor* v_sparse, int64_t num_kv_groups,
                             const rk_tensor* k_new, const rk_tensor* v_new, int32_t* len_full,
                             const rk_tensor* out, int32_t policy, void* workspace,
                             size_t workspace_bytes, void* stream);

/* Query-aware weighting of the Key covariance, replacing
 * kv_pruning_utils.py:116-140: cov [B,H_kv,D,D] F32 (1 <= D <= 128), queries
 * [B,H_kv*G,S,D] F16/BF16/F32 (the last min(window, S) rows are used,
 * window <= 32), out like cov (may alias it). */
int rk_query_weight(const rk_tensor* cov, const rk_tensor* queries, int64_t num_kv_groups, int32_t window,
                    const rk_tensor* out, void* stream);

/* Top-k eigenbasis of each D x D covariance by subspace iteration with
 * Cholesky-QR orthonormalisation, replacing rotation.py:21-91
 * (_power_iter_loop; power_iteration_gpu draws v0 with torch.randn from a
 * seeded device generator and calls this).  cov [B,H,D,D] (1 <= D <= 128),
 * v0 / out [B,H,D,k] F32, 1 <= k <= D; per iteration V = C V, G = V^T V +
 * eps * mean(diag G) * I, V = V chol(G)^-T.  out may alias v0.  info
 * (device int32 [B*H], optional) receives 1 for a matrix whose Cholesky
 * met a pivot that is not positive and finite (its output is then not a
 * basis; the reference's torch.linalg.cholesky raises), else 0. */
int rk_power_iteration(const rk_tensor* cov, const rk_tensor* v0, const rk_tensor* out, int32_t num_iters,
                       float eps, int32_t* info, void* stream);

/* In-place decode append for the span cache (replaces the per-step
 * torch.cat of cache_utils.py:52-53): k_new/v_new [B,H,1,D] are written
 * to slot len_full[b] of k_buf/v_buf [B,H,capacity,D] and len_full[b] is
 * incremented on the device (a full buffer is left unchanged).  v_new and
 * v_buf may both be NULL. */
int rk_append_kv(const rk_tensor* k_new, const rk_tensor* v_new, const rk_tensor* k_buf,
                 const rk_tensor* v_buf, int32_t* len_full, void* stream);

/* Dense (full-channel) decode, the baseline the RotateK speed-up is measured
 * against (full_channel_flash_decoding.py:162-229, gqa_decode.py:254-277):
 * q [B,H_q,D], k/v [B,H_kv,S,D], out [B,H_q,D]. */
int rk_full_channel_decode_check(const rk_tensor* q, const rk_tensor* k,
                                 const rk_tensor* v, int64_t num_kv_groups,
                                 const rk_tensor* out, int32_t policy,
                                 int32_t num_cus, size_t* workspace_bytes);

int rk_full_channel_decode(const rk_tensor* q, const rk_tensor* k,
                           const rk_tensor* v, int64_t num_kv_groups,
                           const rk_tensor* out, int32_t policy,
                           void* workspace, size_t workspace_bytes,
                           void* stream);

/* Bytes at the start of a decode workspace that hold the single-launch
 * merge's counters; rk_decode_workspace_init zeroes them (a kernel on
 * `stream`, not a memset, so it may also be recorded in a graph) and marks
 * the workspace as initialised.  No counterpart in the reference (its
 * Triton launches need no counters).  rk_decode_workspace_release drops
 * that mark, so the next decode on the address initialises it again. */
#define RK_DECODE_TICKET_BYTES (256u * 1024u)
int rk_decode_workspace_init(void* workspace, size_t workspace_bytes, void* stream);
void rk_decode_workspace_release(void* workspace);

/* Merge of the decode entry points: 1 = two launches (split kernel, then a
 * merge kernel), 2 = one launch (the last split workgroup of each unit
 * merges, behind a counter in the workspace's ticket region) whenever the
 * counters fit (up to 49152 units and 16384 batch rows), 0 (default) =
 * one launch for a single round of workgroups with one query head per
 * unit, else two (what measured faster on MI355X).  Both give
 * bit-identical results.  The one-launch merge relies on the cross-XCD
 * store/load coherence of gfx942 / gfx950 and is compiled into the F16 /
 * BF16 kernels at head_dim 128 with 16-byte rows (and the F32 kernel); on
 * any other device or layout every mode runs two launches. */
void rk_set_decode_merge(int32_t mode);

/* Split plan the decode entry points use for a shape (host only), exposed
 * for tests and benchmarks.  Fields are filled on RK_OK. */
typedef struct rk_decode_plan {
  int64_t units;          /* work units (B*H_kv for GQA, B*H_q for paper)    */
  int32_t heads_per_unit; /* query heads handled per unit (<= 16)            */
  int32_t head_blocks;    /* ceil(G / 16) under GQA, else 1                  */
  int32_t wg_vis;         /* workgroups per unit over the visual span        */
  int32_t wg_full;        /* workgroups per unit over the prompt+text span   */
  int64_t chunk_vis;      /* visual tokens per workgroup                     */
  int64_t chunk_full;     /* prompt+text tokens per workgroup                */
  int64_t grid;           /* total workgroups launched                       */
  size_t workspace_bytes;
  int32_t single_launch;  /* 1: the merge runs in the split launch           */
  int32_t chunk_major;    /* 1: workgroup ids run chunk-major (x*units + u)  */
  int32_t n_fast;         /* visual chunks 0 .. n_fast-1 hold chunk_fast     */
  int64_t chunk_fast;     /* tokens (the others chunk_vis)                   */
} rk_decode_plan;

int rk_plan_decode(int64_t B, int64_t H_q, int64_t H_kv, int64_t Dk,
                   int64_t S_v, int64_t S_f, int32_t elem_bytes,
                   int32_t policy, int32_t num_cus, rk_decode_plan* plan);

/* Tuning knobs of the split planner (bytes of K/V streamed per workgroup
 * are clamped to [min_bytes, max_bytes], a max below the min reading as
 * the min, and the planner aims for wgs_per_cu workgroups per compute
 * unit).  These and the knobs below are process-wide and atomic; each
 * plan reads them once, so a decode planned while another thread changes
 * them uses either the old or the new values.  Pass 0 to keep a value;
 * wgs_per_cu < 0 restores the default: two workgroups per CU, one for a
 * single chunk-major round whose two-slot visual chunks would stream
 * <= 128 KB each (192 KB for units of one query head), and one for fp32
 * wherever that is still a single round. */
void rk_set_decode_tuning(int64_t min_bytes, int64_t max_bytes, int32_t wgs_per_cu);

/* Granularity of the visual chunks in tokens (32, 64 or 128: whole
 * 32-token blocks, or one block per wave; 0 = the default, 32 in a
 * chunk-major grid, else 128).  Planner override for sweeps. */
void rk_set_decode_chunk_align(int32_t tokens);

/* One-round grids of short workgroups: 0 = unit-major launch, 1000 =
 * chunk-major launch with equal chunks, 1001..4000 = chunk-major with the
 * first-dispatched chunks of <= 128 KB workgroups given this many
 * thousandths of the others' tokens (default 1300).  Planner override for
 * sweeps. */
void rk_set_decode_skew(int32_t permille);

/* ------------------------------------------------------------------ prefill
 * Keys are the visual span of the layer's Keys, [B, H_kv, S_v, D] in F16,
 * BF16 or F32 (the reference's update_rotatek is plain torch: any float
 * dtype), 1 <= D <= 128, any strides (a head must span < 2^31 elements).
 * For F32 Keys "the key dtype" below is fp32 (no 16-bit rounding), and the
 * products run on the fp32 MFMA.
 *
 * Key covariance (kv_pruning_utils.py:112-115):
 *   mean_out[b,h,:] = fp32 mean of K over S_v                (F32, optional)
 *   cov_out[b,h]    = 0.5 (C + C^T), C = dtype(Kc^T Kc) in fp32,
 *                     Kc = dtype(K - dtype(mean))            (F32 [B,H,D,D])
 * Three launches (mean partials, MFMA covariance partials, finalise); the
 * workspace size comes from rk_key_covariance_check. */
int rk_key_covariance_check(const rk_tensor* keys, const rk_tensor* mean_out,
                            const rk_tensor* cov_out, int32_t num_cus,
                            size_t* workspace_bytes);
int rk_key_covariance(const rk_tensor* keys, const rk_tensor* mean_out,
                      const rk_tensor* cov_out, void* workspace,
                      size_t workspace_bytes, void* stream);

/* Key covariance followed by the query-aware weighting, in the same three
 * launches as rk_key_covariance (the weighting is folded into the last):
 * cov_out = the result of rk_key_covariance then rk_query_weight, bit for
 * bit (kv_pruning_utils.py:112-140).  queries [B,H_kv*G,S_q,D] in the key
 * dtype, window 1..32 (the last min(window, S_q) rows).  Workspace size
 * from the _check variant (the same as rk_key_covariance's). */
int rk_key_covariance_weighted_check(const rk_tensor* keys, const rk_tensor* queries, int64_t num_kv_groups,
                                     int32_t window, const rk_tensor* mean_out, const rk_tensor* cov_out,
                                     int32_t num_cus, size_t* workspace_bytes);
int rk_key_covariance_weighted(const rk_tensor* keys, const rk_tensor* queries, int64_t num_kv_groups,
                               int32_t window, const rk_tensor* mean_out, const rk_tensor* cov_out,
                               void* workspace, size_t workspace_bytes, void* stream);

/* Truncated visual-Key write (kv_pruning_utils.py:152):
 * out[b,h,s,:] = dtype(K[b,h,s,:] @ R_partial[b,h]), R_partial
 * [B,H,D,Dk] (F16/BF16/F32), out [B,H,S_v,Dk] in the key dtype. */
int rk_rotate_keys(const rk_tensor* keys, const rk_tensor* R_partial,
                   const rk_tensor* out, void* stream);

/* Channel scores of the head-wise selection: scores_out[b,h,c] =
 * mean_s |K R_full|[s,c] with fp64 final reduction; R_full [B,H,D,Dc]
 * (Dc <= 128), scores_out [B,H,Dc] F64. */
int rk_channel_scores_check(const rk_tensor* keys, const rk_tensor* R_full,
                            const rk_tensor* scores_out, int32_t num_cus,
                            size_t* workspace_bytes);
int rk_channel_scores(const rk_tensor* keys, const rk_tensor* R_full,
                      const rk_tensor* scores_out, void* workspace,
                      size_t workspace_bytes, void* stream);

/* Head-wise channel top-k (keep mask of kv_pruning_utils.py:158-159):
 * scores [B,H,D] F64 (D <= 128) -> idx_out [B,H,k] I64, the k channels with
 * the largest scores (ties to the lower index) in ascending order, and
 * mask_out [B,H,D] U8 (optional). */
int rk_topk_channels(const rk_tensor* scores, int64_t k, const rk_tensor* idx_out,
                     const rk_tensor* mask_out, void* stream);

/* R_partial / delta_mu (kv_pruning_utils.py:150-156):
 * R_out[b,h,:,j] = dtype(R_full[b,h,:,idx[b,h,j]]) and
 * delta_mu_out[b,h] = dtype(mean - (mean R_out) R_out^T) computed in fp32
 * from the rounded R_out.  R_full [B,H,D,*] F16/BF16/F32, idx [B,H,k] I64,
 * mean [B,H,D] F32, R_out [B,H,D,k] and delta_mu_out [B,H,D] in F16, BF16
 * or F32 (fp32 Keys: no rounding). */
int rk_gather_rotation(const rk_tensor* R_full, const rk_tensor* idx,
                       const rk_tensor* mean, const rk_tensor* R_out,
                       const rk_tensor* delta_mu_out, void* stream);

/* ---- ThinK / SparK baselines (the methods RotateK is compared against).
 * Rounding follows the reference's torch GPU ops: each square rounded to
 * the key dtype, a 16-bit mean = dtype(fp32 sum * float(n_out)/float(n_in)),
 * products of two stored values rounded once.  Head dim D: any 1..128
 * (RK_ERR_HEAD_DIM otherwise), the same in every tensor of a call. */

/* ThinK prefill, replaces rotatek/baselines/think.py:15-58
 * (think_score_and_compact).  keys_vision [B,H,S_v,D] and queries_recent
 * [B,H_q,Q,D] (F16/BF16, same dtype, H_q a multiple of
 * num_kv_heads == H); score[c] = dtype(queries_norm[c] * keys_norm[c]); the
 * prune_count (0..D) smallest scores are pruned, equal scores lowest
 * channel first.  k_compact_out [B,H,S_v,D-prune_count] (kept channels,
 * ascending), keep_mask_out [B,H,D] U8 (1 = kept).  Workspace size from
 * the _check variant. */
int rk_think_score_and_compact_check(const rk_tensor* keys_vision,
                                     const rk_tensor* queries_recent,
                                     int64_t num_kv_heads, int64_t prune_count,
                                     const rk_tensor* k_compact_out,
                                     const rk_tensor* keep_mask_out,
                                     int32_t num_cus, size_t* workspace_bytes);
int rk_think_score_and_compact(const rk_tensor* keys_vision,
                               const rk_tensor* queries_recent,
                               int64_t num_kv_heads, int64_t prune_count,
                               const rk_tensor* k_compact_out,
                               const rk_tensor* keep_mask_out, void* workspace,
                               size_t workspace_bytes, void* stream);

/* SparK prefill, replaces rotatek/baselines/spark.py:15-60
 * (per_token_channel_prune) together with the query group mean of
 * kv_pruning_utils.py:76-79.  keys_vision [B,H,S_v,D]; queries
 * [B,H*num_kv_groups,W,D] are averaged over each KV head's group
 * (num_kv_groups = 1: already grouped), q_norm = dtype(||q||_2 over W); per
 * token score = dtype(dtype(k^2) * q_norm), the D-prune_count largest kept
 * (equal scores lowest channel first).
 * k_compact_out [B,H,S_v,D-prune_count], keep_mask_out [B,H,S_v,D] U8,
 * pruned_mean_out [B,H,S_v,1] = dtype-mean of the pruned values (NaN when
 * prune_count is 0, as torch's mean of nothing). */
int rk_spark_prune_check(const rk_tensor* keys_vision, const rk_tensor* queries,
                         int64_t num_kv_groups, int64_t prune_count,
                         const rk_tensor* k_compact_out,
                         const rk_tensor* keep_mask_out,
                         const rk_tensor* pruned_mean_out, int32_t num_cus,
                         size_t* workspace_bytes);
int rk_spark_prune(const rk_tensor* keys_vision, const rk_tensor* queries,
                   int64_t num_kv_groups, int64_t prune_count,
                   const rk_tensor* k_compact_out, const rk_tensor* keep_mask_out,
                   const rk_tensor* pruned_mean_out, void* workspace,
                   size_t workspace_bytes, void* stream);

/* Decode-time Key recovery, replaces the zero-filled (ThinK) / mean-filled
 * (SparK) tensor, its boolean-index scatter and the torch.cat of
 * llama_visionzip.py:216-234 (qwen2_5vl_visionzip.py:996-1010).  out
 * [B,H,S_p+S_v+S_t,D] gets k_prompt [B,H,S_p,D] (optional, NULL = none),
 * then the S_v recovered rows, then k_text [B,H,S_t,D] (optional).  Each
 * visual row takes its kept channels (mask 1) from k_pruned [B,H,S_v,Dk] in
 * ascending channel order; the others are 0 (ThinK, think_mask [B,H,D] U8)
 * or the row's pruned_mean [B,H,S_v,1] (SparK, spark_mask [B,H,S_v,D] U8).
 * Masks must hold exactly Dk kept channels per head / row, as the prefill
 * entries write them (extra kept channels are filled like pruned ones). */
int rk_think_recover_check(const rk_tensor* k_prompt, const rk_tensor* k_pruned,
                           const rk_tensor* k_text, const rk_tensor* think_mask,
                           const rk_tensor* out);
int rk_think_recover(const rk_tensor* k_prompt, const rk_tensor* k_pruned,
                     const rk_tensor* k_text, const rk_tensor* think_mask,
                     const rk_tensor* out, void* stream);
int rk_spark_recover_check(const rk_tensor* k_prompt, const rk_tensor* k_pruned,
                           const rk_tensor* k_text, const rk_tensor* spark_mask,
                           const rk_tensor* pruned_mean, const rk_tensor* out);
int rk_spark_recover(const rk_tensor* k_prompt, const rk_tensor* k_pruned,
                     const rk_tensor* k_text, const rk_tensor* spark_mask,
                     const rk_tensor* pruned_mean, const rk_tensor* out,
                     void* stream);

/* One-hot selection rotation from a per-head keep mask [B,H,D] U8:
 * R_out[b,h,c,j] = 1 if c is the j-th kept channel (ascending), else 0;
 * R_out [B,H,D,Dk] F16/BF16/F32, 1 <= Dk <= D <= 128.  No counterpart in the reference: with
 * it rk_rotatek_decode (delta_mu NULL) runs ThinK's zero-filled attention
 * straight from the compact Keys, for callers that want ThinK without the
 * recovery pass. */
int rk_channel_selection(const rk_tensor* keep_mask, const rk_tensor* R_out,
                         void* stream);

#ifdef __cplusplus
}
#endif

#endif /* ROTATEK_HIP_H */
