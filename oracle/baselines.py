"""ThinK / SparK baseline oracle (test infrastructure only; see ``oracle/__init__``).

Restates, with numpy, the two channel-pruning baselines the reference
compares RotateK against, and their decode-time Key recovery:

* ``think_score_and_compact``  rotatek/baselines/think.py:15-58
* ``group_queries``            kv_pruning_utils.py:76-79 (mean of the G query
                               heads of each KV head, SparK)
* ``per_token_channel_prune``  rotatek/baselines/spark.py:15-60
* ``recover_think``            llama_visionzip.py:219-225 (pruned channels 0)
* ``recover_spark``            llama_visionzip.py:226-230 (pruned channels =
                               the token's pruned mean)

Arithmetic follows torch's GPU kernels for the ops the reference calls:
``pow`` rounds each square to the storage dtype; a 16-bit ``mean`` is
``dtype(fp32 sum * f)`` with ``f = float(n_out) / float(n_in)`` (ATen
MeanOps); ``norm`` is ``dtype(sqrt(fp32 sum of squares))``; products of two
storage values are rounded once.  Sums are exact here, then rounded to fp32,
so results are exact wherever the device's fp32 sums are (inputs on a coarse
grid), and within one storage ulp otherwise.  Ties: ``topk(largest=False)``
takes equal values at the boundary in index order, so ThinK prunes the lower
channel first; ``argsort(descending)`` keeps equal values in index order, so
SparK keeps the lower channel first; NaN orders above every number.

Pinned by tests/test_oracle_baselines.py: closed forms on inputs whose scores
are known exactly (constant channels, power-of-two lengths), the selection
invariants (exactly ``keep`` kept, every kept score >= every pruned score,
boundary ties resolved by index in the stated direction), exhaustive checks
on 4-channel toy heads, ``recover(compact(K))`` equal to ``K`` on the kept
channels and to the fill elsewhere, and the pruned mean equal to the mean of
the channels the mask drops; tests/test_gpu_baselines.py additionally checks
the rounding and tie rules against torch's own GPU reduction, top-k and sort.
"""
from __future__ import annotations

import numpy as np

from oracle.numerics import mean_factor, round_to


def _mean16(x, axis: int, factor: np.float32, dtype: str) -> np.ndarray:
    """dtype(fp32(sum) * factor) along ``axis`` (values already in dtype)."""
    s = np.asarray(np.asarray(x, np.float64).sum(axis=axis), np.float32)
    with np.errstate(invalid="ignore", over="ignore"):
        return round_to(s * factor, dtype)


def _sq16(x, dtype: str) -> np.ndarray:
    """torch.pow(x, 2) in the storage dtype."""
    x = np.asarray(x, np.float64)
    return round_to(x * x, dtype)


def think_score_and_compact(keys_vision, queries_recent, num_kv_heads: int, prune_count: int, dtype: str):
    """(K_compact [B,H,S,D-prune], keep_mask [B,H,D] bool, scores [B,H,D]).

    queries_norm = dtype-mean over the group of the dtype-mean over the window
    of dtype(q^2); keys_norm = dtype-mean over tokens of dtype(k^2); score =
    dtype(qn * kn); the ``prune_count`` smallest scores are pruned, equal
    scores at the boundary lowest channel first (think.py:37-58).
    """
    K = np.asarray(keys_vision, np.float64)
    Q = np.asarray(queries_recent, np.float64)
    B, H, S, D = K.shape
    Hq, W = Q.shape[1], Q.shape[2]
    G = Hq // num_kv_heads
    keep = D - prune_count
    qn = _mean16(_sq16(Q, dtype), 2, mean_factor(B * Hq * D, B * Hq * W * D), dtype)
    qn = _mean16(qn.reshape(B, num_kv_heads, G, D), 2, mean_factor(B * num_kv_heads * D, B * Hq * D), dtype)
    kn = _mean16(_sq16(K, dtype), 2, mean_factor(B * H * D, B * H * S * D), dtype)
    with np.errstate(invalid="ignore"):
        scores = round_to(qn * kn, dtype)
    nan = np.isnan(scores)
    val = np.where(nan, 0.0, scores)
    chan = np.broadcast_to(np.arange(D), scores.shape)
    order = np.lexsort((chan, val, nan), axis=-1)       # ascending; ties -> lower index first
    keep_mask = np.ones((B, H, D), dtype=bool)
    np.put_along_axis(keep_mask, order[..., :prune_count], False, axis=-1)
    idx = np.sort(order[..., prune_count:], axis=-1)     # kept channels ascending
    assert idx.shape[-1] == keep
    K_compact = np.take_along_axis(K, idx[:, :, None, :].repeat(S, axis=2), axis=-1) if S else \
        np.zeros((B, H, 0, keep))
    return K_compact, keep_mask, scores


def group_queries(queries_window, num_kv_groups: int, dtype: str) -> np.ndarray:
    """[B, H_kv*G, W, D] -> [B, H_kv, W, D]: dtype-mean over the G query heads
    of each KV head (kv_pruning_utils.py:76-79)."""
    Q = np.asarray(queries_window, np.float64)
    B, Hq, W, D = Q.shape
    H = Hq // num_kv_groups
    return _mean16(Q.reshape(B, H, num_kv_groups, W, D), 2, mean_factor(B * H * W * D, B * Hq * W * D), dtype)


def per_token_channel_prune(queries, keys, prune_count: int, dtype: str):
    """(K_compact [B,H,S,D-prune], keep_mask [B,H,S,D] bool, pruned_mean
    [B,H,S,1], scores [B,H,S,D]) for grouped ``queries`` [B,H,W,D].

    q_norm = dtype(sqrt(fp32 sum over the window of q^2)); score =
    dtype(dtype(k^2) * q_norm); each token keeps its ``D - prune_count``
    largest scores, equal scores lowest channel first (stable descending
    sort); pruned_mean = dtype-mean of the token's other channels
    (spark.py:37-60).
    """
    Q = np.asarray(queries, np.float64)
    K = np.asarray(keys, np.float64)
    B, H, S, D = K.shape
    keep = D - prune_count
    ss = np.asarray((Q * Q).sum(axis=2), np.float32)
    qn = round_to(np.sqrt(ss), dtype)                                  # [B, H, D]
    with np.errstate(invalid="ignore", over="ignore"):
        scores = round_to(_sq16(K, dtype) * qn[:, :, None, :], dtype)
    nan = np.isnan(scores)
    val = np.where(nan, 0.0, scores)
    chan = np.broadcast_to(np.arange(D), scores.shape)
    order = np.lexsort((chan, -val, ~nan), axis=-1)    # descending; NaN first; ties -> lower index first
    kept = np.sort(order[..., :keep], axis=-1)
    pruned = order[..., keep:]
    K_compact = np.take_along_axis(K, kept, axis=-1)
    keep_mask = np.zeros((B, H, S, D), dtype=bool)
    np.put_along_axis(keep_mask, kept, True, axis=-1)
    pv = np.take_along_axis(K, pruned, axis=-1)
    pruned_mean = _mean16(pv, 3, mean_factor(B * H * S, B * H * S * prune_count), dtype)[..., None]
    return K_compact, keep_mask, pruned_mean, scores


def recover_think(key_pruned, think_mask) -> np.ndarray:
    """Full-width visual Keys with the kept channels of each head filled from
    ``key_pruned`` in ascending channel order and zeros elsewhere."""
    C = np.asarray(key_pruned, np.float64)
    M = np.asarray(think_mask, bool)
    B, H, S, _ = C.shape
    out = np.zeros((B, H, S, M.shape[-1]))
    for b in range(B):
        for h in range(H):
            out[b, h][:, M[b, h]] = C[b, h]
    return out


def recover_spark(key_pruned, spark_mask, pruned_mean) -> np.ndarray:
    """Full-width visual Keys: each token's kept channels from ``key_pruned``
    in ascending channel order, its pruned channels = its pruned mean."""
    C = np.asarray(key_pruned, np.float64)
    M = np.asarray(spark_mask, bool)
    out = np.broadcast_to(np.asarray(pruned_mean, np.float64), M.shape).copy()
    out[M] = C.reshape(-1)
    return out


def assemble(k_prompt, recovered, k_text) -> np.ndarray:
    """torch.cat([prompt, recovered, text], dim=-2) (llama_visionzip.py:232-234)."""
    return np.concatenate([np.asarray(k_prompt, np.float64), recovered, np.asarray(k_text, np.float64)], axis=2)
