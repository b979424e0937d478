"""Prefill-producer oracle (test infrastructure only; see ``oracle/__init__``).

Restates the RotateK prefill path of the reference with numpy:

* ``split_spans``        kv_pruning_utils.py:26-35
* ``key_covariance``     kv_pruning_utils.py:112-115 (fp32 mean, centering and
                         the covariance einsum rounded to the key dtype, then
                         symmetrised)
* ``query_weight``       kv_pruning_utils.py:116-140
* ``eigh_rotation``      kv_pruning_utils.py:146-150 (eigenvalue-descending
                         top-``keep`` eigenvectors)
* ``power_iteration``    rotation.py:21-53 (given the start block ``V0``)
* ``rotate_keys``        kv_pruning_utils.py:152 (``K_vis @ R_partial`` in the
                         key dtype)
* ``delta_mu``           kv_pruning_utils.py:153-156
* ``channel_scores`` / ``topk_channels``  the head-wise channel selection of
                         BASELINE config 0 (top-k channels by mean |K R_k|,
                         ties to the lower index, indices ascending)
* ``update_rotatek``     kv_pruning_utils.py:92-160 end to end, with either
                         selection rule.

Pinned by tests/test_oracle_prefill.py: ``numpy.cov`` on inputs whose storage
rounding is exact, brute-force loops, the eigen-equation ``C R = R Lambda`` and
orthonormality, ``delta_mu . R = 0`` and the projector identity, exhaustive
top-k on tiny inputs with planted ties, a hand-built even-length median case
for the query-weight floor, and subspace agreement of power iteration with
``eigh`` on a gapped spectrum.
"""
from __future__ import annotations

import numpy as np

from oracle.numerics import mean_factor, round_to

QUERY_WINDOW = 32   # kv_pruning_utils.py:23


def split_spans(total: int, prompt_seqlen: int, query_seqlen: int):
    """((p0,p1), (v0,v1), (t0,t1)) token ranges of prompt, visual and text."""
    p = max(0, min(prompt_seqlen, total))
    q = max(0, min(query_seqlen, max(total - p, 0)))
    vision_end = total - q if q > 0 else total
    text = (total - q, total) if q > 0 else (0, 0)
    return (0, p), (p, vision_end), text


def keep_count(head_dim: int, ratio: float) -> int:
    """Kept channels for a prune ``ratio`` (kv_pruning_utils.py:108)."""
    return head_dim - min(head_dim, max(0, int(head_dim * ratio)))


def key_covariance(keys_vision, dtype: str, mean=None):
    """(mean_fp32 [B,H,D], cov [B,H,D,D]) as the reference computes them.

    mean = fp32 mean of the Keys as torch's GPU mean forms it, fp32(sum) *
    fp32(n_out / n_in) (ATen MeanOps); Kc = dtype(K - dtype(mean)); cov =
    dtype(Kc^T Kc) (the einsum output is in the key dtype) then
    0.5 (cov + cov^T) in fp32.  ``mean`` (fp32 [B,H,D]) replaces the computed
    mean as the centre: the fp32 sum's rounding depends on its order, which
    no restatement shares with torch's reduction, and a centre that rounds
    the other way in the key dtype moves whole rows of the covariance.
    """
    K = np.asarray(keys_vision, np.float64)
    B, H, S, D = K.shape
    if mean is None:
        s32 = np.asarray(K.sum(axis=-2), np.float32)
        with np.errstate(invalid="ignore"):
            mean = (s32 * mean_factor(B * H * D, B * H * S * D)).astype(np.float64)
    else:
        mean = np.asarray(mean, np.float32).astype(np.float64)
    Kc = round_to(K - round_to(mean, dtype)[..., None, :], dtype)
    cov = np.einsum("bhsd,bhse->bhde", Kc, Kc)
    cov = round_to(round_to(cov, "float32"), dtype)
    cov = round_to(0.5 * (cov + np.swapaxes(cov, -1, -2)), "float32")
    return mean, cov


def query_weight(cov, queries, num_kv_groups: int, window: int = QUERY_WINDOW,
                 dtype: str | None = None):
    """Query-aware weighting of the covariance (kv_pruning_utils.py:121-140).

    queries [B, H_q, S_q, D]; uses the last ``window`` queries, group-means
    H_q -> H_kv (the group mean is stored in the query ``dtype`` before the
    fp32 norm, as torch's ``mean`` on a bf16 tensor is), weights cov by outer(||q||, ||q||) with a floor of
    1e-3 * median (lower middle element for an even count, as torch.median),
    symmetrises and adds ridge = 1e-4 * max(mean|diag|, 1e-6) * I (the clamp
    applies to the mean, kv_pruning_utils.py:137-139).  A NaN norm makes the
    median, hence every weight of the head, NaN (torch.median semantics).
    """
    cov = np.asarray(cov, np.float64)
    Q = np.asarray(queries, np.float64)
    B, Hkv, D, _ = cov.shape
    w = min(window, Q.shape[2])
    Qr = Q[..., -w:, :]
    if Qr.shape[1] != Hkv:
        # torch's mean of a bf16/fp16 tensor accumulates in fp32 and scales by
        # the fp32 factor 1/G before rounding to the tensor's dtype
        # (ATen mean_kernel_impl / MeanOps::project: acc * factor); with a
        # non-power-of-two G that differs from an exact division
        # (dtype None / float64: exact arithmetic)
        grp = Qr.reshape(B, Hkv, num_kv_groups, w, D)
        if dtype in ("bfloat16", "float16", "float32"):
            grp = grp.astype(np.float32)
            acc = np.zeros(grp.shape[:2] + grp.shape[3:], np.float32)
            for g in range(num_kv_groups):
                acc = acc + grp[:, :, g]
            f = mean_factor(B * Hkv * w * D, B * Hkv * num_kv_groups * w * D)
            Qr = round_to((acc * f).astype(np.float64), dtype)
        else:
            Qr = grp.mean(axis=2)
    qn = np.sqrt((Qr ** 2).sum(axis=-2))                           # [B,Hkv,D]
    med = np.sort(qn, axis=-1)[..., (D - 1) // 2]                  # lower median
    # torch.median of a row holding a NaN is NaN (torch.nanmedian is the
    # NaN-skipping one), and the clamp against a NaN floor is NaN
    med = np.where(np.isnan(qn).any(axis=-1), np.nan, med)
    qn = np.maximum(qn, 1e-3 * med[..., None])
    cov = cov * (qn[..., :, None] * qn[..., None, :])
    cov = 0.5 * (cov + np.swapaxes(cov, -1, -2))
    ridge = 1e-4 * np.maximum(np.abs(np.diagonal(cov, axis1=-2, axis2=-1)).mean(axis=-1), 1e-6)
    return cov + ridge[..., None, None] * np.eye(D)


def eigh_rotation(cov, keep: int):
    """(R_partial [...,D,keep], eigenvalues descending [...,D]) via eigh."""
    w, V = np.linalg.eigh(np.asarray(cov, np.float64))
    return V[..., ::-1][..., :keep], w[..., ::-1]


def power_iteration(cov, V0, num_iters: int = 5, eps: float = 1e-4):
    """Cholesky-QR subspace iteration (rotation.py:21-53) from start ``V0``."""
    C = np.asarray(cov, np.float64)
    V = np.asarray(V0, np.float64)
    k = V.shape[-1]
    for _ in range(num_iters):
        V = C @ V
        G = np.swapaxes(V, -1, -2) @ V
        tr = np.diagonal(G, axis1=-2, axis2=-1).mean(axis=-1)[..., None, None]
        G = G + eps * tr * np.eye(k)
        L = np.linalg.cholesky(G)
        # V <- V L^{-T}: solve X L^T = V for X
        V = np.swapaxes(np.linalg.solve(L, np.swapaxes(V, -1, -2)), -1, -2)
    return V


def rotate_keys(keys, R, dtype: str):
    """``K @ R`` rounded to the key dtype (kv_pruning_utils.py:152)."""
    return round_to(np.asarray(keys, np.float64) @ np.asarray(R, np.float64), dtype)


def delta_mu(mean_fp32, R_partial, dtype: str):
    """delta_mu = mu - (mu R) R^T with R already in the key dtype
    (kv_pruning_utils.py:153-156)."""
    mu = np.asarray(mean_fp32, np.float64)
    R = np.asarray(R_partial, np.float64)
    proj = np.einsum("bhk,bhdk->bhd", np.einsum("bhd,bhdk->bhk", mu, R), R)
    return round_to(mu - proj, dtype)


def channel_scores(keys, R_full):
    """Mean |K R| per rotated channel, float64 [B,H,D]."""
    Kt = np.asarray(keys, np.float64) @ np.asarray(R_full, np.float64)
    return np.abs(Kt).mean(axis=-2)


def topk_channels(scores, k: int):
    """Head-wise top-k: (indices ascending [B,H,k] int64, mask [B,H,D] bool).

    Order is score descending, ties broken towards the lower channel index.
    """
    s = np.asarray(scores, np.float64)
    D = s.shape[-1]
    order = np.lexsort((np.broadcast_to(np.arange(D), s.shape), -s), axis=-1)
    top = np.sort(order[..., :k], axis=-1).astype(np.int64)
    mask = np.zeros(s.shape, dtype=bool)
    np.put_along_axis(mask, top, True, axis=-1)
    return top, mask


def update_rotatek(key_states, query_states, prompt_seqlen: int, query_seqlen: int,
                   ratio: float, num_kv_groups: int, dtype: str,
                   query_aware: bool = True, select: str = "eig", R_full=None, cov=None, mean=None):
    """ChannelPruner.update_rotatek (kv_pruning_utils.py:92-160), eigh solver.

    select="eig": kept channels are the top-``keep`` eigenvectors (the
    reference rule, kept mask = first ``keep`` rotated channels).
    select="score": rotate by the full basis (``R_full`` if given, else all
    eigenvectors, eigenvalue-descending) and keep the top-``keep`` channels by
    mean |K R|.  ``cov`` (the weighted covariance) and ``mean`` (fp32) replace
    the computed ones, so that a test can compare the stages after them on
    the very same input.  Returns a dict of numpy arrays.
    """
    K = np.asarray(key_states, np.float64)
    B, Hkv, S, D = K.shape
    (p0, p1), (v0, v1), (t0, t1) = split_spans(S, prompt_seqlen, query_seqlen)
    Kv = K[:, :, v0:v1]
    keep = keep_count(D, ratio)
    if cov is None:
        mean_c, cov = key_covariance(Kv, dtype)
        if query_aware:
            cov = query_weight(cov, query_states, num_kv_groups, dtype=dtype)
        mean = mean_c if mean is None else mean
    else:
        cov = np.asarray(cov, np.float64)
        if mean is None:
            mean = key_covariance(Kv, dtype)[0]
        mean = np.asarray(mean, np.float64)
    if select == "eig":
        Rp, evals = eigh_rotation(cov, keep)
        idx = np.broadcast_to(np.arange(keep), (B, Hkv, keep)).copy()
        mask = np.zeros((B, Hkv, D), bool)
        mask[..., :keep] = True
        Rfull = None
    elif select == "score":
        Rfull = np.asarray(R_full, np.float64) if R_full is not None else eigh_rotation(cov, D)[0]
        idx, mask = topk_channels(channel_scores(Kv, Rfull), keep)
        Rp = np.take_along_axis(Rfull, idx[:, :, None, :], axis=-1)
    else:
        raise ValueError(select)
    Rp = round_to(Rp, dtype)
    return {
        "k_sparse": rotate_keys(Kv, Rp, dtype),
        "k_prompt": K[:, :, p0:p1],
        "k_text": K[:, :, t0:t1],
        "keep_mask": mask,
        "keep_idx": idx,
        "R_partial": Rp,
        "delta_mu": delta_mu(mean, Rp, dtype),
        "mean": mean,
        "cov": cov,
        "R_full": Rfull,
    }
