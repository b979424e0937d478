"""RotateK prefill producer on the HIP device.

Functional building blocks of ``ChannelPruner.update_rotatek``
(kv_pruning_utils.py:92-160), each a thin launcher over librotatek_hip.so:

* ``key_covariance``   fp32 mean and dtype-rounded, symmetrised covariance of
                       the visual Keys (MFMA kernel; kv_pruning_utils.py:112-115)
* ``rotate_keys``      truncated visual-Key write ``dtype(K R_partial)``
                       (kv_pruning_utils.py:152)
* ``channel_scores``   mean |K R| per rotated channel (fp64), the head-wise
                       selection score
* ``topk_channels``    head-wise top-k -> ascending indices + keep mask
* ``gather_rotation``  ``R_partial = dtype(R[:, idx])`` and
                       ``delta_mu = dtype(mu - (mu R_partial) R_partial^T)``
                       (kv_pruning_utils.py:150-156)
* ``query_weight``     query-aware weighting of the covariance
                       (kv_pruning_utils.py:116-140)

and, in torch: ``eigen_rotation`` (kv_pruning_utils.py:146-150), on the
device by default (``ROTATEK_EIGH=host`` keeps the reference's CPU route).
"""
from __future__ import annotations

import ctypes
import os

import torch

from rotatek_amd import _lib

QUERY_WINDOW = 32  # kv_pruning_utils.py:23


def _gpu(t: torch.Tensor, name: str) -> None:
    if not t.is_cuda:
        raise RuntimeError(f"{name} must be a GPU tensor: the RotateK prefill kernels run only on the HIP device")


def key_covariance(keys_vision: torch.Tensor, query_states: torch.Tensor | None = None,
                   num_key_value_groups: int = 1):
    """(mean [B,H,D] fp32, cov [B,H,D,D] fp32) of ``keys_vision`` [B,H,S,D].

    With ``query_states`` [B, H*G, S_q, D] the covariance comes back already
    query-weighted (``query_weight``'s result, bit for bit), the weighting
    folded into the covariance's last launch (``rk_key_covariance_weighted``).
    """
    _gpu(keys_vision, "keys_vision")
    B, H, _, D = keys_vision.shape
    lib = _lib.load()
    mean = torch.empty(B, H, D, device=keys_vision.device, dtype=torch.float32)
    cov = torch.empty(B, H, D, D, device=keys_vision.device, dtype=torch.float32)
    dk, dm, dc = _lib.desc(keys_vision), _lib.desc(mean), _lib.desc(cov)
    need = ctypes.c_size_t(0)
    stream = _lib.stream_handle(keys_vision.device)
    if query_states is None:
        _lib.check(lib.rk_key_covariance_check(ctypes.byref(dk), ctypes.byref(dm), ctypes.byref(dc), 0,
                                               ctypes.byref(need)), "key_covariance")
        ws = torch.empty(max(need.value, 256), dtype=torch.uint8, device=keys_vision.device)
        _lib.check(lib.rk_key_covariance(ctypes.byref(dk), ctypes.byref(dm), ctypes.byref(dc), ws.data_ptr(),
                                         ws.numel(), stream), "key_covariance")
        return mean, cov
    dq = _lib.desc(query_states)
    G = int(num_key_value_groups)
    _lib.check(lib.rk_key_covariance_weighted_check(ctypes.byref(dk), ctypes.byref(dq), G, QUERY_WINDOW,
                                                    ctypes.byref(dm), ctypes.byref(dc), 0, ctypes.byref(need)),
               "key_covariance")
    ws = torch.empty(max(need.value, 256), dtype=torch.uint8, device=keys_vision.device)
    _lib.check(lib.rk_key_covariance_weighted(ctypes.byref(dk), ctypes.byref(dq), G, QUERY_WINDOW,
                                              ctypes.byref(dm), ctypes.byref(dc), ws.data_ptr(), ws.numel(),
                                              stream), "key_covariance")
    return mean, cov


def rotate_keys(keys_vision: torch.Tensor, R_partial: torch.Tensor, out: torch.Tensor | None = None):
    """``dtype(keys_vision @ R_partial)`` -> [B,H,S,Dk] (written into ``out``
    when given, e.g. a slice of a preallocated cache)."""
    _gpu(keys_vision, "keys_vision")
    B, H, S, _ = keys_vision.shape
    if out is None:
        out = torch.empty(B, H, S, R_partial.shape[-1], device=keys_vision.device, dtype=keys_vision.dtype)
    dk, dr, do = _lib.desc(keys_vision), _lib.desc(R_partial), _lib.desc(out)
    _lib.check(_lib.load().rk_rotate_keys(ctypes.byref(dk), ctypes.byref(dr), ctypes.byref(do),
                                          _lib.stream_handle(keys_vision.device)), "rotate_keys")
    return out


def channel_scores(keys_vision: torch.Tensor, R_full: torch.Tensor) -> torch.Tensor:
    """mean_s |keys_vision @ R_full| per rotated channel -> [B,H,Dc] float64."""
    _gpu(keys_vision, "keys_vision")
    B, H = keys_vision.shape[:2]
    lib = _lib.load()
    scores = torch.empty(B, H, R_full.shape[-1], device=keys_vision.device, dtype=torch.float64)
    dk, dr, ds = _lib.desc(keys_vision), _lib.desc(R_full), _lib.desc(scores)
    need = ctypes.c_size_t(0)
    _lib.check(lib.rk_channel_scores_check(ctypes.byref(dk), ctypes.byref(dr), ctypes.byref(ds), 0,
                                           ctypes.byref(need)), "channel_scores")
    ws = torch.empty(max(need.value, 256), dtype=torch.uint8, device=keys_vision.device)
    _lib.check(lib.rk_channel_scores(ctypes.byref(dk), ctypes.byref(dr), ctypes.byref(ds), ws.data_ptr(),
                                     ws.numel(), _lib.stream_handle(keys_vision.device)), "channel_scores")
    return scores


def topk_channels(scores: torch.Tensor, k: int):
    """Head-wise top-k of ``scores`` [B,H,D] (float64): (indices [B,H,k] int64
    ascending, keep mask [B,H,D] bool).  Ties go to the lower channel."""
    _gpu(scores, "scores")
    B, H, D = scores.shape
    idx = torch.empty(B, H, k, device=scores.device, dtype=torch.int64)
    mask = torch.empty(B, H, D, device=scores.device, dtype=torch.uint8)
    ds, di, dm = _lib.desc(scores), _lib.desc(idx), _lib.desc(mask)
    _lib.check(_lib.load().rk_topk_channels(ctypes.byref(ds), int(k), ctypes.byref(di), ctypes.byref(dm),
                                            _lib.stream_handle(scores.device)), "topk_channels")
    return idx, mask.bool()


def gather_rotation(R_full: torch.Tensor, idx: torch.Tensor, mean: torch.Tensor, dtype: torch.dtype):
    """(R_partial [B,H,D,k], delta_mu [B,H,D]) in ``dtype`` from the columns
    ``idx`` of ``R_full`` and the fp32 Key mean."""
    _gpu(R_full, "R_full")
    B, H, D = mean.shape
    k = idx.shape[-1]
    Rp = torch.empty(B, H, D, k, device=R_full.device, dtype=dtype)
    dmu = torch.empty(B, H, D, device=R_full.device, dtype=dtype)
    d = [_lib.desc(t) for t in (R_full, idx, mean, Rp, dmu)]
    _lib.check(_lib.load().rk_gather_rotation(*[ctypes.byref(x) for x in d],
                                              _lib.stream_handle(R_full.device)), "gather_rotation")
    return Rp, dmu


def query_weight(cov: torch.Tensor, query_states: torch.Tensor, num_key_value_groups: int,
                 out: torch.Tensor | None = None) -> torch.Tensor:
    """Query-aware weighting of the covariance (kv_pruning_utils.py:116-140)
    in one HIP kernel (``rk_query_weight``): the last ``QUERY_WINDOW``
    queries, group-mean H_q -> H_kv in the query dtype, per-channel L2 norm
    over tokens floored at 1e-3 x the lower median, ``cov * outer(qn, qn)``,
    symmetrised, plus a ridge of 1e-4 x max(mean|diag|, 1e-6) on the
    diagonal (the clamp binds to the mean, kv_pruning_utils.py:137-139).
    ``out`` may be ``cov`` itself."""
    _gpu(cov, "cov")
    if out is None:
        out = torch.empty_like(cov)
    dc, dq, do = _lib.desc(cov), _lib.desc(query_states), _lib.desc(out)
    _lib.check(_lib.load().rk_query_weight(ctypes.byref(dc), ctypes.byref(dq), int(num_key_value_groups),
                                           QUERY_WINDOW, ctypes.byref(do), _lib.stream_handle(cov.device)),
               "query_weight")
    return out


# ROTATEK_EIGH: "device" (default) runs torch.linalg.eigh on the GPU; "host"
# copies the covariances to the CPU first, as the reference does
# (kv_pruning_utils.py:148).  On MI355X the device solver takes ~2.2 ms for 32
# 128 x 128 matrices against ~19 ms on the host, with the same fp32 accuracy.
_EIGH_ON_HOST = os.environ.get("ROTATEK_EIGH", "device").strip().lower() == "host"


def eigen_rotation(cov: torch.Tensor, on_host: bool | None = None) -> torch.Tensor:
    """All eigenvectors of ``cov`` [B,H,D,D] as columns, eigenvalue-descending
    (eigh, flipped; kv_pruning_utils.py:146-150).  The decomposition stays in
    torch; ``on_host`` (default from ``ROTATEK_EIGH``) selects the reference's
    LAPACK-on-CPU route instead of the device solver."""
    host = _EIGH_ON_HOST if on_host is None else on_host
    src = cov.cpu() if host else cov
    _, vecs = torch.linalg.eigh(src)
    return vecs.flip(dims=[-1]).to(cov.device, non_blocking=True)


__all__ = ["key_covariance", "rotate_keys", "channel_scores", "topk_channels", "gather_rotation",
           "query_weight", "eigen_rotation", "QUERY_WINDOW"]
