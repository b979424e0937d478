"""SparK per-token channel pruning on the HIP device (drop-in for
rotatek/baselines/spark.py:15-60).

``spark_prune`` is the whole prefill step of ``update_spark``
(kv_pruning_utils.py:63-90): the mean of the G query heads of each KV head,
the per-channel L2 norm over the window, and one wave per visual token that
scores its D <= 128 channels, keeps the ``D - prune_count`` largest (equal scores
lowest channel first, as torch's GPU argsort(descending) orders them) by a
radix select, and writes the compact Keys, the per-token mask and the mean
of the pruned values.  ``per_token_channel_prune`` is the reference's
function on already-grouped queries.
"""
from __future__ import annotations

import ctypes
from typing import Tuple

import torch

from rotatek_amd import _lib


def spark_prune(keys_vision: torch.Tensor, queries: torch.Tensor, num_kv_groups: int,
                prune_count: int) -> Tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """(K_compact [B,H,S,D-prune], keep_mask [B,H,S,D] bool, pruned_mean
    [B,H,S,1]) from ``keys_vision`` [B,H,S,D] and the query window
    ``queries`` [B, H*num_kv_groups, W, D] (grouped in the kernel)."""
    if not keys_vision.is_cuda:
        raise RuntimeError("keys_vision must be a GPU tensor: the SparK kernels run only on the HIP device")
    B, H, S, D = keys_vision.shape
    keep = D - int(prune_count)
    dev, dt = keys_vision.device, keys_vision.dtype
    K_compact = torch.empty(B, H, S, max(keep, 0), device=dev, dtype=dt)
    keep_mask = torch.empty(B, H, S, D, device=dev, dtype=torch.bool)
    pruned_mean = torch.empty(B, H, S, 1, device=dev, dtype=dt)
    dk, dq, dc, dm, dp = (_lib.desc(t) for t in (keys_vision, queries, K_compact, keep_mask, pruned_mean))
    lib = _lib.load()
    need = ctypes.c_size_t(0)
    args = (ctypes.byref(dk), ctypes.byref(dq), int(num_kv_groups), int(prune_count), ctypes.byref(dc),
            ctypes.byref(dm), ctypes.byref(dp))
    _lib.check(lib.rk_spark_prune_check(*args, 0, ctypes.byref(need)), "spark_prune")
    ws = torch.empty(max(need.value, 256), dtype=torch.uint8, device=dev)
    _lib.check(lib.rk_spark_prune(*args, ws.data_ptr(), ws.numel(), _lib.stream_handle(dev)), "spark_prune")
    return K_compact, keep_mask, pruned_mean


def per_token_channel_prune(queries: torch.Tensor, keys: torch.Tensor, ratio: float):
    """Per-token channel pruning, compact storage (spark.py:15-60).

    ``queries`` [B, H, W, D] (grouped), ``keys`` [B, H, S, D] (visual
    tokens), ``ratio`` the fraction of channels to prune; returns
    ``(K_compact, keep_mask, pruned_mean)`` as the reference.
    """
    head_dim = keys.shape[-1]
    prune_count = int(head_dim * ratio)
    if not 0 <= prune_count <= head_dim:
        raise ValueError(f"ratio {ratio} prunes {prune_count} of {head_dim} channels")
    return spark_prune(keys, queries, 1, prune_count)


__all__ = ["per_token_channel_prune", "spark_prune"]
