"""ThinK channel pruning on the HIP device (drop-in for
rotatek/baselines/think.py:15-58).

One launch chain (``rk_think_score_and_compact``): split-S sums of
dtype(k^2), the per-head selection, and the compact gather.  The channel
score and its rounding follow the reference's torch ops on the GPU
(``pow``, 16-bit ``mean``, the product in the key dtype); the
``prune_count`` smallest scores are pruned, equal scores at the boundary
lowest channel first, as torch's GPU ``topk(largest=False)`` picks them.
"""
from __future__ import annotations

import ctypes
from typing import Tuple

import torch

from rotatek_amd import _lib


def think_score_and_compact(
    keys_vision: torch.Tensor,
    queries_recent: torch.Tensor,
    num_kv_heads: int,
    prune_count: int,
) -> Tuple[torch.Tensor, torch.Tensor]:
    """ThinK score + top-k + gather + bool mask (think.py:15-58).

    ``keys_vision`` [B, H_kv, S_v, D] and ``queries_recent`` [B, H_q, Q, D]
    (already sliced to the query window, same dtype); returns
    ``K_compact`` [B, H_kv, S_v, D - prune_count] (kept channels in ascending
    order) and ``keep_mask`` [B, H_kv, D] bool, for any head dim ``D`` <= 128.
    """
    if not keys_vision.is_cuda:
        raise RuntimeError("keys_vision must be a GPU tensor: the ThinK kernels run only on the HIP device")
    B, H, S, D = keys_vision.shape
    keep = D - int(prune_count)
    dev = keys_vision.device
    K_compact = torch.empty(B, H, S, max(keep, 0), device=dev, dtype=keys_vision.dtype)
    keep_mask = torch.empty(B, H, D, device=dev, dtype=torch.bool)
    dk, dq, dc, dm = (_lib.desc(t) for t in (keys_vision, queries_recent, K_compact, keep_mask))
    lib = _lib.load()
    need = ctypes.c_size_t(0)
    args = (ctypes.byref(dk), ctypes.byref(dq), int(num_kv_heads), int(prune_count), ctypes.byref(dc),
            ctypes.byref(dm))
    _lib.check(lib.rk_think_score_and_compact_check(*args, 0, ctypes.byref(need)), "think_score_and_compact")
    ws = torch.empty(max(need.value, 256), dtype=torch.uint8, device=dev)
    _lib.check(lib.rk_think_score_and_compact(*args, ws.data_ptr(), ws.numel(), _lib.stream_handle(dev)),
               "think_score_and_compact")
    return K_compact, keep_mask


__all__ = ["think_score_and_compact"]
