"""Shared launcher: torch tensors -> rk_tensor descriptors -> C ABI.

Both kernel families (``paper`` and ``gqa``) launch the same HIP kernels;
the family only picks the work decomposition (one unit per query head, or
the query heads of a KV group sharing each K/V tile).
"""
from __future__ import annotations

import ctypes

import torch

from rotatek_amd import _lib


def _require_gpu(t: torch.Tensor, name: str) -> None:
    if not t.is_cuda:
        raise RuntimeError(f"{name} must be a GPU tensor: the RotateK kernels run only on the HIP device")


def rotatek_decode(q_full, R_partial, delta_mu, k_full, v_full, mask_full, k_sparse, v_sparse,
                   num_kv_groups: int, policy: int) -> torch.Tensor:
    """Validate, allocate ``out [B, H_q, D]`` (dtype of q) and launch."""
    bsz, heads, head_dim = q_full.shape
    _require_gpu(q_full, "q_full")
    lib = _lib.load()
    d = [_lib.desc(t) for t in (q_full, R_partial, delta_mu, k_full, v_full, mask_full, k_sparse,
                                v_sparse)]
    out = torch.empty((bsz, heads, head_dim), dtype=q_full.dtype, device=q_full.device)
    do = _lib.desc(out)
    need = ctypes.c_size_t(0)
    _lib.check(lib.rk_rotatek_decode_check(*[_lib.ref(x) for x in d], int(num_kv_groups),
                                           ctypes.byref(do), policy, 0, ctypes.byref(need)),
               "rotatek_decode")
    ws = _lib.workspace(q_full.device, need.value)
    _lib.check(lib.rk_rotatek_decode(*[_lib.ref(x) for x in d], int(num_kv_groups), ctypes.byref(do),
                                     policy, ws.data_ptr(), ws.numel(),
                                     _lib.stream_handle(q_full.device)),
               "rotatek_decode")
    return out


def full_channel_decode(q, k, v, num_kv_groups: int, policy: int) -> torch.Tensor:
    bsz, heads, head_dim = q.shape
    _require_gpu(q, "q")
    lib = _lib.load()
    dq, dk, dv = _lib.desc(q), _lib.desc(k), _lib.desc(v)
    out = torch.empty((bsz, heads, head_dim), dtype=q.dtype, device=q.device)
    do = _lib.desc(out)
    need = ctypes.c_size_t(0)
    _lib.check(lib.rk_full_channel_decode_check(ctypes.byref(dq), ctypes.byref(dk), ctypes.byref(dv),
                                                int(num_kv_groups), ctypes.byref(do), policy, 0,
                                                ctypes.byref(need)),
               "full_channel_decode")
    ws = _lib.workspace(q.device, need.value)
    _lib.check(lib.rk_full_channel_decode(ctypes.byref(dq), ctypes.byref(dk), ctypes.byref(dv),
                                          int(num_kv_groups), ctypes.byref(do), policy, ws.data_ptr(),
                                          ws.numel(), _lib.stream_handle(q.device)),
               "full_channel_decode")
    return out
