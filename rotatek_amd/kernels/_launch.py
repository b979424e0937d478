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
    refs = [_lib.ref(x) for x in d]

    def launch(ws):
        return lib.rk_rotatek_decode(*refs, int(num_kv_groups), ctypes.byref(do), policy, ws.data_ptr(),
                                     ws.numel(), _lib.stream_handle(q_full.device))

    # the cached workspace first (the entry validates everything and checks
    # its size before it launches); sized by the query only when it is short
    st = launch(_lib.workspace(q_full.device, 0))
    if st == _lib.RK_ERR_WORKSPACE:
        need = ctypes.c_size_t(0)
        _lib.check(lib.rk_rotatek_decode_check(*refs, int(num_kv_groups), ctypes.byref(do), policy, 0,
                                               ctypes.byref(need)), "rotatek_decode")
        st = launch(_lib.workspace(q_full.device, need.value))
    _lib.check(st, "rotatek_decode")
    return out


def full_channel_decode(q, k, v, num_kv_groups: int, policy: int) -> torch.Tensor:
    bsz, heads, head_dim = q.shape
    _require_gpu(q, "q")
    lib = _lib.load()
    dq, dk, dv = _lib.desc(q), _lib.desc(k), _lib.desc(v)
    out = torch.empty((bsz, heads, head_dim), dtype=q.dtype, device=q.device)
    do = _lib.desc(out)
    refs = (ctypes.byref(dq), ctypes.byref(dk), ctypes.byref(dv))

    def launch(ws):
        return lib.rk_full_channel_decode(*refs, int(num_kv_groups), ctypes.byref(do), policy, ws.data_ptr(),
                                          ws.numel(), _lib.stream_handle(q.device))

    st = launch(_lib.workspace(q.device, 0))
    if st == _lib.RK_ERR_WORKSPACE:
        need = ctypes.c_size_t(0)
        _lib.check(lib.rk_full_channel_decode_check(*refs, int(num_kv_groups), ctypes.byref(do), policy, 0,
                                                    ctypes.byref(need)), "full_channel_decode")
        st = launch(_lib.workspace(q.device, need.value))
    _lib.check(st, "full_channel_decode")
    return out


def rotatek_decode_varlen(q_full, R_partial, delta_mu, k_full, v_buf, v_gap_at: int, v_gap: int,
                          mask_full, k_sparse, v_sparse, num_kv_groups: int, len_full: torch.Tensor,
                          policy: int, out: torch.Tensor | None = None, k_new=None,
                          v_new=None) -> torch.Tensor:
    """RotateK decode over capacity-sized span buffers (rk_rotatek_decode_varlen).

    ``k_full [B,H_kv,C,D]`` holds prompt then text Keys; ``v_buf`` holds the
    Values with the visual span between prompt and text (logical row ``t``
    at ``t + v_gap`` once ``t >= v_gap_at``); only rows ``t < len_full[b]``
    (device int32) are attended.  Shapes stay fixed as the cache grows, so
    the launch can be captured once and replayed every decode step.
    With ``k_new`` / ``v_new`` ([B,H_kv,1,D]) the step first appends that
    token (attended, stored at row ``len_full[b]``, length advanced).
    """
    _require_gpu(q_full, "q_full")
    if len_full.dtype != torch.int32 or not len_full.is_cuda or len_full.dim() != 1 \
            or len_full.shape[0] != q_full.shape[0] or not len_full.is_contiguous():
        raise ValueError("len_full must be a contiguous device int32 tensor [B]")
    lib = _lib.load()
    d = [_lib.desc(t) for t in (q_full, R_partial, delta_mu, k_full, v_buf, mask_full, k_sparse, v_sparse)]
    if out is None:
        out = torch.empty(q_full.shape, dtype=q_full.dtype, device=q_full.device)
    do = _lib.desc(out)
    dkn, dvn = _lib.desc(k_new), _lib.desc(v_new)
    head, tail = [_lib.ref(x) for x in d[:5]], [_lib.ref(x) for x in d[5:]]

    def launch(ws):
        return lib.rk_rotatek_decode_varlen(*head, int(v_gap_at), int(v_gap), *tail, int(num_kv_groups),
                                            _lib.ref(dkn), _lib.ref(dvn), len_full.data_ptr(), ctypes.byref(do),
                                            policy, ws.data_ptr(), ws.numel(), _lib.stream_handle(q_full.device))

    # the cached workspace first (a captured step finds it pre-sized); sized
    # by the query only when it is short
    st = launch(_lib.workspace(q_full.device, 0))
    if st == _lib.RK_ERR_WORKSPACE:
        need = varlen_workspace_bytes(q_full, R_partial, delta_mu, k_full, v_buf, mask_full, k_sparse,
                                      v_sparse, num_kv_groups, policy)
        st = launch(_lib.workspace(q_full.device, need))
    _lib.check(st, "rotatek_decode_varlen")
    return out


def varlen_workspace_bytes(q_full, R_partial, delta_mu, k_full, v_buf, mask_full, k_sparse, v_sparse,
                           num_kv_groups: int, policy: int) -> int:
    """Workspace bytes ``rotatek_decode_varlen`` needs (host-only; the plan
    depends only on the capacity-sized shapes)."""
    S_f = k_full.shape[2]
    d = [_lib.desc(t) for t in (q_full, R_partial, delta_mu, k_full, None, mask_full, k_sparse, v_sparse)]
    d[4] = _lib.desc(v_buf.narrow(2, 0, min(S_f, v_buf.shape[2])))
    need = ctypes.c_size_t(0)
    _lib.check(_lib.load().rk_rotatek_decode_check(*[_lib.ref(x) for x in d], int(num_kv_groups), None, policy,
                                                   0, ctypes.byref(need)),
               "rotatek_decode_varlen")
    return need.value


def append_kv(k_new, v_new, k_buf, v_buf, len_full: torch.Tensor) -> None:
    """Write one token's K/V [B,H,1,D] at row ``len_full[b]`` of the span
    buffers and advance ``len_full`` on the device (rk_append_kv)."""
    _require_gpu(k_buf, "k_buf")
    if len_full.dtype != torch.int32 or not len_full.is_cuda or not len_full.is_contiguous():
        raise ValueError("len_full must be a contiguous device int32 tensor [B]")
    if len_full.numel() != k_buf.shape[0]:
        raise ValueError("len_full must hold one length per batch row")
    d = [_lib.desc(t) for t in (k_new, v_new, k_buf, v_buf)]
    _lib.check(_lib.load().rk_append_kv(*[_lib.ref(x) for x in d], len_full.data_ptr(),
                                        _lib.stream_handle(k_buf.device)),
               "append_kv")
