"""ctypes binding of ``librotatek_hip.so`` (declared in include/rotatek_hip.h).

The library is the only compute path: if it is missing, every entry point
raises ``RuntimeError`` telling the caller to build it; there is no CPU or
PyTorch fallback.  Torch is used here only to pass device pointers, strides
and the current HIP stream, and to allocate the cached decode workspace.
"""
from __future__ import annotations

import ctypes
import os
import struct
import threading

import torch

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "librotatek_hip.so")

RK_F16, RK_BF16, RK_F32, RK_F64, RK_U8, RK_I32, RK_I64 = range(7)
RK_POLICY_PAPER, RK_POLICY_GQA = 0, 1
# rk_status (include/rotatek_hip.h)
(RK_OK, RK_ERR_NULL, RK_ERR_RANK, RK_ERR_DTYPE, RK_ERR_SHAPE, RK_ERR_HEADS, RK_ERR_HEAD_DIM, RK_ERR_KEEP_DIM,
 RK_ERR_STRIDE, RK_ERR_WORKSPACE, RK_ERR_ARG, RK_ERR_HIP, RK_ERR_NO_DEVICE,
 RK_ERR_SCRATCH) = (0, -1, -2, -3, -4, -5, -6, -7, -8, -9, -10, -11, -12, -13)
NOALLOC_SCRATCH_BYTES = 16 * 1024 * 1024  # RK_NOALLOC_SCRATCH_BYTES

_DTYPES = {
    torch.float16: RK_F16,
    torch.bfloat16: RK_BF16,
    torch.float32: RK_F32,
    torch.float64: RK_F64,
    torch.uint8: RK_U8,
    torch.bool: RK_U8,
    torch.int32: RK_I32,
    torch.int64: RK_I64,
}

# status codes whose Python counterpart is ValueError (bad arguments)
_VALUE_ERRORS = {-2, -3, -4, -5, -6, -7, -8, -10, -13}


class RkTensor(ctypes.Structure):
    _fields_ = [
        ("data", ctypes.c_void_p),
        ("dtype", ctypes.c_int32),
        ("ndim", ctypes.c_int32),
        ("shape", ctypes.c_int64 * 4),
        ("stride", ctypes.c_int64 * 4),
    ]


class RkDecodePlan(ctypes.Structure):
    _fields_ = [
        ("units", ctypes.c_int64),
        ("heads_per_unit", ctypes.c_int32),
        ("head_blocks", ctypes.c_int32),
        ("wg_vis", ctypes.c_int32),
        ("wg_full", ctypes.c_int32),
        ("chunk_vis", ctypes.c_int64),
        ("chunk_full", ctypes.c_int64),
        ("grid", ctypes.c_int64),
        ("workspace_bytes", ctypes.c_size_t),
        ("single_launch", ctypes.c_int32),
        ("chunk_major", ctypes.c_int32),
        ("n_fast", ctypes.c_int32),
        ("chunk_fast", ctypes.c_int64),
    ]


_P = ctypes.POINTER(RkTensor)
_SIGNATURES = {
    "rk_strerror": (ctypes.c_char_p, [ctypes.c_int]),
    "rk_abi_version": (ctypes.c_int, []),
    "rk_device_cu_count": (ctypes.c_int, [ctypes.c_int, ctypes.POINTER(ctypes.c_int)]),
    "rk_rotatek_decode_check": (ctypes.c_int, [_P, _P, _P, _P, _P, _P, _P, _P, ctypes.c_int64, _P,
                                               ctypes.c_int32, ctypes.c_int32,
                                               ctypes.POINTER(ctypes.c_size_t)]),
    "rk_rotatek_decode": (ctypes.c_int, [_P, _P, _P, _P, _P, _P, _P, _P, ctypes.c_int64, _P,
                                         ctypes.c_int32, ctypes.c_void_p, ctypes.c_size_t,
                                         ctypes.c_void_p]),
    "rk_rotatek_decode_noalloc": (ctypes.c_int, [_P, _P, _P, _P, _P, _P, _P, _P, ctypes.c_int64, _P,
                                                 ctypes.c_int32, ctypes.c_void_p]),
    "rk_rotatek_decode_varlen": (ctypes.c_int, [_P, _P, _P, _P, _P, ctypes.c_int64, ctypes.c_int64, _P, _P, _P,
                                                ctypes.c_int64, _P, _P, ctypes.c_void_p, _P, ctypes.c_int32,
                                                ctypes.c_void_p, ctypes.c_size_t, ctypes.c_void_p]),
    "rk_query_weight": (ctypes.c_int, [_P, _P, ctypes.c_int64, ctypes.c_int32, _P, ctypes.c_void_p]),
    "rk_power_iteration": (ctypes.c_int, [_P, _P, _P, ctypes.c_int32, ctypes.c_float, ctypes.c_void_p,
                                          ctypes.c_void_p]),
    "rk_append_kv": (ctypes.c_int, [_P, _P, _P, _P, ctypes.c_void_p, ctypes.c_void_p]),
    "rk_full_channel_decode_check": (ctypes.c_int, [_P, _P, _P, ctypes.c_int64, _P, ctypes.c_int32,
                                                    ctypes.c_int32, ctypes.POINTER(ctypes.c_size_t)]),
    "rk_full_channel_decode": (ctypes.c_int, [_P, _P, _P, ctypes.c_int64, _P, ctypes.c_int32,
                                              ctypes.c_void_p, ctypes.c_size_t, ctypes.c_void_p]),
    "rk_plan_decode": (ctypes.c_int, [ctypes.c_int64] * 6 + [ctypes.c_int32] * 3
                       + [ctypes.POINTER(RkDecodePlan)]),
    "rk_set_decode_tuning": (None, [ctypes.c_int64, ctypes.c_int64, ctypes.c_int32]),
    "rk_set_decode_merge": (None, [ctypes.c_int32]),
    "rk_set_decode_chunk_align": (None, [ctypes.c_int32]),
    "rk_set_decode_skew": (None, [ctypes.c_int32]),
    "rk_decode_workspace_init": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_size_t, ctypes.c_void_p]),
    "rk_decode_workspace_release": (None, [ctypes.c_void_p]),
    "rk_key_covariance_check": (ctypes.c_int, [_P, _P, _P, ctypes.c_int32, ctypes.POINTER(ctypes.c_size_t)]),
    "rk_key_covariance": (ctypes.c_int, [_P, _P, _P, ctypes.c_void_p, ctypes.c_size_t, ctypes.c_void_p]),
    "rk_key_covariance_weighted_check": (ctypes.c_int, [_P, _P, ctypes.c_int64, ctypes.c_int32, _P, _P,
                                                        ctypes.c_int32, ctypes.POINTER(ctypes.c_size_t)]),
    "rk_key_covariance_weighted": (ctypes.c_int, [_P, _P, ctypes.c_int64, ctypes.c_int32, _P, _P,
                                                  ctypes.c_void_p, ctypes.c_size_t, ctypes.c_void_p]),
    "rk_rotate_keys": (ctypes.c_int, [_P, _P, _P, ctypes.c_void_p]),
    "rk_channel_scores_check": (ctypes.c_int, [_P, _P, _P, ctypes.c_int32, ctypes.POINTER(ctypes.c_size_t)]),
    "rk_channel_scores": (ctypes.c_int, [_P, _P, _P, ctypes.c_void_p, ctypes.c_size_t, ctypes.c_void_p]),
    "rk_topk_channels": (ctypes.c_int, [_P, ctypes.c_int64, _P, _P, ctypes.c_void_p]),
    "rk_gather_rotation": (ctypes.c_int, [_P, _P, _P, _P, _P, ctypes.c_void_p]),
    "rk_think_score_and_compact_check": (ctypes.c_int, [_P, _P, ctypes.c_int64, ctypes.c_int64, _P, _P,
                                                        ctypes.c_int32, ctypes.POINTER(ctypes.c_size_t)]),
    "rk_think_score_and_compact": (ctypes.c_int, [_P, _P, ctypes.c_int64, ctypes.c_int64, _P, _P,
                                                  ctypes.c_void_p, ctypes.c_size_t, ctypes.c_void_p]),
    "rk_spark_prune_check": (ctypes.c_int, [_P, _P, ctypes.c_int64, ctypes.c_int64, _P, _P, _P,
                                            ctypes.c_int32, ctypes.POINTER(ctypes.c_size_t)]),
    "rk_spark_prune": (ctypes.c_int, [_P, _P, ctypes.c_int64, ctypes.c_int64, _P, _P, _P,
                                      ctypes.c_void_p, ctypes.c_size_t, ctypes.c_void_p]),
    "rk_think_recover_check": (ctypes.c_int, [_P, _P, _P, _P, _P]),
    "rk_think_recover": (ctypes.c_int, [_P, _P, _P, _P, _P, ctypes.c_void_p]),
    "rk_spark_recover_check": (ctypes.c_int, [_P, _P, _P, _P, _P, _P]),
    "rk_spark_recover": (ctypes.c_int, [_P, _P, _P, _P, _P, _P, ctypes.c_void_p]),
    "rk_channel_selection": (ctypes.c_int, [_P, _P, ctypes.c_void_p]),
}

_lib = None
_lock = threading.Lock()
ABI_VERSION = 3  # RK_ABI_VERSION of include/rotatek_hip.h


class HipLibraryMissing(RuntimeError):
    pass


def load(path: str = LIB_PATH) -> ctypes.CDLL:
    """Load (once) and return the HIP library with typed signatures."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is None:
            if not os.path.exists(path):
                raise HipLibraryMissing(
                    f"{path} is not built; run `python -m rotatek_amd.build` "
                    "(there is no CPU fallback for the RotateK kernels)")
            lib = ctypes.CDLL(path)
            lib.rk_abi_version.restype = ctypes.c_int
            if lib.rk_abi_version() != ABI_VERSION:
                raise HipLibraryMissing(
                    f"{path} has ABI version {lib.rk_abi_version()}, this package needs {ABI_VERSION}; "
                    "rebuild with `python -m rotatek_amd.build`")
            for name, (res, args) in _SIGNATURES.items():
                fn = getattr(lib, name)
                fn.restype = res
                fn.argtypes = args
            _lib = lib
    return _lib


def strerror(status: int) -> str:
    return load().rk_strerror(status).decode()


def check(status: int, what: str) -> None:
    if status == 0:
        return
    msg = f"{what}: {strerror(status)} (status {status})"
    if status in _VALUE_ERRORS:
        raise ValueError(msg)
    raise RuntimeError(msg)


# rk_tensor's layout: data, dtype, ndim, shape[4], stride[4] (80 bytes)
_RK_TENSOR = struct.Struct("=Qii4q4q")
_PAD = ((), (0,), (0, 0), (0, 0, 0), (0, 0, 0, 0))


def desc(t: torch.Tensor | None):
    """rk_tensor descriptor of a torch tensor (None -> NULL pointer).  Packed
    in one step (a field-by-field ctypes fill costs ~4 us per tensor, most of
    an eager decode call's host time); entries past ndim are zero."""
    if t is None:
        return None
    nd = t.dim()
    if nd > 4:
        raise ValueError("tensors of rank > 4 are not supported")
    code = _DTYPES.get(t.dtype)
    if code is None:
        raise ValueError(f"unsupported dtype {t.dtype}")
    pad = _PAD[4 - nd]
    return RkTensor.from_buffer_copy(_RK_TENSOR.pack(t.data_ptr() if t.numel() > 0 else 0, code, nd,
                                                     *t.shape, *pad, *t.stride(), *pad))


def ref(d):
    return None if d is None else ctypes.byref(d)


def stream_handle(device: torch.device) -> int:
    return torch.cuda.current_stream(device).cuda_stream


# ---------------------------------------------------------------- workspace
_WORKSPACE: dict = {}
# Buffers a larger request replaced.  A captured HIP graph keeps the address
# it was recorded with, so a replaced buffer is never handed back to the
# allocator: graph replays keep writing memory that no other tensor owns.
_RETIRED: list = []


def workspace(device: torch.device, nbytes: int) -> torch.Tensor:
    """Decode workspace (split partials), cached per device and grown on
    demand, so steady-state calls allocate nothing.  A graph captured with
    one buffer stays valid after a later call grows the workspace: the old
    buffer is retired, not freed; growth is by at least half the current
    size, so a run of growing shapes retires few buffers.  Concurrent
    decodes on different streams of one device share it and must not
    overlap."""
    idx = device.index if device.index is not None else torch.cuda.current_device()
    buf = _WORKSPACE.get(idx)
    if buf is None or buf.numel() < nbytes:
        size = max(nbytes, 256)
        if buf is not None:
            _RETIRED.append(buf)
            size = max(size, buf.numel() * 3 // 2)
        dev = torch.device("cuda", idx)
        buf = torch.empty(size, dtype=torch.uint8, device=dev)
        # the single-launch merge's counters start at zero (every call leaves them so)
        check(load().rk_decode_workspace_init(buf.data_ptr(), buf.numel(), stream_handle(dev)),
              "decode_workspace_init")
        _WORKSPACE[idx] = buf
    return buf


def plan_decode(B, H_q, H_kv, Dk, S_v, S_f, elem_bytes=2, policy=RK_POLICY_GQA, num_cus=256):
    p = RkDecodePlan()
    check(load().rk_plan_decode(B, H_q, H_kv, Dk, S_v, S_f, elem_bytes, policy, num_cus,
                                ctypes.byref(p)), "rk_plan_decode")
    return {f: getattr(p, f) for f, _ in RkDecodePlan._fields_}


def set_decode_tuning(min_bytes=0, max_bytes=0, wgs_per_cu=0):
    """Planner overrides for sweeps: workgroup byte bounds and workgroups per
    CU (0 keeps a value; ``wgs_per_cu < 0`` restores the default, two per CU
    or one for a single round of small chunk-major workgroups)."""
    load().rk_set_decode_tuning(int(min_bytes), int(max_bytes), int(wgs_per_cu))


def set_decode_chunk_align(tokens: int) -> None:
    """Visual chunk granularity of the decode planner (32, 64 or 128 tokens;
    0 = the default: 32 in a chunk-major grid, else 128)."""
    load().rk_set_decode_chunk_align(int(tokens))


def set_decode_skew(permille: int) -> None:
    """One-round decode grids of short workgroups: 0 = unit-major launch,
    1000 = chunk-major with equal chunks, 1001..4000 = chunk-major with the
    first-dispatched chunks of <= 128 KB workgroups given this many
    thousandths of the others' tokens (default 1300)."""
    load().rk_set_decode_skew(int(permille))


MERGE_AUTO, MERGE_TWO_LAUNCHES, MERGE_SINGLE_LAUNCH = 0, 1, 2
DECODE_TICKET_BYTES = 256 * 1024  # RK_DECODE_TICKET_BYTES


def set_decode_merge(mode: int) -> None:
    """Decode merge: MERGE_AUTO (the default: one launch for a single round
    of one-query-head units, else two), MERGE_TWO_LAUNCHES or
    MERGE_SINGLE_LAUNCH (bit-identical results)."""
    load().rk_set_decode_merge(int(mode))
