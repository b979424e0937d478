"""Storage-precision emulation for the oracle (test infrastructure only).

The reference stores Keys, rotations and outputs in fp16 / bf16 and computes
in fp32 (e.g. kv_pruning_utils.py:113-114 rounds the centered Keys and the
covariance einsum to the key dtype).  These helpers round float arrays to
those formats with IEEE round-to-nearest-even and return them as float64 /
float32 so later arithmetic can proceed at oracle precision.

Pinned by: tests/test_oracle_numerics.py (exhaustive agreement with numpy's
float16 cast for fp16; bit-level checks of bf16 rounding on ties, carries,
infinities and NaN).
"""
from __future__ import annotations

import numpy as np

DTYPES = ("float16", "bfloat16", "float32", "float64")


def round_bf16(x) -> np.ndarray:
    """Round to bfloat16 (RNE) and return float32 values."""
    f = np.asarray(x, dtype=np.float32)
    u = f.view(np.uint32).astype(np.uint64)
    lsb = (u >> 16) & 1
    r = ((u + 0x7FFF + lsb) >> 16) << 16
    r = r.astype(np.uint32)
    nan = np.isnan(f)
    if np.any(nan):
        r = np.where(nan, np.uint32(0x7FC00000), r)
    return r.view(np.float32)


def bf16_bits(x) -> np.ndarray:
    """uint16 bit patterns of ``round_bf16(x)``."""
    return (round_bf16(x).view(np.uint32) >> 16).astype(np.uint16)


def from_bf16_bits(bits) -> np.ndarray:
    """float32 values of bfloat16 bit patterns."""
    return (np.asarray(bits, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def round_to(x, dtype: str) -> np.ndarray:
    """Round ``x`` to storage ``dtype`` and return it in float64."""
    if dtype == "float16":
        return np.asarray(x, dtype=np.float32).astype(np.float16).astype(np.float64)
    if dtype == "bfloat16":
        return round_bf16(x).astype(np.float64)
    if dtype == "float32":
        return np.asarray(x, dtype=np.float32).astype(np.float64)
    if dtype == "float64":
        return np.asarray(x, dtype=np.float64)
    raise ValueError(f"unknown dtype {dtype!r}")


def mean_factor(n_out: int, n_in: int) -> np.float32:
    """torch's GPU mean factor ``float(n_out) / float(n_in)`` in fp32 (ATen
    MeanOps multiplies the fp32 sum by it; inf when ``n_in`` is 0, so the
    mean of nothing is NaN)."""
    with np.errstate(divide="ignore", invalid="ignore"):
        return np.float32(np.float32(n_out) / np.float32(n_in))
