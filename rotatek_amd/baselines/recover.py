"""Decode-time recovery of full-width visual Keys for the ThinK / SparK
baselines (drop-in for llama_visionzip.py:216-233 and
qwen2_5vl_visionzip.py:996-1008).

The reference builds a zero (ThinK) or pruned-mean (SparK) filled
[B, H, S_v, D] tensor, scatters the compact Keys into it with a boolean
index, then ``torch.cat``s prompt, recovered and text Keys for the dense
decode.  Here one HIP launch writes the recovered rows straight into
``out`` (which may be a slice of a preallocated buffer) and, given
``k_prompt`` / ``k_text``, the prompt and text rows around them, so the
concatenation is the same pass.
"""
from __future__ import annotations

import ctypes

import torch

from rotatek_amd import _lib


def _out(key_pruned, mask, k_prompt, k_text, out):
    """The output rows [B, H, rows, D], D the mask's channel count."""
    B, H, S, _ = key_pruned.shape
    rows = S + (0 if k_prompt is None else k_prompt.shape[2]) + (0 if k_text is None else k_text.shape[2])
    if out is None:
        out = torch.empty(B, H, rows, mask.shape[-1], device=key_pruned.device, dtype=key_pruned.dtype)
    return out


def recover_think(key_pruned: torch.Tensor, think_mask: torch.Tensor, out: torch.Tensor | None = None,
                  k_prompt: torch.Tensor | None = None, k_text: torch.Tensor | None = None) -> torch.Tensor:
    """[prompt |] recovered [| text] Keys: kept channels of each head (``think_mask``
    [B,H,D], True = kept; D <= 128) from ``key_pruned`` [B,H,S_v,D_keep] in
    ascending channel order, pruned channels 0 (llama_visionzip.py:219-225)."""
    if not key_pruned.is_cuda:
        raise RuntimeError("key_pruned must be a GPU tensor: the recovery kernels run only on the HIP device")
    out = _out(key_pruned, think_mask, k_prompt, k_text, out)
    d = [_lib.desc(t) for t in (k_prompt, key_pruned, k_text, think_mask, out)]
    _lib.check(_lib.load().rk_think_recover(*[_lib.ref(x) for x in d], _lib.stream_handle(key_pruned.device)),
               "recover_think")
    return out


def recover_spark(key_pruned: torch.Tensor, spark_mask: torch.Tensor, pruned_mean: torch.Tensor,
                  out: torch.Tensor | None = None, k_prompt: torch.Tensor | None = None,
                  k_text: torch.Tensor | None = None) -> torch.Tensor:
    """[prompt |] recovered [| text] Keys: each token's kept channels
    (``spark_mask`` [B,H,S_v,D]) from ``key_pruned`` in ascending channel
    order, the others = ``pruned_mean`` [B,H,S_v,1] (llama_visionzip.py:226-230)."""
    if not key_pruned.is_cuda:
        raise RuntimeError("key_pruned must be a GPU tensor: the recovery kernels run only on the HIP device")
    out = _out(key_pruned, spark_mask, k_prompt, k_text, out)
    d = [_lib.desc(t) for t in (k_prompt, key_pruned, k_text, spark_mask, pruned_mean, out)]
    _lib.check(_lib.load().rk_spark_recover(*[_lib.ref(x) for x in d], _lib.stream_handle(key_pruned.device)),
               "recover_spark")
    return out


def selection_rotation(think_mask: torch.Tensor, keep: int, dtype: torch.dtype) -> torch.Tensor:
    """One-hot R [B,H,D,keep]: R[c, j] = 1 iff c is the j-th kept channel.

    With it, ``q R`` gathers the kept query channels, so the RotateK decode
    (``delta_mu=None``) over ``K_compact`` computes exactly ThinK's
    attention over zero-filled Keys without materialising them."""
    B, H, D = think_mask.shape
    R = torch.empty(B, H, D, keep, device=think_mask.device, dtype=dtype)
    dm, dr = _lib.desc(think_mask), _lib.desc(R)
    _lib.check(_lib.load().rk_channel_selection(ctypes.byref(dm), ctypes.byref(dr),
                                                _lib.stream_handle(think_mask.device)), "selection_rotation")
    return R


__all__ = ["recover_think", "recover_spark", "selection_rotation"]
