"""Decode-attention oracle (test infrastructure only; see ``oracle/__init__``).

Restates, on the CPU with numpy, what one RotateK decode step computes in
the reference:

* ``rotatek_decode``      closed form of rotatek/kernels/fused_decode.py:131-296
                          (sparse split kernel + combined full/merge kernel)
                          and gqa_decode.py:121-251 (same maths, query heads of
                          a KV group sharing tiles);
* ``rotatek_decode_paper_splitk``  step-by-step restatement of the paper
                          family's two kernels: split policy of
                          fused_decode.py:343-347, 64-token online-softmax
                          blocks (158-183), full-width pass with ``mask_full``
                          (243-273), sequential merge (277-290) and the
                          ``acc / (l + 1e-6)`` output (293);
* ``full_channel_decode`` closed form of full_channel_flash_decoding.py:34-155
                          (dense split-K baseline) and gqa_decode.py:67-118;
* ``rotatek_decode_torch`` the closed form as batched torch ops on CPU
                          tensors (the CPU baseline's timed restatement).

Semantics fixed by the reference and kept here:

* query head ``h`` reads KV head ``h // num_kv_groups`` (fused_decode.py:124);
* ``scale = 1/sqrt(D)`` (fused_decode.py:340);
* visual logit ``(k~ . (q R)) * scale + (q . delta_mu) * scale``
  (fused_decode.py:140-148, 167); ``delta_mu=None`` drops the bias (349-356);
* prompt/text tokens with ``mask_full == 0`` are excluded (254-258);
* the running max starts at ``-1e30`` and the output is
  ``acc / (l + 1e-6)`` with ``l`` taken relative to the global max
  (151, 238, 293; full_channel_flash_decoding.py:133, 153).

Pinned by tests/test_oracle_decode.py: a pure-Python brute force on tiny
shapes, textbook softmax attention (``scipy.special.softmax``) with HF-style
``repeat_kv`` head expansion, the rank-D_keep identity (RotateK equals dense
attention over the original Keys when ``K = 1 mu^T + Z R^T``), the single-token
``1/(1+1e-6)`` value, mask/removal equivalence, and agreement of the split-K
restatement with the closed form for every split count.
"""
from __future__ import annotations

import math

import numpy as np

NEG_INIT = -1e30   # running-max initial value (fused_decode.py:151)
DENOM_EPS = 1e-6   # output denominator guard (fused_decode.py:293)


def _f(x, dt):
    return None if x is None else np.asarray(x, dtype=dt)


def rotatek_decode(q_full, R_partial, delta_mu, k_full, v_full, mask_full,
                   k_sparse, v_sparse, num_kv_groups, compute_dtype=np.float64):
    """One RotateK decode step.  Returns ``out [B, 1, H_q, D]`` (compute dtype).

    Shapes follow fused_decode.py:303-313: q_full [B,H_q,D], R_partial
    [B,H_kv,D,Dk], delta_mu [B,H_kv,D] or None, k_full/v_full [B,H_kv,S_f,D],
    mask_full [B,S_f] (nonzero = attend), k_sparse [B,H_kv,S_v,Dk],
    v_sparse [B,H_kv,S_v,D].
    """
    dt = compute_dtype
    q = _f(q_full, dt)
    R = _f(R_partial, dt)
    dm = _f(delta_mu, dt)
    kf, vf = _f(k_full, dt), _f(v_full, dt)
    ks, vs = _f(k_sparse, dt), _f(v_sparse, dt)
    B, Hq, D = q.shape
    Hkv = R.shape[1]
    G = int(num_kv_groups)
    if Hq // G != Hkv:
        raise ValueError(f"R_partial H_kv={Hkv} but H_q={Hq}, num_kv_groups={G}")
    scale = dt(1.0 / math.sqrt(D)) if dt is not np.float64 else 1.0 / math.sqrt(D)
    mask = np.ones((B, kf.shape[2]), dtype=bool) if mask_full is None else (np.asarray(mask_full) != 0)
    out = np.zeros((B, Hq, D), dtype=dt)
    for b in range(B):
        for kv in range(Hkv):
            qg = q[b, kv * G:(kv + 1) * G]                     # [G, D]
            qt = qg @ R[b, kv]                                 # [G, Dk]
            s_vis = (qt @ ks[b, kv].T) * scale                 # [G, S_v]
            if dm is not None:
                s_vis = s_vis + (qg @ dm[b, kv])[:, None] * scale
            s_full = (qg @ kf[b, kv].T) * scale                # [G, S_f]
            s_full = np.where(mask[b][None, :], s_full, -np.inf)
            m = np.full((G, 1), NEG_INIT, dtype=dt)
            if s_vis.shape[1]:
                m = np.maximum(m, s_vis.max(axis=1, keepdims=True))
            if s_full.shape[1]:
                m = np.maximum(m, s_full.max(axis=1, keepdims=True))
            p_vis = np.exp(s_vis - m)
            p_full = np.exp(s_full - m)
            l = p_vis.sum(axis=1) + p_full.sum(axis=1)
            acc = p_vis @ vs[b, kv] + p_full @ vf[b, kv]
            out[b, kv * G:(kv + 1) * G] = acc / (l + DENOM_EPS)[:, None]
    return out[:, None]


def full_channel_decode(q, k, v, num_kv_groups=1, compute_dtype=np.float64):
    """Dense decode over full-width K/V; ``out [B, 1, H_q, D]``.

    Restates full_channel_flash_decoding.py:162-229 (and gqa_decode.py:254-277):
    identical to ``rotatek_decode`` with an empty visual span and an all-ones
    mask.
    """
    dt = compute_dtype
    q = _f(q, dt)
    k, v = _f(k, dt), _f(v, dt)
    B, Hq, D = q.shape
    Hkv = k.shape[1]
    G = int(num_kv_groups)
    empty_k = np.zeros((B, Hkv, 0, 1), dtype=dt)
    empty_v = np.zeros((B, Hkv, 0, D), dtype=dt)
    R = np.zeros((B, Hkv, D, 1), dtype=dt)
    return rotatek_decode(q, R, None, k, v, None, empty_k, empty_v, G, compute_dtype=dt)


def paper_num_splits(seq_sparse: int, block_n: int = 64) -> tuple[int, int]:
    """Split policy of fused_decode.py:343-347: (num_splits, per_split)."""
    ns = max(1, min((seq_sparse + block_n - 1) // block_n, 64))
    return ns, (seq_sparse + ns - 1) // ns


def rotatek_decode_paper_splitk(q_full, R_partial, delta_mu, k_full, v_full,
                                mask_full, k_sparse, v_sparse, num_kv_groups,
                                num_splits=None, block_n=64):
    """Step-by-step restatement of the paper family (fused_decode.py:88-296).

    Kernel 1 (88-189): per (b, h_q, split) rotate q, add q.delta_mu, walk
    64-token blocks with an online softmax, store (m, l, acc).  Kernel 2
    (207-296): full-width online softmax over prompt+text honouring
    ``mask_full``, then merge the sparse partials one by one, then
    ``acc / (l + 1e-6)``.  ``num_splits`` overrides the policy so split
    invariance can be tested.  float64 throughout.
    """
    q = np.asarray(q_full, np.float64)
    R = np.asarray(R_partial, np.float64)
    dm = None if delta_mu is None else np.asarray(delta_mu, np.float64)
    kf, vf = np.asarray(k_full, np.float64), np.asarray(v_full, np.float64)
    ks, vs = np.asarray(k_sparse, np.float64), np.asarray(v_sparse, np.float64)
    B, Hq, D = q.shape
    G = int(num_kv_groups)
    S_v, S_f = ks.shape[2], kf.shape[2]
    scale = 1.0 / math.sqrt(D)
    if num_splits is None:
        ns, per = paper_num_splits(S_v, block_n)
    else:
        ns = int(num_splits)
        per = (S_v + ns - 1) // ns
    mask = np.ones((B, S_f), bool) if mask_full is None else (np.asarray(mask_full) != 0)

    def online(m, l, acc, logits, valid, v):
        logits = np.where(valid, logits, -np.inf)
        new_m = max(m, logits.max()) if logits.size else m
        corr = math.exp(m - new_m)
        p = np.where(valid, np.exp(logits - new_m), 0.0)
        return new_m, l * corr + p.sum(), acc * corr + p @ v

    out = np.zeros((B, Hq, D))
    for b in range(B):
        for h in range(Hq):
            kv = h // G
            qh = q[b, h]
            qt = qh @ R[b, kv]
            bias = float(qh @ dm[b, kv]) if dm is not None else 0.0
            parts = []
            for s in range(ns):                                   # kernel 1
                m, l, acc = NEG_INIT, 0.0, np.zeros(D)
                start, end = s * per, min(s * per + per, S_v)
                for blk in range(0, per, block_n):
                    idx = np.arange(start + blk, start + blk + block_n)
                    valid = idx < end
                    idc = np.minimum(idx, S_v - 1)
                    logits = (ks[b, kv, idc] @ qt) * scale + bias * scale
                    v = np.where(valid[:, None], vs[b, kv, idc], 0.0)
                    m, l, acc = online(m, l, acc, logits, valid, v)
                parts.append((m, l, acc))
            m, l, acc = NEG_INIT, 0.0, np.zeros(D)               # kernel 2 (a)
            for blk in range(0, S_f, block_n):
                idx = np.arange(blk, blk + block_n)
                inb = idx < S_f
                idc = np.minimum(idx, S_f - 1)
                valid = inb & mask[b, idc]
                logits = (kf[b, kv, idc] @ qh) * scale
                v = np.where(inb[:, None], vf[b, kv, idc], 0.0)
                m, l, acc = online(m, l, acc, logits, valid, v)
            for (ms, ls, accs) in parts:                          # kernel 2 (b)
                new_m = max(m, ms)
                c, cs = math.exp(m - new_m), math.exp(ms - new_m)
                l = l * c + ls * cs
                acc = acc * c + accs * cs
                m = new_m
            out[b, h] = acc / (l + DENOM_EPS)                     # kernel 2 (c)
    return out[:, None]



def rotatek_decode_torch(q_full, R_partial, delta_mu, k_full, v_full, mask_full,
                         k_sparse, v_sparse, num_kv_groups):
    """Batched torch restatement of ``rotatek_decode`` on CPU tensors, in
    their dtype (fp32 for the CPU baseline): whole-span products over
    [B, H_kv, G, S] (the G query heads of a KV head as one matrix) instead
    of a loop over (b, kv).  Same maths as fused_decode.py:131-296: visual
    logits (q R) k~ s + (q . delta_mu) s, prompt/text logits q k s with
    ``mask_full == 0`` excluded, one softmax over both spans with the
    running max floored at -1e30, ``acc / (l + 1e-6)``.  Returns
    [B, 1, H_q, D].  Pinned by tests/test_oracle_decode.py against
    ``rotatek_decode`` (fp64) on random shapes, GQA groups, masks and empty
    spans."""
    import torch

    q = torch.as_tensor(q_full)
    B, Hq, D = q.shape
    R = torch.as_tensor(R_partial)
    Hkv = R.shape[1]
    G = int(num_kv_groups)
    if Hq // G != Hkv:
        raise ValueError(f"R_partial H_kv={Hkv} but H_q={Hq}, num_kv_groups={G}")
    scale = 1.0 / math.sqrt(D)
    qg = q.reshape(B, Hkv, G, D)
    ks, vs = torch.as_tensor(k_sparse), torch.as_tensor(v_sparse)
    kf, vf = torch.as_tensor(k_full), torch.as_tensor(v_full)
    s_vis = torch.matmul(torch.matmul(qg, R), ks.transpose(-1, -2)) * scale          # [B,Hkv,G,S_v]
    if delta_mu is not None:
        bias = torch.matmul(qg, torch.as_tensor(delta_mu).unsqueeze(-1)) * scale     # [B,Hkv,G,1]
        s_vis = s_vis + bias
    s_full = torch.matmul(qg, kf.transpose(-1, -2)) * scale                          # [B,Hkv,G,S_f]
    if mask_full is not None:
        keep = torch.as_tensor(mask_full).to(torch.bool).reshape(B, 1, 1, -1)
        s_full = s_full.masked_fill(~keep, float("-inf"))
    m = torch.full((B, Hkv, G, 1), NEG_INIT, dtype=s_vis.dtype)
    if s_vis.shape[-1]:
        m = torch.maximum(m, s_vis.amax(dim=-1, keepdim=True))
    if s_full.shape[-1]:
        m = torch.maximum(m, s_full.amax(dim=-1, keepdim=True))
    p_vis, p_full = torch.exp(s_vis - m), torch.exp(s_full - m)
    l = p_vis.sum(-1, keepdim=True) + p_full.sum(-1, keepdim=True)
    acc = torch.matmul(p_vis, vs) + torch.matmul(p_full, vf)
    return (acc / (l + DENOM_EPS)).reshape(B, Hq, D)[:, None]
