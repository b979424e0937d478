"""Write the known-answer fixtures in tests/golden/ (run from the repo root:
``python tests/golden/make_golden.py``).

The reference repository ships no golden vectors, so these are computed
here by explicit float64 loops written independently of ``oracle/`` (no
numpy linear algebra, no shared code), on inputs that are exactly
representable in both fp16 and bf16 (multiples of 1/8 in [-2, 2]):

decode_*.npz      one RotateK decode step per the semantics of
                  fused_decode.py:131-296: visual logit
                  (k~ . q R + q . delta_mu) / sqrt(D), prompt/text logit
                  (k . q) / sqrt(D) with mask_full, running max from -1e30,
                  out = acc / (l + 1e-6); head h reads KV head h // G.
covariance.npz    kv_pruning_utils.py:112-115 on integer Keys whose mean is
                  an integer, where every storage rounding is exact.
topk.npz          head-wise top-k (score desc, index asc) with planted ties.
"""
from __future__ import annotations

import math
import os
import random

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
D = 128


def q8(rng, *shape, lim=16):
    """Random multiples of 1/8 in [-lim/8, lim/8] (exact in fp16 and bf16)."""
    n = 1
    for s in shape:
        n *= s
    return np.array([rng.randint(-lim, lim) / 8.0 for _ in range(n)]).reshape(shape)


def decode_case(name, seed, B, Hq, Hkv, Dk, S_v, S_f, with_bias, mask_p):
    rng = random.Random(seed)
    G = Hq // Hkv
    q = q8(rng, B, Hq, D, lim=4)
    R = q8(rng, B, Hkv, D, Dk, lim=2)
    dm = q8(rng, B, Hkv, D, lim=4) if with_bias else None
    kf = q8(rng, B, Hkv, S_f, D)
    vf = q8(rng, B, Hkv, S_f, D)
    mask = np.array([[1 if rng.random() >= mask_p else 0 for _ in range(S_f)] for _ in range(B)], np.uint8)
    ks = q8(rng, B, Hkv, S_v, Dk)
    vs = q8(rng, B, Hkv, S_v, D)
    scale = 1.0 / math.sqrt(D)
    out = np.zeros((B, 1, Hq, D))
    for b in range(B):
        for h in range(Hq):
            kv = h // G
            qt = [0.0] * Dk
            for c in range(Dk):
                acc = 0.0
                for d in range(D):
                    acc += q[b, h, d] * R[b, kv, d, c]
                qt[c] = acc
            bias = 0.0
            if dm is not None:
                for d in range(D):
                    bias += q[b, h, d] * dm[b, kv, d]
            logits, rows = [], []
            for s in range(S_v):
                acc = 0.0
                for c in range(Dk):
                    acc += ks[b, kv, s, c] * qt[c]
                logits.append(acc * scale + bias * scale)
                rows.append(vs[b, kv, s])
            for s in range(S_f):
                if mask[b, s]:
                    acc = 0.0
                    for d in range(D):
                        acc += kf[b, kv, s, d] * q[b, h, d]
                    logits.append(acc * scale)
                    rows.append(vf[b, kv, s])
            m = -1e30
            for x in logits:
                m = max(m, x)
            ps = [math.exp(x - m) for x in logits]
            den = 0.0
            for p in ps:
                den += p
            for d in range(D):
                acc = 0.0
                for p, row in zip(ps, rows):
                    acc += p * row[d]
                out[b, 0, h, d] = acc / (den + 1e-6)
    arrays = dict(q_full=q, R_partial=R, k_full=kf, v_full=vf, mask_full=mask, k_sparse=ks, v_sparse=vs,
                  num_kv_groups=np.array(G), out=out)
    if dm is not None:
        arrays["delta_mu"] = dm
    np.savez_compressed(os.path.join(HERE, f"decode_{name}.npz"), **arrays)


def covariance_case():
    rng = random.Random(7)
    B, H, half = 1, 2, 24
    K = np.zeros((B, H, 2 * half, D))
    cov = np.zeros((B, H, D, D))
    mean = np.zeros((B, H, D))
    for b in range(B):
        for h in range(H):
            c = [rng.randint(-3, 3) for _ in range(D)]
            X = [[rng.randint(-1, 1) for _ in range(D)] for _ in range(half)]
            for s in range(half):
                for d in range(D):
                    K[b, h, s, d] = X[s][d] + c[d]
                    K[b, h, half + s, d] = -X[s][d] + c[d]
            for d in range(D):
                mean[b, h, d] = c[d]
            for i in range(D):
                for j in range(D):
                    acc = 0.0
                    for s in range(2 * half):
                        acc += (K[b, h, s, i] - c[i]) * (K[b, h, s, j] - c[j])
                    cov[b, h, i, j] = acc
    np.savez_compressed(os.path.join(HERE, "covariance.npz"), keys=K, mean=mean, cov=cov)


def topk_case():
    rng = random.Random(3)
    B, H, k = 2, 3, 32
    scores = np.array([[[float(rng.randint(0, 9)) for _ in range(D)] for _ in range(H)] for _ in range(B)])
    idx = np.zeros((B, H, k), np.int64)
    mask = np.zeros((B, H, D), bool)
    for b in range(B):
        for h in range(H):
            order = sorted(range(D), key=lambda c: (-scores[b, h, c], c))[:k]
            kept = sorted(order)
            idx[b, h] = kept
            for c in kept:
                mask[b, h, c] = True
    np.savez_compressed(os.path.join(HERE, "topk.npz"), scores=scores, k=np.array(k), idx=idx, mask=mask)


if __name__ == "__main__":
    decode_case("mha", 1, B=1, Hq=2, Hkv=2, Dk=32, S_v=45, S_f=19, with_bias=True, mask_p=0.25)
    decode_case("gqa", 2, B=2, Hq=4, Hkv=1, Dk=16, S_v=33, S_f=8, with_bias=True, mask_p=0.0)
    decode_case("nobias", 3, B=1, Hq=2, Hkv=1, Dk=40, S_v=70, S_f=0, with_bias=False, mask_p=0.0)
    covariance_case()
    topk_case()
    print("wrote", sorted(f for f in os.listdir(HERE) if f.endswith(".npz")))
