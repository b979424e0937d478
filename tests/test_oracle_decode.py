"""Pins the decode oracle (oracle/decode.py) against independent checks.

Each check is chosen so a plausible slip in the oracle (a dropped bias, a
wrong sign, R used transposed, a wrong KV-head map, a missing mask, the wrong
denominator guard) fails at least one of them:

* brute force: explicit per-token Python loops in float64 (tiny shapes);
* textbook attention: ``scipy.special.softmax`` over concatenated logits with
  HF-style ``repeat_kv`` expansion of the KV heads;
* the rank-D_keep identity: with ``K_vis = 1 mu^T + Z R^T`` and
  ``delta_mu = mu (I - R R^T)`` RotateK equals dense attention over ``K_vis``;
* one token: the output is ``v / (1 + 1e-6)``;
* masking a prompt/text token equals deleting it;
* the split-K restatement of the paper kernels equals the closed form for
  every split count.
"""
import math

import numpy as np
import pytest
from scipy.special import softmax

from oracle import decode as od


def _inputs(rng, B=2, Hq=4, G=2, D=16, Dk=4, S_v=37, S_f=11, with_bias=True, mask_p=0.0):
    Hkv = Hq // G
    q = rng.standard_normal((B, Hq, D))
    R = np.linalg.qr(rng.standard_normal((B, Hkv, D, D)))[0][..., :Dk]
    dm = rng.standard_normal((B, Hkv, D)) * 0.3 if with_bias else None
    kf = rng.standard_normal((B, Hkv, S_f, D))
    vf = rng.standard_normal((B, Hkv, S_f, D))
    mask = (rng.random((B, S_f)) >= mask_p).astype(np.uint8)
    ks = rng.standard_normal((B, Hkv, S_v, Dk))
    vs = rng.standard_normal((B, Hkv, S_v, D))
    return q, R, dm, kf, vf, mask, ks, vs, G


def _brute(q, R, dm, kf, vf, mask, ks, vs, G):
    B, Hq, D = q.shape
    Dk = R.shape[-1]
    scale = 1.0 / math.sqrt(D)
    out = np.zeros((B, 1, Hq, D))
    for b in range(B):
        for h in range(Hq):
            kv = h // G
            qt = [sum(q[b, h, d] * R[b, kv, d, c] for d in range(D)) for c in range(Dk)]
            bias = sum(q[b, h, d] * dm[b, kv, d] for d in range(D)) if dm is not None else 0.0
            logits, vals = [], []
            for s in range(ks.shape[2]):
                logits.append(sum(ks[b, kv, s, c] * qt[c] for c in range(Dk)) * scale + bias * scale)
                vals.append(vs[b, kv, s])
            for s in range(kf.shape[2]):
                if mask[b, s]:
                    logits.append(sum(kf[b, kv, s, d] * q[b, h, d] for d in range(D)) * scale)
                    vals.append(vf[b, kv, s])
            m = max(logits + [-1e30])
            ps = [math.exp(x - m) for x in logits]
            num = np.zeros(D)
            for p, v in zip(ps, vals):
                num += p * v
            out[b, 0, h] = num / (sum(ps) + 1e-6)
    return out


def _repeat_kv(x, G):
    return np.repeat(x, G, axis=1)


def _textbook(q, K, V, G):
    """softmax(q K^T / sqrt(D)) V with repeat_kv; [B,1,Hq,D]."""
    D = q.shape[-1]
    K, V = _repeat_kv(K, G), _repeat_kv(V, G)
    logits = np.einsum("bhd,bhsd->bhs", q, K) / math.sqrt(D)
    return np.einsum("bhs,bhsd->bhd", softmax(logits, axis=-1), V)[:, None]


@pytest.mark.parametrize("G,with_bias,mask_p", [(1, True, 0.0), (2, True, 0.3), (4, False, 0.5)])
def test_oracle_matches_brute_force(G, with_bias, mask_p):
    rng = np.random.default_rng(10 + G)
    args = _inputs(rng, B=2, Hq=4, G=G, D=8, Dk=3, S_v=9, S_f=5, with_bias=with_bias, mask_p=mask_p)
    got = od.rotatek_decode(*args)
    want = _brute(*args)
    np.testing.assert_allclose(got, want, rtol=1e-12, atol=1e-12)


@pytest.mark.parametrize("G", [1, 2, 4])
def test_identity_rotation_reduces_to_textbook_attention(G):
    rng = np.random.default_rng(20 + G)
    B, Hq, D, S_v, S_f = 2, 4, 16, 23, 7
    Hkv = Hq // G
    q = rng.standard_normal((B, Hq, D))
    Kv, Vv = rng.standard_normal((B, Hkv, S_v, D)), rng.standard_normal((B, Hkv, S_v, D))
    Kf, Vf = rng.standard_normal((B, Hkv, S_f, D)), rng.standard_normal((B, Hkv, S_f, D))
    R = np.broadcast_to(np.eye(D), (B, Hkv, D, D))
    got = od.rotatek_decode(q, R, np.zeros((B, Hkv, D)), Kf, Vf, np.ones((B, S_f), np.uint8), Kv, Vv, G)
    want = _textbook(q, np.concatenate([Kv, Kf], 2), np.concatenate([Vv, Vf], 2), G)
    # acc / (l + 1e-6) vs exact softmax: relative gap <= 1e-6 since l >= 1
    np.testing.assert_allclose(got, want, rtol=2e-6, atol=1e-9)
    dense = od.full_channel_decode(q, np.concatenate([Kv, Kf], 2), np.concatenate([Vv, Vf], 2), G)
    np.testing.assert_allclose(dense, want, rtol=2e-6, atol=1e-9)


@pytest.mark.parametrize("G,Dk", [(1, 4), (2, 8), (4, 1)])
def test_rank_dkeep_identity(G, Dk):
    """K_vis = 1 mu^T + Z R^T  =>  q~.k~ + q.delta_mu = q.k exactly."""
    rng = np.random.default_rng(30 + Dk)
    B, Hq, D, S_v, S_f = 2, 4, 16, 31, 6
    Hkv = Hq // G
    R = np.linalg.qr(rng.standard_normal((B, Hkv, D, D)))[0][..., :Dk]
    mu = rng.standard_normal((B, Hkv, D)) * 2.0
    Z = rng.standard_normal((B, Hkv, S_v, Dk)) * 1.5
    Kvis = mu[:, :, None, :] + np.einsum("bhsk,bhdk->bhsd", Z, R)
    Ksp = np.einsum("bhsd,bhdk->bhsk", Kvis, R)
    dmu = mu - np.einsum("bhk,bhdk->bhd", np.einsum("bhd,bhdk->bhk", mu, R), R)
    q = rng.standard_normal((B, Hq, D))
    Vv = rng.standard_normal((B, Hkv, S_v, D))
    Kf, Vf = rng.standard_normal((B, Hkv, S_f, D)), rng.standard_normal((B, Hkv, S_f, D))
    got = od.rotatek_decode(q, R, dmu, Kf, Vf, np.ones((B, S_f), np.uint8), Ksp, Vv, G)
    want = _textbook(q, np.concatenate([Kvis, Kf], 2), np.concatenate([Vv, Vf], 2), G)
    np.testing.assert_allclose(got, want, rtol=2e-6, atol=1e-9)
    # dropping the bias must break the identity (mu has a component outside span(R))
    bad = od.rotatek_decode(q, R, None, Kf, Vf, np.ones((B, S_f), np.uint8), Ksp, Vv, G)
    assert np.max(np.abs(bad - want)) > 1e-3


def test_single_token_denominator_guard():
    D = 8
    v = np.arange(D, dtype=np.float64)[None, None, None, :] + 1.0
    q = np.ones((1, 1, D))
    R = np.ones((1, 1, D, 2))
    out = od.rotatek_decode(q, R, None, np.zeros((1, 1, 0, D)), np.zeros((1, 1, 0, D)),
                            np.zeros((1, 0), np.uint8), np.ones((1, 1, 1, 2)) * 3.0, v, 1)
    np.testing.assert_allclose(out[0, 0, 0], v[0, 0, 0] / (1.0 + 1e-6), rtol=1e-15)


def test_all_masked_and_empty_give_zero():
    rng = np.random.default_rng(4)
    q, R, dm, kf, vf, _, ks, vs, G = _inputs(rng, S_v=0, S_f=5)
    out = od.rotatek_decode(q, R, dm, kf, vf, np.zeros((2, 5), np.uint8), ks, vs, G)
    assert np.all(out == 0.0)


def test_mask_equals_removal():
    rng = np.random.default_rng(5)
    q, R, dm, kf, vf, mask, ks, vs, G = _inputs(rng, B=1, S_f=9)
    mask[0, [1, 4, 5]] = 0
    keep = mask[0] != 0
    got = od.rotatek_decode(q, R, dm, kf, vf, mask, ks, vs, G)
    want = od.rotatek_decode(q, R, dm, kf[:, :, keep], vf[:, :, keep], np.ones((1, keep.sum()), np.uint8),
                             ks, vs, G)
    np.testing.assert_allclose(got, want, rtol=1e-13, atol=1e-14)


def test_token_permutation_invariance():
    rng = np.random.default_rng(6)
    q, R, dm, kf, vf, mask, ks, vs, G = _inputs(rng, S_v=40, S_f=12)
    pv, pf = rng.permutation(40), rng.permutation(12)
    got = od.rotatek_decode(q, R, dm, kf[:, :, pf], vf[:, :, pf], mask[:, pf], ks[:, :, pv], vs[:, :, pv], G)
    want = od.rotatek_decode(q, R, dm, kf, vf, mask, ks, vs, G)
    np.testing.assert_allclose(got, want, rtol=1e-12, atol=1e-13)


@pytest.mark.parametrize("num_splits", [None, 1, 2, 3, 7, 64])
def test_paper_splitk_restatement_matches_closed_form(num_splits):
    rng = np.random.default_rng(7)
    args = _inputs(rng, B=1, Hq=4, G=2, D=16, Dk=4, S_v=150, S_f=70, mask_p=0.2)
    got = od.rotatek_decode_paper_splitk(*args, num_splits=num_splits)
    want = od.rotatek_decode(*args)
    np.testing.assert_allclose(got, want, rtol=1e-12, atol=1e-13)


def test_paper_split_policy():
    assert od.paper_num_splits(0) == (1, 0)
    assert od.paper_num_splits(1) == (1, 1)
    assert od.paper_num_splits(64) == (1, 64)
    assert od.paper_num_splits(65) == (2, 33)
    assert od.paper_num_splits(14000) == (64, 219)


def test_head_count_mismatch_raises():
    rng = np.random.default_rng(8)
    q, R, dm, kf, vf, mask, ks, vs, G = _inputs(rng, Hq=4, G=2)
    with pytest.raises(ValueError):
        od.rotatek_decode(q, R, dm, kf, vf, mask, ks, vs, 4)


@pytest.mark.parametrize("G,with_bias,mask_p,S_v,S_f", [(1, True, 0.0, 37, 11), (2, True, 0.3, 50, 20),
                                                         (4, False, 0.5, 0, 9), (2, True, 0.0, 40, 0),
                                                         (1, True, 1.0, 30, 5)])
def test_batched_torch_restatement_matches_oracle(G, with_bias, mask_p, S_v, S_f):
    """The CPU baseline's batched torch restatement equals the closed form
    (and, on the first case, the brute force) on random shapes, GQA groups,
    masks (all-masked included) and empty spans, in fp64 and within fp32
    rounding in fp32."""
    import torch
    rng = np.random.default_rng(G * 100 + S_v + S_f)
    a = _inputs(rng, G=G, with_bias=with_bias, mask_p=mask_p, S_v=S_v, S_f=S_f, Hq=8)
    want = od.rotatek_decode(*a)
    t64 = [None if x is None else torch.tensor(x) for x in a[:-1]]
    got = od.rotatek_decode_torch(*t64, a[-1])
    np.testing.assert_allclose(got.numpy(), want, rtol=1e-12, atol=1e-12)
    t32 = [None if x is None else torch.tensor(x, dtype=torch.float32 if x.dtype != np.uint8 else torch.uint8)
           for x in a[:-1]]
    got32 = od.rotatek_decode_torch(*t32, a[-1])
    assert got32.dtype == torch.float32
    np.testing.assert_allclose(got32.numpy(), want, rtol=0, atol=2e-6)
    if S_v == 37:
        np.testing.assert_allclose(got.numpy(), _brute(*a), rtol=1e-10, atol=1e-12)
