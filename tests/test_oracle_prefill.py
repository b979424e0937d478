"""Pins the prefill oracle (oracle/prefill.py) and its storage rounding
(oracle/numerics.py) against independent checks."""
import itertools

import numpy as np
import pytest

from oracle import prefill as op
from oracle.numerics import bf16_bits, from_bf16_bits, round_bf16, round_to


# ----------------------------------------------------------------- numerics
def test_fp16_rounding_is_numpy_cast():
    x = np.random.default_rng(0).standard_normal(10000) * 100
    np.testing.assert_array_equal(round_to(x, "float16"), x.astype(np.float32).astype(np.float16))


def test_bf16_rounding_bits():
    # exact, tie-to-even (down and up), carry into exponent, inf, nan
    vals = np.array([1.0, 1.0 + 2.0 ** -8, 1.0 + 3 * 2.0 ** -8, 1.0 + 2.0 ** -7 + 2.0 ** -9,
                     (2 - 2.0 ** -8), np.inf, -np.inf, 3.4e38], dtype=np.float32)
    want = np.array([0x3F80, 0x3F80, 0x3F82, 0x3F81, 0x4000, 0x7F80, 0xFF80, 0x7F80], np.uint16)
    np.testing.assert_array_equal(bf16_bits(vals), want)
    assert np.isnan(round_bf16(np.array([np.nan], np.float32)))[0]
    # every bf16 value round-trips exactly
    allbits = np.arange(0, 0x10000, dtype=np.uint32).astype(np.uint16)
    f = from_bf16_bits(allbits)
    fin = np.isfinite(f)
    np.testing.assert_array_equal(bf16_bits(f[fin]), allbits[fin])


def test_bf16_rounding_is_nearest():
    rng = np.random.default_rng(1)
    x = (rng.standard_normal(20000) * 10).astype(np.float32)
    r = round_bf16(x).astype(np.float64)
    # the neighbour bf16 values on either side are no closer
    up = from_bf16_bits(bf16_bits(x) + 1).astype(np.float64)
    dn = from_bf16_bits(bf16_bits(x) - 1).astype(np.float64)
    err = np.abs(r - x)
    assert np.all(err <= np.abs(up - x)) and np.all(err <= np.abs(dn - x))


# ----------------------------------------------------------------- spans
def test_split_spans():
    assert op.split_spans(100, 10, 20) == ((0, 10), (10, 80), (80, 100))
    assert op.split_spans(100, 0, 0) == ((0, 0), (0, 100), (0, 0))
    assert op.split_spans(100, 150, 5) == ((0, 100), (100, 100), (0, 0))
    assert op.split_spans(30, 10, 50) == ((0, 10), (10, 10), (10, 30))


def test_keep_count():
    assert op.keep_count(128, 0.75) == 32
    assert op.keep_count(128, 0.5) == 64
    assert op.keep_count(128, 0.875) == 16
    assert op.keep_count(128, 0.0) == 128
    assert op.keep_count(128, 1.5) == 0


# ----------------------------------------------------------------- covariance
@pytest.mark.parametrize("dtype", ["bfloat16", "float16"])
def test_covariance_exact_case_matches_numpy_cov(dtype):
    """Integer Keys whose mean is an integer: every storage rounding is exact,
    so the oracle must equal numpy's textbook covariance times S."""
    rng = np.random.default_rng(2)
    B, H, half, D = 2, 3, 8, 16
    X = rng.integers(-1, 2, size=(B, H, half, D)).astype(np.float64)
    c = rng.integers(-5, 6, size=(B, H, 1, D)).astype(np.float64)
    K = np.concatenate([X, -X], axis=2) + c
    mean, cov = op.key_covariance(K, dtype)
    np.testing.assert_array_equal(mean, c[:, :, 0])
    for b in range(B):
        for h in range(H):
            want = np.cov(K[b, h], rowvar=False, bias=True) * K.shape[2]
            np.testing.assert_array_equal(cov[b, h], want)


def test_covariance_rounding_tolerance():
    rng = np.random.default_rng(3)
    K = rng.standard_normal((1, 2, 300, 16)) * 2 + 0.7
    mean, cov = op.key_covariance(K, "bfloat16")
    for h in range(2):
        want = np.cov(K[0, h], rowvar=False, bias=True) * 300
        np.testing.assert_allclose(cov[0, h], want, rtol=0, atol=2.0 ** -6 * np.abs(want).max())
    np.testing.assert_allclose(mean, K.mean(axis=2), rtol=1e-6)


# ----------------------------------------------------------------- query weight
def test_query_weight_hand_case():
    """D=4 (even count): norms [4, 1e-9, 2, 3]; lower median 2 -> floor 2e-3."""
    D = 4
    q = np.zeros((1, 1, 2, D))
    q[0, 0, 0] = [4.0, 1e-9, 0.0, 3.0]
    q[0, 0, 1] = [0.0, 0.0, 2.0, 0.0]
    cov = np.eye(D)[None, None]
    got = op.query_weight(cov, q, num_kv_groups=1)
    qn = np.array([4.0, 2e-3, 2.0, 3.0])
    diag = qn ** 2
    ridge = 1e-4 * max(diag.mean(), 1e-6)
    np.testing.assert_allclose(got[0, 0], np.diag(diag + ridge), rtol=1e-12, atol=1e-15)


@pytest.mark.parametrize("scale,ridge", [(1e-3, 1e-7), (1e-8, 1e-10), (2.0, 2e-4)])
def test_query_weight_ridge_clamps_the_mean(scale, ridge):
    """ridge = 1e-4 * mean|diag|.clamp(min=1e-6) (kv_pruning_utils.py:137-139:
    the clamp binds to the mean, before the product).  With unit query norms
    the weighted diagonal is ``scale``; the numbers are written out, so a
    clamp moved outside the product (max(1e-4 m, 1e-6)) fails the first two."""
    D = 4
    q = np.zeros((1, 1, 1, D))
    q[0, 0, 0] = 1.0
    got = op.query_weight(scale * np.eye(D)[None, None], q, num_kv_groups=1)
    np.testing.assert_allclose(np.diag(got[0, 0]), np.full(D, scale + ridge), rtol=1e-12)


def test_query_weight_nan_norm_poisons_the_head():
    """torch.median of a row with a NaN is NaN (torch.nanmedian is the one
    that skips NaNs), so q_floor is NaN and the clamp against it makes every
    weight of that head NaN; other heads are untouched.  A median that
    skipped the NaN (numpy's sort puts it last) would leave the other
    channels finite."""
    D = 6
    q = np.ones((1, 2, 3, D))
    q[0, 0, 1, 2] = np.nan
    cov = np.broadcast_to(np.eye(D), (1, 2, D, D)).copy()
    got = op.query_weight(cov, q, num_kv_groups=1)
    assert np.all(np.isnan(got[0, 0]))
    assert np.all(np.isfinite(got[0, 1]))
    np.testing.assert_allclose(np.diag(got[0, 1]), 3.0 + 1e-4 * 3.0, rtol=1e-12)


def test_query_weight_window_and_group_mean():
    rng = np.random.default_rng(4)
    B, Hkv, G, S, D = 1, 2, 3, 40, 6
    q = rng.standard_normal((B, Hkv * G, S, D))
    cov = np.broadcast_to(np.eye(D), (B, Hkv, D, D)).copy()
    got = op.query_weight(cov, q, num_kv_groups=G)
    for h in range(Hkv):
        grp = q[0, h * G:(h + 1) * G, -32:, :].mean(axis=0)          # [32, D]
        qn = np.sqrt((grp ** 2).sum(axis=0))
        qn = np.maximum(qn, 1e-3 * np.sort(qn)[(D - 1) // 2])
        diag = qn ** 2
        np.testing.assert_allclose(np.diag(got[0, h]), diag + 1e-4 * max(diag.mean(), 1e-6), rtol=1e-12)
        off = got[0, h] - np.diag(np.diag(got[0, h]))
        assert np.all(off == 0.0)


# ----------------------------------------------------------------- eigenbasis
def test_eigh_rotation_known_spectrum():
    rng = np.random.default_rng(5)
    D, keep = 12, 4
    Q = np.linalg.qr(rng.standard_normal((D, D)))[0]
    lam = np.array([50, 40, 30, 20] + [1.0 - 0.05 * i for i in range(D - 4)])
    C = (Q * lam) @ Q.T
    R, ev = op.eigh_rotation(C[None, None], keep)
    R = R[0, 0]
    np.testing.assert_allclose(R.T @ R, np.eye(keep), atol=1e-12)
    np.testing.assert_allclose(C @ R, R * ev[0, 0, :keep], atol=1e-10)
    np.testing.assert_allclose(ev[0, 0, :4], [50, 40, 30, 20], rtol=1e-12)
    np.testing.assert_allclose(R @ R.T, Q[:, :4] @ Q[:, :4].T, atol=1e-10)


def test_power_iteration_subspace():
    rng = np.random.default_rng(6)
    D, k = 32, 6
    Q = np.linalg.qr(rng.standard_normal((D, D)))[0]
    lam = np.concatenate([np.linspace(100, 60, k), np.linspace(3, 0.1, D - k)])
    C = (Q * lam) @ Q.T
    V0 = rng.standard_normal((D, k))
    V = op.power_iteration(C, V0, num_iters=5, eps=1e-6)
    np.testing.assert_allclose(V.T @ V, np.eye(k), atol=1e-5)
    P = Q[:, :k] @ Q[:, :k].T
    assert np.linalg.norm(V @ V.T - P) < 1e-4
    # one iteration from a random start is far from converged: the check bites
    V1 = op.power_iteration(C, V0, num_iters=1, eps=1e-6)
    assert np.linalg.norm(V1 @ V1.T - P) > 1e-3


# ----------------------------------------------------------------- rotate / delta-mu
def test_rotate_keys_brute_force():
    rng = np.random.default_rng(7)
    K = rng.standard_normal((1, 1, 5, 6))
    R = rng.standard_normal((1, 1, 6, 3))
    got = op.rotate_keys(K, R, "float64")
    for s in range(5):
        for c in range(3):
            assert abs(got[0, 0, s, c] - sum(K[0, 0, s, d] * R[0, 0, d, c] for d in range(6))) < 1e-12


def test_delta_mu_projector_identity():
    rng = np.random.default_rng(8)
    D, k = 16, 5
    R = np.linalg.qr(rng.standard_normal((1, 2, D, D)))[0][..., :k]
    mu = rng.standard_normal((1, 2, D))
    dm = op.delta_mu(mu, R, "float64")
    np.testing.assert_allclose(np.einsum("bhd,bhdk->bhk", dm, R), 0.0, atol=1e-12)
    np.testing.assert_allclose(dm + np.einsum("bhk,bhdk->bhd", np.einsum("bhd,bhdk->bhk", mu, R), R), mu,
                               atol=1e-12)


# ----------------------------------------------------------------- selection
def test_channel_scores_brute_force():
    rng = np.random.default_rng(9)
    K = rng.standard_normal((1, 1, 7, 4))
    R = rng.standard_normal((1, 1, 4, 4))
    got = op.channel_scores(K, R)
    for c in range(4):
        want = sum(abs(sum(K[0, 0, s, d] * R[0, 0, d, c] for d in range(4))) for s in range(7)) / 7
        assert abs(got[0, 0, c] - want) < 1e-12


def test_topk_exhaustive_with_ties():
    D, k = 6, 3
    for vals in itertools.product([0.0, 1.0, 2.0], repeat=D):
        s = np.array(vals)[None, None]
        idx, mask = op.topk_channels(s, k)
        want = sorted(sorted(range(D), key=lambda i: (-vals[i], i))[:k])
        assert idx[0, 0].tolist() == want
        assert mask[0, 0].tolist() == [i in want for i in range(D)]


# ----------------------------------------------------------------- end to end
def test_update_rotatek_eig_rule_shapes_and_mask():
    rng = np.random.default_rng(10)
    B, Hkv, G, S, D = 1, 2, 2, 90, 16
    K = rng.standard_normal((B, Hkv, S, D))
    Q = rng.standard_normal((B, Hkv * G, S, D))
    r = op.update_rotatek(K, Q, prompt_seqlen=5, query_seqlen=10, ratio=0.75, num_kv_groups=G,
                          dtype="bfloat16")
    assert r["k_sparse"].shape == (B, Hkv, 75, 4)
    assert r["k_prompt"].shape == (B, Hkv, 5, D) and r["k_text"].shape == (B, Hkv, 10, D)
    assert r["keep_mask"][..., :4].all() and not r["keep_mask"][..., 4:].any()
    # stored values are bf16-representable
    np.testing.assert_array_equal(r["k_sparse"], round_to(r["k_sparse"], "bfloat16"))
    np.testing.assert_array_equal(r["R_partial"], round_to(r["R_partial"], "bfloat16"))


def test_update_rotatek_score_rule_picks_outlier_channels():
    """With R_full = I the rotated channels are the raw channels: the planted
    x8 outliers must be among the kept ones."""
    rng = np.random.default_rng(11)
    B, H, S, D = 1, 2, 200, 16
    K = rng.standard_normal((B, H, S, D))
    K[..., [2, 9]] *= 8.0
    Q = rng.standard_normal((B, H, S, D))
    r = op.update_rotatek(K, Q, 0, 0, ratio=0.75, num_kv_groups=1, dtype="float32",
                          select="score", R_full=np.broadcast_to(np.eye(D), (B, H, D, D)))
    for h in range(H):
        assert {2, 9} <= set(r["keep_idx"][0, h].tolist())
    np.testing.assert_allclose(r["R_partial"][0, 0], np.eye(D)[:, r["keep_idx"][0, 0]])


def test_query_weight_group_mean_uses_fp32_factor():
    """The bf16 group mean is fp32(sum) * fp32(1/G), rounded (torch's MeanOps),
    not the exact quotient: find a group of 7 bf16 values where the two
    roundings differ and check the oracle takes the torch one."""
    from oracle.numerics import round_bf16
    rng = np.random.default_rng(11)
    G, D = 7, 128
    for _ in range(200):
        vals = round_bf16(rng.standard_normal((G, D)) * 3).astype(np.float64)
        s32 = vals.astype(np.float32).sum(axis=0, dtype=np.float32)
        torch_like = round_bf16((s32 * np.float32(1.0 / G)).astype(np.float64))
        exact = round_bf16(vals.sum(axis=0) / G)
        if np.any(torch_like != exact):
            break
    else:
        pytest.fail("no distinguishing group found")
    q = np.zeros((1, G, 1, D))
    q[0, :, 0, :] = vals
    cov = np.eye(D)[None, None]
    got = op.query_weight(cov, q, num_kv_groups=G, dtype="bfloat16")
    qn = np.abs(torch_like).astype(np.float64)
    qn = np.maximum(qn, 1e-3 * np.sort(qn)[(D - 1) // 2])
    d = np.diag(got[0, 0])
    np.testing.assert_allclose(d - 1e-4 * max((qn ** 2).mean(), 1e-6), qn ** 2, rtol=1e-12)
