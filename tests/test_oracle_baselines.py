"""Pins oracle/baselines.py (ThinK / SparK) with checks that do not restate it:
closed forms on inputs whose scores are known exactly, brute-force
enumeration of the selection on 4-channel toy heads with planted ties, the
selection invariants on random data, and the recovery identities.  A plausible
slip (pruning the largest scores, breaking ties the other way, dropping the
group mean, using the sum instead of the mean, filling with the kept mean)
fails at least one of them.
"""
import itertools

import numpy as np
import pytest

from oracle import baselines as ob
from oracle.numerics import round_to

DTYPES = ["bfloat16", "float16"]


def _grid(rng, shape, dtype):
    """Values m/8, |m| <= 15: exact in fp16 / bf16, squares exact, sums of up
    to 2^15 squares exact in fp32."""
    return round_to(rng.integers(-15, 16, size=shape) / 8.0, dtype)


def test_mean_factor_matches_reciprocal_and_empty_is_inf():
    for n_out, S in [(4096, 12000), (128, 1), (7, 33)]:
        assert ob.mean_factor(n_out, n_out * S) == np.float32(1.0) / np.float32(S)
    assert np.isinf(ob.mean_factor(5, 0))
    # above 2^24 the element count itself rounds, so the factor is not 1/S
    n_out, S = 3 * 7 * 128, 16001
    f = ob.mean_factor(n_out, n_out * S)
    assert f == np.float32(np.float32(n_out) / np.float32(n_out * S))


# ------------------------------------------------------------------ ThinK
@pytest.mark.parametrize("dtype", DTYPES)
def test_think_closed_form_scores_and_prunes_smallest(dtype):
    """Channel c constant a_c over tokens, queries constant b_c: keys_norm =
    a_c^2, queries_norm = b_c^2 (power-of-two lengths), score = a_c^2 b_c^2."""
    rng = np.random.default_rng(1)
    B, H, G, S, W, D = 1, 2, 2, 64, 8, 128
    a = round_to(rng.integers(1, 16, size=(B, H, 1, D)) / 4.0, dtype)
    b = round_to(rng.integers(1, 16, size=(B, H * G, 1, D)) / 4.0, dtype)
    K = np.broadcast_to(a, (B, H, S, D))
    Q = np.broadcast_to(b, (B, H * G, W, D))
    prune = 80
    Kc, mask, scores = ob.think_score_and_compact(K, Q, H, prune, dtype)
    qn = round_to(round_to(b[:, :, 0] ** 2, dtype).reshape(B, H, G, D).mean(axis=2), dtype)
    expect = round_to(qn * round_to(a[:, :, 0] ** 2, dtype), dtype)
    np.testing.assert_array_equal(scores, expect)
    for h in range(H):
        s = expect[0, h]
        pruned = sorted(range(D), key=lambda c: (s[c], c))[:prune]
        want = np.ones(D, bool)
        want[pruned] = False
        np.testing.assert_array_equal(mask[0, h], want)
        assert s[~want].max() <= s[want].min()
        np.testing.assert_array_equal(Kc[0, h], K[0, h][:, want])


def test_think_equal_scores_prune_the_lowest_channels():
    B, H, S, D = 1, 1, 16, 128
    K = np.full((B, H, S, D), 0.5)
    Q = np.full((B, 2, 4, D), 0.25)
    for prune in (0, 1, 50, 127, 128):
        _, mask, _ = ob.think_score_and_compact(K, Q, 1, prune, "bfloat16")
        np.testing.assert_array_equal(mask[0, 0], np.arange(D) >= prune)


def test_think_exhaustive_toy_heads_against_brute_force():
    """4 channels, scores from {0, 1, 2} (every tie pattern), every prune
    count: the pruned set is the lexicographically first set P of size p with
    max(score[P]) <= min(score[rest])."""
    D = 4
    for pattern in itertools.product([1.0, 2.0, 4.0], repeat=D):
        a = np.sqrt(np.array(pattern))          # keys_norm = pattern exactly (S = 1)
        K = a.reshape(1, 1, 1, D)
        Q = np.ones((1, 1, 1, D))
        for p in range(D + 1):
            _, mask, scores = ob.think_score_and_compact(K, Q, 1, p, "float16")
            s = scores[0, 0]
            valid = [P for P in itertools.combinations(range(D), p)
                     if not P or len(P) == D or max(s[list(P)]) <= min(np.delete(s, list(P)))]
            want = np.ones(D, bool)
            want[list(min(valid))] = False
            np.testing.assert_array_equal(mask[0, 0], want, err_msg=f"{pattern} p={p}")


@pytest.mark.parametrize("dtype", DTYPES)
def test_think_random_selection_invariants(dtype):
    rng = np.random.default_rng(2)
    B, H, G, S, W, D = 2, 3, 4, 200, 32, 128
    K = round_to(rng.standard_normal((B, H, S, D)) * np.where(np.arange(D) % 9 == 0, 6.0, 1.0), dtype)
    Q = round_to(rng.standard_normal((B, H * G, W, D)), dtype)
    prune = 96
    Kc, mask, scores = ob.think_score_and_compact(K, Q, H, prune, dtype)
    assert Kc.shape == (B, H, S, D - prune)
    for b in range(B):
        for h in range(H):
            m, s = mask[b, h], scores[b, h]
            assert m.sum() == D - prune
            assert s[~m].max() <= s[m].min()
            v = s[~m].max()
            tied_pruned = np.flatnonzero(~m & (s == v))
            tied_kept = np.flatnonzero(m & (s == v))
            if len(tied_kept) and len(tied_pruned):
                assert tied_pruned.max() < tied_kept.min()
            np.testing.assert_array_equal(Kc[b, h], K[b, h][:, m])


def test_think_group_mean_and_window_mean_are_means_not_sums():
    """Two query heads per KV head with constant 1 and 3 on channel 0: the
    group mean of the window means of q^2 is (1 + 9) / 2 = 5, so channel 0
    (score 5 * 1) outranks channel 1 (keys 2, queries 1: score 4)."""
    D = 128
    K = np.zeros((1, 1, 8, D))
    K[..., 0] = 1.0
    K[..., 1] = 2.0
    Q = np.zeros((1, 2, 4, D))
    Q[0, 0, :, 0], Q[0, 1, :, 0] = 1.0, 3.0
    Q[0, :, :, 1] = 1.0
    _, mask, scores = ob.think_score_and_compact(K, Q, 1, D - 1, "bfloat16")
    assert scores[0, 0, 0] == 5.0 and scores[0, 0, 1] == 4.0
    assert mask[0, 0].tolist() == [True] + [False] * (D - 1)


# ------------------------------------------------------------------ SparK
def test_group_queries_means():
    rng = np.random.default_rng(3)
    Q = _grid(rng, (2, 6, 5, 128), "bfloat16")
    np.testing.assert_array_equal(ob.group_queries(Q, 1, "bfloat16"), Q)
    g = ob.group_queries(Q, 2, "float16")
    np.testing.assert_array_equal(g, (Q[:, 0::2] + Q[:, 1::2]) / 2)   # exact on the grid


@pytest.mark.parametrize("dtype", DTYPES)
def test_spark_closed_form(dtype):
    """q constant b_c over W = 4 tokens: q_norm = 2|b_c|; token t has
    k = c-dependent grid values; expected kept sets by plain sorting."""
    rng = np.random.default_rng(4)
    B, H, S, W, D = 1, 2, 6, 4, 128
    b = round_to(rng.integers(1, 8, size=(B, H, 1, D)) / 4.0, dtype)
    Q = np.broadcast_to(b, (B, H, W, D))
    K = _grid(rng, (B, H, S, D), dtype)
    prune = 100
    Kc, mask, pm, scores = ob.per_token_channel_prune(Q, K, prune, dtype)
    qn = round_to(2 * b[:, :, 0], dtype)
    expect = round_to(round_to(K ** 2, dtype) * qn[:, :, None, :], dtype)
    np.testing.assert_array_equal(scores, expect)
    for h in range(H):
        for t in range(S):
            s = expect[0, h, t]
            kept = sorted(sorted(range(D), key=lambda c: (-s[c], c))[:D - prune])
            want = np.zeros(D, bool)
            want[kept] = True
            np.testing.assert_array_equal(mask[0, h, t], want)
            np.testing.assert_array_equal(Kc[0, h, t], K[0, h, t, kept])
            assert pm[0, h, t, 0] == round_to(K[0, h, t, ~want].mean(), dtype)


def test_spark_exhaustive_toy_tokens_against_brute_force():
    """4 channels, k^2 from {1, 2, 4} (every tie pattern), every keep count:
    the kept set is the lexicographically first set K of that size with
    min(score[K]) >= max(score[rest]); pruned mean = mean of the rest."""
    D = 4
    for pattern in itertools.product([1.0, 2.0, 4.0], repeat=D):
        k = np.sqrt(np.array(pattern)).reshape(1, 1, 1, D)
        q = np.ones((1, 1, 1, D))
        for p in range(D + 1):
            _, mask, pm, scores = ob.per_token_channel_prune(q, k, p, "float16")
            s = scores[0, 0, 0]
            keep = D - p
            valid = [Ks for Ks in itertools.combinations(range(D), keep)
                     if not Ks or len(Ks) == D or min(s[list(Ks)]) >= max(np.delete(s, list(Ks)))]
            want = np.zeros(D, bool)
            want[list(min(valid))] = True
            np.testing.assert_array_equal(mask[0, 0, 0], want, err_msg=f"{pattern} p={p}")
            if p:
                assert pm[0, 0, 0, 0] == round_to(k[0, 0, 0, ~want].mean(), "float16")
            else:
                assert np.isnan(pm[0, 0, 0, 0])


def test_spark_nan_scores_are_kept_first_and_inf_keys():
    D = 128
    K = np.ones((1, 1, 1, D))
    K[..., 5] = np.inf              # k^2 = inf, q = 0 there -> NaN score
    Q = np.ones((1, 1, 2, D))
    Q[..., 5] = 0.0
    _, mask, _, scores = ob.per_token_channel_prune(Q, K, D - 1, "float16")
    assert np.isnan(scores[0, 0, 0, 5])
    assert np.flatnonzero(mask[0, 0, 0]).tolist() == [5]


# --------------------------------------------------------------- recovery
@pytest.mark.parametrize("dtype", DTYPES)
def test_recover_think_inverts_compaction(dtype):
    rng = np.random.default_rng(5)
    B, H, S, W, D = 2, 2, 30, 8, 128
    K = _grid(rng, (B, H, S, D), dtype)
    Q = _grid(rng, (B, 2 * H, W, D), dtype)
    Kc, mask, _ = ob.think_score_and_compact(K, Q, H, 77, dtype)
    R = ob.recover_think(Kc, mask)
    m = np.broadcast_to(mask[:, :, None, :], R.shape)
    np.testing.assert_array_equal(R[m], K[m])
    assert np.all(R[~m] == 0)


@pytest.mark.parametrize("dtype", DTYPES)
def test_recover_spark_inverts_compaction(dtype):
    rng = np.random.default_rng(6)
    B, H, S, W, D = 2, 2, 30, 8, 128
    K = _grid(rng, (B, H, S, D), dtype)
    Q = _grid(rng, (B, H, W, D), dtype)
    Kc, mask, pm, _ = ob.per_token_channel_prune(Q, K, 90, dtype)
    R = ob.recover_spark(Kc, mask, pm)
    np.testing.assert_array_equal(R[mask], K[mask])
    np.testing.assert_array_equal(R[~mask], np.broadcast_to(pm, R.shape)[~mask])
    for b, h, t in [(0, 0, 0), (1, 1, 29)]:
        assert pm[b, h, t, 0] == round_to(K[b, h, t, ~mask[b, h, t]].mean(), dtype)
