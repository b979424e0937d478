"""GPU parity of the prefill kernels at head sizes other than 128 and on
fp32 Keys.

The reference's update_rotatek is plain torch (kv_pruning_utils.py:110-159):
it takes any head size and any float dtype, and rotation.py:86-91 takes D
from the covariance.  Bars as in test_gpu_prefill.py: exact where the
arithmetic is exact, one storage ulp for stored 16-bit values, and for fp32
1e-5 of the largest entry (fp32 sums in another order than the oracle's
fp64).  Kept-channel indices are bit-exact on heads whose top-k boundary gap
exceeds the score rounding.
"""
import sys

import numpy as np
import pytest
import torch

from oracle import prefill as op
from oracle.numerics import round_to

pytestmark = pytest.mark.gpu

DT = {torch.float16: "float16", torch.bfloat16: "bfloat16", torch.float32: "float32"}
ULP = {torch.float16: 2.0 ** -10, torch.bfloat16: 2.0 ** -7}


def _np(t):
    return t.detach().cpu().to(torch.float64).numpy()


def _say(msg):
    print(f"[case] {msg}", flush=True)
    sys.stdout.flush()


def _storage_ulp(a, b, dtype):
    m = np.maximum(np.abs(a), np.abs(b))
    e = np.floor(np.log2(np.maximum(m, 1e-30)))
    return 2.0 ** e * ULP[dtype]


def _keys(B, H, S, D, dtype, seed, offset=0.5, outliers=True):
    g = torch.Generator(device="cuda").manual_seed(seed)
    K = torch.randn(B, H, S, D, generator=g, device="cuda")
    if outliers:
        K[..., ::37] *= 8.0
    return (K + offset).to(dtype)


def _lowrank(B, H, S, D, dtype, seed, rank=12):
    g = torch.Generator(device="cuda").manual_seed(seed)
    U = torch.linalg.qr(torch.randn(B, H, D, rank, generator=g, device="cuda"))[0]
    Z = torch.randn(B, H, S, rank, generator=g, device="cuda")
    E = torch.randn(B, H, S, D, generator=g, device="cuda")
    mu = torch.randn(B, H, 1, D, generator=g, device="cuda") * 2
    return (4.0 * Z @ U.transpose(-1, -2) + 0.5 * E + mu).to(dtype)


# ----------------------------------------------------------------- covariance
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("D", [64, 80, 96, 40, 100])
def test_covariance_head_dim(dtype, D):
    """D % 8 == 0: 16-byte rows with the channel slots past D masked; D = 100:
    element-wise loads.  Mean to 1e-5, covariance to one storage ulp about
    the kernel's own centre, exactly symmetric, shape [B, H, D, D]."""
    from rotatek_amd import prefill
    _say(f"covariance head_dim {D} {dtype}")
    B, H, S = 2, 4, 1000
    full = _keys(B, H, S + 70, D, dtype, seed=D, outliers=dtype == torch.bfloat16)
    Kv = full[:, :, 30:30 + S]
    mean, cov = prefill.key_covariance(Kv)
    torch.cuda.synchronize()
    assert mean.shape == (B, H, D) and cov.shape == (B, H, D, D)
    om, _ = op.key_covariance(_np(Kv), DT[dtype])
    np.testing.assert_allclose(_np(mean), om, rtol=1e-5, atol=1e-6)
    _, oc = op.key_covariance(_np(Kv), DT[dtype], mean=_np(mean))
    scale = np.abs(oc).max(axis=(-1, -2), keepdims=True)
    err = np.abs(_np(cov) - oc)
    assert np.all(err <= _storage_ulp(oc, _np(cov), dtype) + 1e-6 * scale), err.max()
    c = _np(cov)
    np.testing.assert_array_equal(c, np.swapaxes(c, -1, -2))


@pytest.mark.parametrize("D", [64, 72, 33])
def test_covariance_exact_integer_head_dim(D):
    """Integer Keys with an integer mean at D < 128: every rounding exact, so
    the covariance equals the oracle bit for bit (a channel past D that
    leaked into the sums or the centre would break it)."""
    from rotatek_amd import prefill
    _say(f"covariance exact head_dim {D}")
    rng = np.random.default_rng(D)
    B, H, half = 2, 3, 96
    X = rng.integers(-1, 2, size=(B, H, half, D)).astype(np.float32)
    c = rng.integers(-4, 5, size=(B, H, 1, D)).astype(np.float32)
    K = np.concatenate([X, -X], axis=2) + c
    # a view of a 128-wide tensor whose extra channels hold large values
    wide = np.full((B, H, 2 * half, 128), 3.0e4, np.float32)
    wide[..., :D] = K
    Kt = torch.tensor(wide, device="cuda").to(torch.bfloat16)[..., :D]
    mean, cov = prefill.key_covariance(Kt)
    torch.cuda.synchronize()
    om, oc = op.key_covariance(K, "bfloat16")
    np.testing.assert_array_equal(_np(mean), om)
    np.testing.assert_array_equal(_np(cov), oc)


@pytest.mark.parametrize("D,G", [(64, 7), (80, 4), (96, 1), (40, 2)])
def test_weighted_covariance_head_dim(D, G):
    """Fused weighting (rk_key_covariance_weighted) bit-identical to the two
    stages, and both against the oracle's weighting (lower median of the D
    norms, ridge over D diagonal entries)."""
    from rotatek_amd import prefill
    _say(f"weighted covariance head_dim {D} G={G}")
    B, H, S = 2, 3, 900
    K = _lowrank(B, H, S, D, torch.bfloat16, seed=D + G)
    Q = (torch.randn(B, H * G, 50, D, device="cuda") * 1.5).to(torch.bfloat16)
    m0, c0 = prefill.key_covariance(K)
    two = prefill.query_weight(c0, Q, G)
    m1, one = prefill.key_covariance(K, Q, G)
    torch.cuda.synchronize()
    assert torch.equal(m0, m1) and torch.equal(one, two)
    ref = op.query_weight(_np(c0), _np(Q), G, dtype="bfloat16")
    assert np.abs(_np(one) - ref).max() <= 1e-5 * np.abs(ref).max()


# ----------------------------------------------------------- rotate / select
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("D,Dk", [(64, 16), (80, 40), (96, 96), (100, 20)])
def test_rotate_and_scores_head_dim(dtype, D, Dk):
    from rotatek_amd import prefill
    _say(f"rotate / scores head_dim {D} Dk={Dk} {dtype}")
    B, H, S = 2, 3, 777
    K = _keys(B, H, S, D, dtype, seed=D + Dk)
    Rf = torch.linalg.qr(torch.randn(B, H, D, D, device="cuda", dtype=torch.float64))[0].float()
    R = Rf[..., :Dk].contiguous().to(dtype)
    out = prefill.rotate_keys(K, R)
    sc = prefill.channel_scores(K, Rf)
    torch.cuda.synchronize()
    want = op.rotate_keys(_np(K), _np(R), DT[dtype])
    err = np.abs(_np(out) - want)
    assert np.all(err <= ULP[dtype] * np.abs(want) + 1e-3 * ULP[dtype]), err.max()
    wsc = op.channel_scores(_np(K), round_to(_np(Rf), DT[dtype]))
    np.testing.assert_allclose(_np(sc), wsc, rtol=1e-5, atol=1e-7)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("D", [64, 80])
def test_gather_rotation_head_dim(dtype, D):
    from rotatek_amd import prefill
    _say(f"gather head_dim {D} {dtype}")
    B, H, k = 2, 3, 24
    R = torch.linalg.qr(torch.randn(B, H, D, D, device="cuda"))[0].contiguous()
    idx = torch.stack([torch.randperm(D, device="cuda")[:k].sort().values for _ in range(B * H)]).view(B, H, k)
    mean = torch.randn(B, H, D, device="cuda") * 3
    Rp, dm = prefill.gather_rotation(R, idx, mean, dtype)
    torch.cuda.synchronize()
    wantR = round_to(np.take_along_axis(_np(R), idx.cpu().numpy()[:, :, None, :], axis=-1), DT[dtype])
    np.testing.assert_array_equal(_np(Rp), wantR)
    wantd = op.delta_mu(_np(mean), wantR, DT[dtype])
    tol = ULP[dtype] * np.abs(wantd) + 1e-5 if dtype != torch.float32 else 1e-5 * np.abs(wantd).max()
    assert np.all(np.abs(_np(dm) - wantd) <= tol)


# ------------------------------------------------------------ power iteration
@pytest.mark.parametrize("D,k", [(64, 16), (80, 32), (96, 64), (100, 72), (48, 48)])
def test_power_iteration_head_dim(D, k):
    """The HIP subspace iteration on a D x D covariance equals the oracle's
    from the same start block (power_iteration_hip; zero-padded rows stay
    exact zeros), and power_iteration_gpu spans eigh's dominant subspace."""
    from rotatek_amd.rotation import power_iteration_gpu, power_iteration_hip
    _say(f"power iteration head_dim {D} k={k}")
    B, H = 1, 4
    g = torch.Generator(device="cuda").manual_seed(D + k)
    Q = torch.linalg.qr(torch.randn(B, H, D, D, generator=g, device="cuda", dtype=torch.float64))[0]
    lam = torch.cat([torch.linspace(100, 50, k, dtype=torch.float64), torch.linspace(1, 0.1, D - k, dtype=torch.float64)])
    C = (Q * lam.cuda()) @ Q.transpose(-1, -2)
    C = (0.5 * (C + C.transpose(-1, -2))).float().contiguous()
    V0 = torch.randn(B, H, D, k, generator=g, device="cuda")
    got = power_iteration_hip(C, V0, 5, 1e-4)
    torch.cuda.synchronize()
    want = op.power_iteration(_np(C), _np(V0), 5, 1e-4)
    tol = 2e-3 if k <= 64 else 1e-2
    assert np.abs(_np(got) - want).max() <= tol * np.abs(want).max()
    R = power_iteration_gpu(C, k)
    torch.cuda.synchronize()
    assert R.shape == (B, H, D, k)
    P = _np(R) @ np.swapaxes(_np(R), -1, -2)
    Qk = _np(Q)[..., :k]
    assert np.abs(P - Qk @ np.swapaxes(Qk, -1, -2)).max() <= 1e-3


# ------------------------------------------------------------------- fp32 Keys
@pytest.mark.parametrize("S", [1, 31, 2304])
@pytest.mark.parametrize("D", [128, 64])
def test_covariance_fp32(S, D):
    """fp32 Keys: Kc = K - mean in fp32 and the covariance summed in fp32 on
    the fp32 MFMA (no rounding to a 16-bit type, as the reference's fp32
    einsum)."""
    from rotatek_amd import prefill
    _say(f"covariance fp32 S={S} D={D}")
    B, H = 2, 4
    K = _keys(B, H, S + 40, D, torch.float32, seed=S + D)[:, :, 20:20 + S]
    mean, cov = prefill.key_covariance(K)
    torch.cuda.synchronize()
    om, _ = op.key_covariance(_np(K), "float32")
    np.testing.assert_allclose(_np(mean), om, rtol=1e-5, atol=1e-6)
    _, oc = op.key_covariance(_np(K), "float32", mean=_np(mean))
    scale = np.abs(oc).max(axis=(-1, -2), keepdims=True)
    assert np.all(np.abs(_np(cov) - oc) <= 1e-5 * scale)
    c = _np(cov)
    np.testing.assert_array_equal(c, np.swapaxes(c, -1, -2))


@pytest.mark.parametrize("G", [1, 7])
def test_weighted_covariance_fp32(G):
    from rotatek_amd import prefill
    _say(f"weighted covariance fp32 G={G}")
    B, H, S = 2, 4, 1200
    K = _lowrank(B, H, S, 128, torch.float32, seed=G)
    Q = torch.randn(B, H * G, 60, 128, device="cuda") * 1.5
    m0, c0 = prefill.key_covariance(K)
    two = prefill.query_weight(c0, Q, G)
    m1, one = prefill.key_covariance(K, Q, G)
    torch.cuda.synchronize()
    assert torch.equal(m0, m1) and torch.equal(one, two)
    ref = op.query_weight(_np(c0), _np(Q), G, dtype="float32")
    assert np.abs(_np(one) - ref).max() <= 1e-5 * np.abs(ref).max()


@pytest.mark.parametrize("Dk", [16, 32, 128])
def test_rotate_keys_and_scores_fp32(Dk):
    from rotatek_amd import prefill
    _say(f"rotate / scores fp32 Dk={Dk}")
    B, H, S = 2, 3, 777
    K = _keys(B, H, S, 128, torch.float32, seed=Dk)
    Rf = torch.linalg.qr(torch.randn(B, H, 128, 128, device="cuda", dtype=torch.float64))[0].float()
    R = Rf[..., :Dk].contiguous()
    out = prefill.rotate_keys(K, R)
    sc = prefill.channel_scores(K, Rf)
    torch.cuda.synchronize()
    assert out.dtype == torch.float32
    want = op.rotate_keys(_np(K), _np(R), "float32")
    assert np.abs(_np(out) - want).max() <= 1e-5 * np.abs(want).max()
    np.testing.assert_allclose(_np(sc), op.channel_scores(_np(K), _np(Rf)), rtol=2e-6, atol=1e-7)


def test_config0_selection_fp32_bit_exact():
    """BASELINE config 0 at its precision: fp32 Keys (N(0,1), four x8 outlier
    channels per head), R_k = QR of a seeded Gaussian per head, keep the
    top-32 channels by mean |K R_k|.  The HIP scores (fp32 MFMA, fp64 final
    sum) select exactly the oracle's channels (fp64) on a fixture whose every
    head has a top-32 boundary gap above the fp32 score rounding (asserted);
    the keep mask, R_partial (an exact gather) and delta_mu follow."""
    from rotatek_amd import prefill, synth
    _say("config-0 selection fp32 bit-exact")
    B, H, S, keep = 1, 32, 2304, 32
    for seed in range(0, 40):
        g = torch.Generator(device="cuda").manual_seed(seed)
        K = torch.randn(B, H, S, 128, generator=g, device="cuda")
        gc = torch.Generator().manual_seed(seed + 1)
        ch = torch.stack([torch.randperm(128, generator=gc)[:4] for _ in range(H)])
        scale = torch.ones(H, 128).scatter_(1, ch, 8.0).view(1, H, 1, 128).cuda()
        K = (K * scale).contiguous()
        Rk = synth.random_rotations(B, H, 128, seed=seed + 2).float().cuda()
        want_sc = op.channel_scores(_np(K), _np(Rk))
        srt = -np.sort(-want_sc, axis=-1)
        if ((srt[..., keep - 1] - srt[..., keep]) / srt[..., keep - 1]).min() > 1e-5:
            break
    else:
        pytest.fail("no fixture seed with a top-k boundary gap above the score rounding")
    sc = prefill.channel_scores(K, Rk)
    idx, mask = prefill.topk_channels(sc, keep)
    mean, _ = prefill.key_covariance(K)
    Rp, dm = prefill.gather_rotation(Rk, idx, mean, torch.float32)
    ks = prefill.rotate_keys(K, Rp)
    torch.cuda.synchronize()
    np.testing.assert_allclose(_np(sc), want_sc, rtol=2e-6)
    wi, wm = op.topk_channels(want_sc, keep)
    np.testing.assert_array_equal(idx.cpu().numpy(), wi)
    np.testing.assert_array_equal(mask.cpu().numpy(), wm)
    wR = np.take_along_axis(_np(Rk), wi[:, :, None, :], axis=-1)
    np.testing.assert_array_equal(_np(Rp), wR)
    wd = op.delta_mu(_np(mean), wR, "float32")
    assert np.abs(_np(dm) - wd).max() <= 1e-5 * np.abs(wd).max() + 1e-7
    wk = op.rotate_keys(_np(K), wR, "float32")
    assert np.abs(_np(ks) - wk).max() <= 1e-5 * np.abs(wk).max()


@pytest.mark.parametrize("dtype,D", [(torch.float32, 128), (torch.float32, 64), (torch.bfloat16, 80)])
@pytest.mark.parametrize("solver", ["eigh", "power_iter"])
def test_update_rotatek_fp32_and_head_dim(dtype, D, solver):
    """ChannelPruner.update_rotatek end to end on fp32 Keys and at D < 128:
    the weighted covariance against the oracle from the Keys, then (eigh)
    R_partial with column signs aligned, or (power iteration) the kept
    projector, and the truncated Keys mapped back."""
    from rotatek_amd import prefill
    from rotatek_amd.pruning import ChannelPruner
    _say(f"update_rotatek {solver} {dtype} D={D}")
    B, H, G, S = 2, 4, 7, 1200
    ratio = 0.875
    # Keys of rank keep (plus noise), so the kept subspace is well separated
    # and five subspace iterations settle on it
    K = _lowrank(B, H, S, D, dtype, seed=D, rank=op.keep_count(D, ratio))
    Q = torch.randn(B, H * G, S, D, device="cuda").to(dtype)
    pr = ChannelPruner(ratio=ratio, prompt_seqlen=30, query_seqlen=40, solver=solver, query_aware=True)
    kept, kp, kt, mask, v = pr.update_rotatek(K, Q, None, None, G)
    vis = K[:, :, 30:S - 40]
    mean, covw = prefill.key_covariance(vis, Q, G)
    torch.cuda.synchronize()
    keep = op.keep_count(D, ratio)
    assert kept.shape == (B, H, S - 70, keep) and kept.dtype == dtype
    assert int(mask[0, 0].sum()) == keep and mask.shape == (B, H, D)
    full = op.update_rotatek(_np(K), _np(Q), 30, 40, ratio, G, DT[dtype], query_aware=True)
    got, want = _np(covw), full["cov"]
    if dtype == torch.float32:
        assert np.abs(got - want).max() <= 1e-5 * np.abs(want).max()
    else:
        # the weighted entries are fp32 products of the covariance stored in
        # the key dtype: one storage ulp of that covariance (where fp32 and
        # fp64 sums round to neighbouring 16-bit values) times the weight is
        # at most two storage ulps of the weighted entry
        err = np.abs(got - want)
        assert np.all(err <= 2 * _storage_ulp(got, want, dtype) + 1e-6 * np.abs(want).max()), err.max()
    ref = op.update_rotatek(_np(K), _np(Q), 30, 40, ratio, G, DT[dtype], query_aware=True,
                            cov=_np(covw), mean=_np(mean))
    R = _np(pr.current_rotatek_R_partial)
    Rw = ref["R_partial"]
    P, Pw = R @ np.swapaxes(R, -1, -2), Rw @ np.swapaxes(Rw, -1, -2)
    assert np.abs(P - Pw).max() <= (2e-3 if solver == "eigh" else 1e-2)
    back = _np(kept) @ np.swapaxes(R, -1, -2)
    want_back = ref["k_sparse"] @ np.swapaxes(Rw, -1, -2)
    assert np.abs(back - want_back).max() <= 1e-2 * np.abs(want_back).max()
