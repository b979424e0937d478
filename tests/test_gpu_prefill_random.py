"""Seeded random shapes for the prefill covariance path against the oracle.

The covariance launches depend on the shape: (B*H, S) set the split counts
of the mean and covariance passes (and so which workgroups hold a partial or
an empty chunk), D < 128 masks channel slots, strided views take the
element-wise loads, and the weighted form adds the query-norm column to the
mean launch and reads the partials' diagonals back for the ridge.  This test
draws 40 shapes with a fixed seed (B 1-4, H 1-6, S from one token to past
several split boundaries, D in {128, 96, 64, 40, 100, 8}, fp16 / bf16 / fp32
Keys, G in {1, 2, 4, 7}, contiguous or sliced out of a longer and wider
buffer;
x8 outlier channels except in fp16, whose covariance would overflow to
infinity as the reference's does) and checks, per shape:

  * the mean against the oracle's fp32 mean (1e-5 relative);
  * the covariance against the oracle centred on the kernel's own mean: one
    storage ulp of the key dtype (fp32 Keys: 1e-5 of the largest entry);
  * the weighted covariance bit for bit against the two-stage result
    (covariance, then the standalone weighting kernel);
  * the weighted covariance against the oracle's weighting applied to the
    kernel's own covariance (1e-5 of the largest entry: fp32 against fp64
    arithmetic on identical inputs).

A second draw of 24 shapes (head dims as above, any keep from 1 to D)
runs the selection and write stages: channel scores, head-wise top-k, the
R_partial / delta_mu gather and the truncated Key write.

Every case prints its parameters before it touches the GPU.
"""
import sys

import numpy as np
import pytest
import torch

from oracle import prefill as op

pytestmark = pytest.mark.gpu

DT = {torch.float16: "float16", torch.bfloat16: "bfloat16", torch.float32: "float32"}
ULP = {torch.float16: 2.0 ** -10, torch.bfloat16: 2.0 ** -7}
S_CHOICES = [1, 2, 7, 31, 32, 33, 255, 256, 257, 511, 513, 1000, 2049, 4097]


def _np(t):
    return t.detach().cpu().to(torch.float64).numpy()


def _say(msg):
    print(f"[case] {msg}", flush=True)
    sys.stdout.flush()


def _storage_ulp(a, b, dtype):
    m = np.maximum(np.abs(a), np.abs(b))
    e = np.floor(np.log2(np.maximum(m, 1e-30)))
    return 2.0 ** e * ULP[dtype]


def _cases(n=40, seed=7):
    rng = np.random.default_rng(seed)
    out = []
    for i in range(n):
        D = int(rng.choice([128, 128, 128, 96, 64, 40, 100, 8]))
        out.append(dict(i=i, B=int(rng.integers(1, 5)), H=int(rng.integers(1, 7)), S=int(rng.choice(S_CHOICES)),
                        D=D, dtype=[torch.float16, torch.bfloat16, torch.float32][int(rng.integers(0, 3))],
                        G=int(rng.choice([1, 2, 4, 7])), sliced=bool(rng.integers(0, 2)),
                        offset=float(rng.choice([0.0, 0.5, 3.0]))))
    return out


@pytest.mark.parametrize("case", _cases(), ids=lambda c: f"{c['i']}")
def test_covariance_random_shapes(case):
    from rotatek_amd import prefill
    c = case
    B, H, S, D, dtype, G = c["B"], c["H"], c["S"], c["D"], c["dtype"], c["G"]
    _say(f"prefill random {c}")
    g = torch.Generator(device="cuda").manual_seed(1000 + c["i"])
    pad = 23 if c["sliced"] else 0
    # sliced views also take a row stride wider than D (16-byte rows stay
    # aligned: D + 32 channels)
    wide = D + 32 if c["sliced"] and D % 8 == 0 else D
    full = torch.randn(B, H, S + 2 * pad, wide, generator=g, device="cuda")
    if dtype != torch.float16:
        # x8 outlier channels; fp16 keeps unit variance, so that a diagonal
        # sum over 4097 tokens stays inside its range (65504)
        full[..., ::37] *= 8.0
    full = (full + c["offset"]).to(dtype)
    K = full[:, :, pad:pad + S, :D]
    Q = torch.randn(B, H * G, 48, D, generator=g, device="cuda").to(dtype)

    mean, cov = prefill.key_covariance(K)
    mean_w, cov_w = prefill.key_covariance(K, Q, G)
    two = prefill.query_weight(cov, Q, G)
    torch.cuda.synchronize()

    Kn = _np(K)
    om, _ = op.key_covariance(Kn, DT[dtype])
    np.testing.assert_allclose(_np(mean), om, rtol=1e-5, atol=1e-6)
    _, oc = op.key_covariance(Kn, DT[dtype], mean=_np(mean))
    got = _np(cov)
    if dtype == torch.float32:
        assert np.abs(got - oc).max() <= 1e-5 * max(np.abs(oc).max(), 1e-30)
    else:
        scale = np.abs(oc).max(axis=(-1, -2), keepdims=True)
        err = np.abs(got - oc)
        assert np.all(err <= _storage_ulp(oc, got, dtype) + 1e-6 * scale), err.max()
    np.testing.assert_array_equal(got, np.swapaxes(got, -1, -2))

    # the weighted launches: the same mean, and the two-stage result bit for bit
    assert torch.equal(mean_w, mean)
    assert torch.equal(cov_w, two)
    ow = op.query_weight(got, _np(Q), G, dtype=DT[dtype])
    assert np.abs(_np(cov_w) - ow).max() <= 1e-5 * np.abs(ow).max()


def _rot_cases(n=24, seed=11):
    rng = np.random.default_rng(seed)
    out = []
    for i in range(n):
        D = int(rng.choice([128, 128, 96, 64, 40, 100, 8]))
        out.append(dict(i=i, B=int(rng.integers(1, 4)), H=int(rng.integers(1, 5)), S=int(rng.choice(S_CHOICES)),
                        D=D, keep=int(rng.integers(1, D + 1)),
                        dtype=[torch.float16, torch.bfloat16, torch.float32][int(rng.integers(0, 3))],
                        sliced=bool(rng.integers(0, 2))))
    return out


@pytest.mark.parametrize("case", _rot_cases(), ids=lambda c: f"{c['i']}")
def test_rotate_score_select_random_shapes(case):
    """The selection and write stages on the same kind of draws: channel
    scores against the oracle on R rounded to the key dtype (1e-5 relative),
    head-wise top-k bit for bit against the oracle's on the kernel's own
    scores, the R_partial gather exact and delta_mu within one storage ulp
    (fp32: 1e-6 relative), the truncated Key write within one storage ulp
    (fp32: 1e-5 of the largest entry)."""
    from rotatek_amd import prefill
    from oracle.numerics import round_to
    c = case
    B, H, S, D, keep, dtype = c["B"], c["H"], c["S"], c["D"], c["keep"], c["dtype"]
    _say(f"rotate/score/select random {c}")
    g = torch.Generator(device="cuda").manual_seed(2000 + c["i"])
    pad = 17 if c["sliced"] else 0
    wide = D + 32 if c["sliced"] and D % 8 == 0 else D
    full = torch.randn(B, H, S + 2 * pad, wide, generator=g, device="cuda")
    K = (full + 0.5).to(dtype)[:, :, pad:pad + S, :D]
    R = torch.linalg.qr(torch.randn(B, H, D, D, generator=g, device="cuda", dtype=torch.float64))[0].float()
    mean = torch.randn(B, H, D, generator=g, device="cuda") * 2

    sc = prefill.channel_scores(K, R)
    idx, mask = prefill.topk_channels(sc, keep)
    Rp, dm = prefill.gather_rotation(R, idx, mean, dtype)
    kept = prefill.rotate_keys(K, Rp)
    torch.cuda.synchronize()

    Kn = _np(K)
    want = op.channel_scores(Kn, round_to(_np(R), DT[dtype]))
    np.testing.assert_allclose(_np(sc), want, rtol=1e-5, atol=1e-7)
    wi, wm = op.topk_channels(_np(sc), keep)
    np.testing.assert_array_equal(idx.cpu().numpy(), wi)
    np.testing.assert_array_equal(mask.cpu().numpy(), wm)
    wR = round_to(np.take_along_axis(_np(R), wi[:, :, None, :], axis=-1), DT[dtype])
    np.testing.assert_array_equal(_np(Rp), wR)
    wd = op.delta_mu(_np(mean), wR, DT[dtype])
    wk = op.rotate_keys(Kn, wR, DT[dtype])
    if dtype == torch.float32:
        assert np.abs(_np(dm) - wd).max() <= 1e-6 * max(np.abs(wd).max(), 1.0)
        assert np.abs(_np(kept) - wk).max() <= 1e-5 * max(np.abs(wk).max(), 1e-30)
    else:
        err = np.abs(_np(dm) - wd)
        assert np.all(err <= _storage_ulp(wd, _np(dm), dtype) + 1e-5), err.max()
        err = np.abs(_np(kept) - wk)
        assert np.all(err <= _storage_ulp(wk, _np(kept), dtype) + 1e-3 * ULP[dtype]), err.max()


def test_prefill_stages_past_the_reported_grid_y():
    """B * H = 66560 heads (B=2080, 32 KV heads, 40 tokens): every prefill
    stage puts the head in blockIdx.y (or x), past the 65536 that
    hipDeviceProp_t.maxGridSize[1] reports.  Sampled heads, the last one
    included, against the oracle as in the random cases above."""
    from rotatek_amd import prefill
    from oracle.numerics import round_to
    B, H, S, D, keep, dtype = 2080, 32, 40, 128, 32, torch.bfloat16
    _say(f"prefill stages B={B} H={H} S={S}")
    g = torch.Generator(device="cuda").manual_seed(4)
    K = (torch.randn(B, H, S, D, generator=g, device="cuda") + 0.5).to(dtype)
    Q = torch.randn(B, H, 8, D, generator=g, device="cuda").to(dtype)
    R1 = torch.linalg.qr(torch.randn(D, D, generator=g, device="cuda", dtype=torch.float64))[0].float()
    R = R1.expand(B, H, D, D).contiguous()
    mean, cov = prefill.key_covariance(K)
    _, cov_w = prefill.key_covariance(K, Q, 1)
    sc = prefill.channel_scores(K, R)
    idx, mask = prefill.topk_channels(sc, keep)
    Rp, dm = prefill.gather_rotation(R, idx, mean, dtype)
    kept = prefill.rotate_keys(K, Rp)
    torch.cuda.synchronize()
    for b, h in ((0, 0), (1037, 17), (B - 1, H - 1)):
        Kn = _np(K[b:b + 1, h:h + 1])
        om, _ = op.key_covariance(Kn, "bfloat16")
        np.testing.assert_allclose(_np(mean[b:b + 1, h:h + 1]), om, rtol=1e-5, atol=1e-6)
        _, oc = op.key_covariance(Kn, "bfloat16", mean=_np(mean[b:b + 1, h:h + 1]))
        got = _np(cov[b:b + 1, h:h + 1])
        scale = np.abs(oc).max()
        assert np.all(np.abs(got - oc) <= _storage_ulp(oc, got, dtype) + 1e-6 * scale)
        ow = op.query_weight(got, _np(Q[b:b + 1, h:h + 1]), 1, dtype="bfloat16")
        assert np.abs(_np(cov_w[b:b + 1, h:h + 1]) - ow).max() <= 1e-5 * np.abs(ow).max()
        want = op.channel_scores(Kn, round_to(_np(R[b:b + 1, h:h + 1]), "bfloat16"))
        np.testing.assert_allclose(_np(sc[b:b + 1, h:h + 1]), want, rtol=1e-5, atol=1e-7)
        wi, wm = op.topk_channels(_np(sc[b:b + 1, h:h + 1]), keep)
        np.testing.assert_array_equal(idx[b:b + 1, h:h + 1].cpu().numpy(), wi)
        np.testing.assert_array_equal(mask[b:b + 1, h:h + 1].cpu().numpy(), wm)
        wR = round_to(np.take_along_axis(_np(R[b:b + 1, h:h + 1]), wi[:, :, None, :], axis=-1), "bfloat16")
        np.testing.assert_array_equal(_np(Rp[b:b + 1, h:h + 1]), wR)
        wk = op.rotate_keys(Kn, wR, "bfloat16")
        err = np.abs(_np(kept[b:b + 1, h:h + 1]) - wk)
        assert np.all(err <= _storage_ulp(wk, _np(kept[b:b + 1, h:h + 1]), dtype) + 1e-3 * ULP[dtype])
