"""Seeded random decode shapes against the CPU oracle.

The grid planner, the per-unit chunk rotation (XCD balance) and the grouped
one-unit-per-query-head mapping all depend on the shape: (B, H_q, H_kv,
D_keep, S_v, S_f) decide the workgroups per unit, whether chunk numbers are
rotated, and which workgroup ids carry which (unit, chunk).  This test draws
48 shapes with a fixed seed over both families and both 16-bit dtypes,
including odd and empty spans, G up to 20 and D_keep from 8 to 128, and
checks every output against the float64 oracle at the north-star bars
(max-abs 2e-3 fp16, 1e-2 bf16), under each planner layout of one-round
grids (unit-major, chunk-major, chunk-major with enlarged first-dispatched
chunks at two workgroups per CU, the default, which takes one workgroup per
CU for a round of small workgroups).  A second draw of 32 shapes runs
fp32 inputs (the VALU kernels, one query head per unit or grouped units of
up to 8 heads of one KV head; D_keep from 0 to 128, G up to 16) at max-abs
1e-4.  A third draw of 24 runs the full-channel baseline through both of its
entries (head dims 8-128, 1 to 9001 tokens, G up to 20, fp16 / bf16 / fp32,
contiguous or sliced K / V).  Every case prints its parameters first.
"""
import sys

import numpy as np
import pytest
import torch

from oracle import decode as od

pytestmark = pytest.mark.gpu

TOL = {torch.float16: 2e-3, torch.bfloat16: 1e-2}
D = 128


def _cases(n=48, seed=2024):
    rng = np.random.default_rng(seed)
    out = []
    for i in range(n):
        hkv = int(rng.choice([1, 2, 4, 8]))
        G = int(rng.choice([1, 1, 2, 4, 7, 8, 16, 20]))
        B = int(rng.choice([1, 2, 3, 5]))
        dk = int(rng.choice([8, 16, 24, 32, 32, 40, 64, 128]))
        S_v = int(rng.choice([0, 1, 63, 129, 777, 2049, 4097, 9001]))
        S_f = int(rng.choice([0, 1, 17, 80, 300, 1025]))
        if S_v + S_f == 0:
            S_f = 5
        dtype = torch.float16 if rng.random() < 0.5 else torch.bfloat16
        family = "paper" if rng.random() < 0.5 else "gqa"
        mask_p = float(rng.choice([0.0, 0.0, 0.3]))
        out.append((i, B, hkv * G, hkv, dk, S_v, S_f, dtype, family, mask_p))
    return out


CASES = _cases()


@pytest.fixture
def planner(request):
    from rotatek_amd import _lib
    skew, wgs = request.param
    _lib.set_decode_skew(skew)
    _lib.set_decode_tuning(0, 0, wgs)
    yield request.param
    _lib.set_decode_skew(1300)
    _lib.set_decode_tuning(0, 0, -1)


# planner layouts of one-round grids, (skew permille, workgroups per CU):
# unit-major, chunk-major, chunk-major with the first-dispatched chunks
# enlarged for short workgroups (two per CU), the default (-1)
@pytest.mark.parametrize("planner", [(0, -1), (1000, 2), (1300, 2), (1300, -1)], indirect=True,
                         ids=["um", "cm", "skew", "default"])
@pytest.mark.parametrize("case", CASES, ids=[f"c{c[0]}" for c in CASES])
def test_random_shape_matches_oracle(case, planner):
    from rotatek_amd.kernels.fused_decode import rotatek_decode_fused
    from rotatek_amd.kernels.gqa_decode import rotatek_decode_gqa
    i, B, Hq, Hkv, dk, S_v, S_f, dtype, family, mask_p = case
    print(f"[case] {case} planner={planner}", flush=True)
    sys.stdout.flush()
    g = torch.Generator(device="cuda").manual_seed(1000 + i)

    def rn(*s, scale=1.0):
        return (torch.randn(*s, generator=g, device="cuda") * scale).to(dtype)

    R = torch.linalg.qr(torch.randn(B, Hkv, D, D, generator=g, device="cuda"))[0][..., :dk].contiguous().to(dtype)
    V = rn(B, Hkv, S_v + S_f, D)
    mask = (torch.rand(B, S_f, generator=g, device="cuda") >= mask_p).to(torch.uint8)
    inp = dict(q_full=rn(B, Hq, D), R_partial=R, delta_mu=rn(B, Hkv, D, scale=0.5), k_full=rn(B, Hkv, S_f, D),
               v_full=V[:, :, S_v:], mask_full=mask, k_sparse=rn(B, Hkv, S_v, dk, scale=2.0),
               v_sparse=V[:, :, :S_v], num_kv_groups=Hq // Hkv)
    fn = rotatek_decode_gqa if family == "gqa" else rotatek_decode_fused
    out = fn(**inp)[0]
    torch.cuda.synchronize()
    a = {k: (v.detach().float().cpu().numpy().astype(np.float64) if torch.is_tensor(v) else v)
         for k, v in inp.items()}
    want = od.rotatek_decode(a["q_full"], a["R_partial"], a["delta_mu"], a["k_full"], a["v_full"],
                             a["mask_full"], a["k_sparse"], a["v_sparse"], a["num_kv_groups"])
    got = out.float().cpu().numpy().astype(np.float64)
    assert got.shape == want.shape
    err = float(np.nanmax(np.abs(got - want))) if got.size else 0.0
    assert np.isfinite(got).all() and err <= TOL[dtype], (case, err)


def _cases32(n=32, seed=4242):
    rng = np.random.default_rng(seed)
    out = []
    for i in range(n):
        hkv = int(rng.choice([1, 2, 4]))
        G = int(rng.choice([1, 1, 2, 3, 7, 8, 9, 16]))
        B = int(rng.choice([1, 2, 3]))
        dk = int(rng.choice([0, 8, 16, 32, 32, 40, 64, 128]))
        S_v = int(rng.choice([0, 1, 63, 129, 777, 2049, 4097]))
        S_f = int(rng.choice([0, 1, 17, 80, 300, 1025]))
        if S_v + S_f == 0:
            S_f = 5
        family = "paper" if rng.random() < 0.5 else "gqa"
        mask_p = float(rng.choice([0.0, 0.0, 0.3]))
        out.append((i, B, hkv * G, hkv, dk, S_v, S_f, torch.float32, family, mask_p))
    return out


CASES32 = _cases32()


@pytest.mark.parametrize("case", CASES32, ids=[f"f{c[0]}" for c in CASES32])
def test_random_shape_fp32_matches_oracle(case):
    """fp32 inputs (the VALU kernels: one query head per unit, or up to 8
    heads of one KV head sharing its K/V rows), random shapes including
    zero kept channels, empty and odd spans and groups of 9 and 16 heads
    (two units per KV head), max-abs 1e-4 against the float64 oracle."""
    from rotatek_amd.kernels.fused_decode import rotatek_decode_fused
    from rotatek_amd.kernels.gqa_decode import rotatek_decode_gqa
    i, B, Hq, Hkv, dk, S_v, S_f, dtype, family, mask_p = case
    print(f"[case] fp32 {case}", flush=True)
    sys.stdout.flush()
    g = torch.Generator(device="cuda").manual_seed(3000 + i)

    def rn(*s, scale=1.0):
        return torch.randn(*s, generator=g, device="cuda") * scale

    R = torch.linalg.qr(torch.randn(B, Hkv, D, D, generator=g, device="cuda"))[0][..., :dk].contiguous()
    V = rn(B, Hkv, S_v + S_f, D)
    mask = (torch.rand(B, S_f, generator=g, device="cuda") >= mask_p).to(torch.uint8)
    inp = dict(q_full=rn(B, Hq, D), R_partial=R, delta_mu=rn(B, Hkv, D, scale=0.5), k_full=rn(B, Hkv, S_f, D),
               v_full=V[:, :, S_v:], mask_full=mask, k_sparse=rn(B, Hkv, S_v, dk, scale=2.0),
               v_sparse=V[:, :, :S_v], num_kv_groups=Hq // Hkv)
    fn = rotatek_decode_gqa if family == "gqa" else rotatek_decode_fused
    out = fn(**inp)[0]
    torch.cuda.synchronize()
    a = {k: (v.detach().cpu().numpy().astype(np.float64) if torch.is_tensor(v) else v) for k, v in inp.items()}
    want = od.rotatek_decode(a["q_full"], a["R_partial"], a["delta_mu"], a["k_full"], a["v_full"],
                             a["mask_full"], a["k_sparse"], a["v_sparse"], a["num_kv_groups"])
    got = out.cpu().numpy().astype(np.float64)
    assert got.shape == want.shape
    err = float(np.nanmax(np.abs(got - want))) if got.size else 0.0
    assert np.isfinite(got).all() and err <= 1e-4, (case, err)


def _dense_cases(n=24, seed=99):
    rng = np.random.default_rng(seed)
    out = []
    for i in range(n):
        hkv = int(rng.choice([1, 2, 4, 8]))
        out.append(dict(i=i, B=int(rng.choice([1, 2, 3, 5])), Hkv=hkv, G=int(rng.choice([1, 1, 2, 4, 7, 16, 20])),
                        S=int(rng.choice([1, 2, 31, 33, 257, 1000, 4097, 9001])),
                        D=int(rng.choice([128, 128, 96, 64, 40, 8])),
                        dtype=[torch.float16, torch.bfloat16, torch.float32][int(rng.integers(0, 3))],
                        strided=bool(rng.integers(0, 2))))
    return out


@pytest.mark.parametrize("case", _dense_cases(), ids=lambda c: f"d{c['i']}")
def test_dense_baseline_random_shapes(case):
    """The full-channel baseline (rk_full_channel_decode) on seeded random
    shapes: both entries (one unit per query head, and the grouped one that
    reads each K / V row once per KV head), head dims 8-128, one to 9001
    tokens, G up to 20, fp16 / bf16 / fp32, contiguous or sliced K / V,
    against the float64 oracle at the decode bars (fp32: 1e-4)."""
    from rotatek_amd.kernels.full_channel_flash_decoding import full_channel_decode
    from rotatek_amd.kernels.gqa_decode import full_channel_decode_gqa
    c = case
    B, Hkv, G, S, D, dtype = c["B"], c["Hkv"], c["G"], c["S"], c["D"], c["dtype"]
    print(f"[case] dense random {c}", flush=True)
    sys.stdout.flush()
    g = torch.Generator(device="cuda").manual_seed(7000 + c["i"])

    def rn(*s):
        return torch.randn(*s, generator=g, device="cuda").to(dtype)

    q = rn(B, Hkv * G, D)
    if c["strided"]:
        big_k, big_v = rn(B, Hkv, S + 9, D + 8 if D % 8 == 0 else D), rn(B, Hkv, S + 9, D)
        k, v = big_k[:, :, 4:4 + S, :D], big_v[:, :, 5:5 + S]
    else:
        k, v = rn(B, Hkv, S, D), rn(B, Hkv, S, D)
    want = od.full_channel_decode(_np_t(q), _np_t(k), _np_t(v), G)
    tol = 1e-4 if dtype == torch.float32 else TOL[dtype]
    for fn in (full_channel_decode, full_channel_decode_gqa):
        out = fn(q, k, v, G)
        torch.cuda.synchronize()
        got = _np_t(out)
        assert got.shape == want.shape
        assert np.isfinite(got).all()
        err = float(np.abs(got - want).max())
        assert err <= tol, (fn.__name__, err)


def _np_t(t):
    return t.detach().float().cpu().numpy().astype(np.float64)
