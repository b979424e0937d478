"""Seeded random shapes for the span cache's decode step (rk_rotatek_decode_varlen
with a fused append) against the oracle.

The fused append touches every part of the launch: workgroup 0 of each unit
stages k_new / v_new, the first unit of each KV head stores them at row
len_full[b] (the Value row shifted past the visual span once it lies in the
text part), wave 0 attends the new token, and the merge launch advances
len_full[b] behind its merge.  This test draws 24 cases with a fixed seed:
fp16 / bf16, head_dim 128 / 96 / 64, B 1-4, 1-4 KV heads of 1-7 query
heads, 0-64 kept channels, 0-30 prompt rows, 1-2049 visual tokens, a text
capacity of 8-130 rows, per-row lengths anywhere from 0 to past the
capacity (full rows neither store nor attend the token), an optional
random mask_full, and both decode families.  Each case runs two steps in a
row and checks, per step:

  * the K / V buffers against the expected writes (bit for bit);
  * len_full against the expected advance (exact);
  * the output against the float64 oracle over the rows then attended
    (rows below the old length where mask_full is set, plus the new token)
    at the north-star bars (max-abs 2e-3 fp16, 1e-2 bf16).

Every case prints its parameters before it touches the GPU.
"""
import sys

import numpy as np
import pytest
import torch

from oracle import decode as od

pytestmark = pytest.mark.gpu

TOL = {torch.float16: 2e-3, torch.bfloat16: 1e-2}


def _np(t):
    return None if t is None else t.detach().float().cpu().numpy().astype(np.float64)


def _cases(n=24, seed=515):
    rng = np.random.default_rng(seed)
    out = []
    for i in range(n):
        D = int(rng.choice([128, 128, 96, 64]))
        B = int(rng.integers(1, 5))
        cap = int(rng.choice([8, 40, 130]))
        s_p = int(rng.choice([0, 1, 5, 30]))
        C = s_p + cap
        # lengths: empty, one short of full, full, past full, anywhere
        lens = [int(rng.choice([0, C - 1, C, C + 2, int(rng.integers(0, C + 1))])) for _ in range(B)]
        out.append(dict(i=i, D=D, B=B, Hkv=int(rng.integers(1, 5)), G=int(rng.choice([1, 2, 4, 7])),
                        Dk=int(rng.choice([0, 8, 16, 32, 32, 64])) if D >= 64 else 8,
                        s_p=s_p, s_v=int(rng.choice([1, 63, 200, 777, 2049])), cap=cap, lens=lens,
                        dtype=[torch.float16, torch.bfloat16][int(rng.integers(0, 2))],
                        masked=bool(rng.integers(0, 2)), policy=int(rng.integers(0, 2))))
    return out


@pytest.mark.parametrize("case", _cases(), ids=lambda c: f"{c['i']}")
def test_fused_append_random_shapes(case):
    from rotatek_amd.kernels import _launch
    c = case
    D, B, Hkv, G, Dk, s_p, s_v, cap, dtype = c["D"], c["B"], c["Hkv"], c["G"], c["Dk"], c["s_p"], c["s_v"], \
        c["cap"], c["dtype"]
    C, Hq = s_p + cap, c["Hkv"] * c["G"]
    print(f"[case] fused append random {c}", flush=True)
    sys.stdout.flush()
    g = torch.Generator(device="cuda").manual_seed(5000 + c["i"])

    def rn(*s, scale=1.0):
        return (torch.randn(*s, generator=g, device="cuda") * scale).to(dtype)

    R = torch.linalg.qr(torch.randn(B, Hkv, D, D, generator=g, device="cuda"))[0][..., :Dk].contiguous().to(dtype)
    dm = rn(B, Hkv, D, scale=0.5)
    ks = rn(B, Hkv, s_v, Dk, scale=2.0)
    kf = rn(B, Hkv, C, D)
    vbuf = rn(B, Hkv, s_p + s_v + cap, D)
    mask = (torch.rand(B, C, generator=g, device="cuda") >= 0.3).to(torch.uint8) if c["masked"] else None
    lens = torch.tensor(c["lens"], dtype=torch.int32, device="cuda")
    vrow = np.array([t + (s_v if t >= s_p else 0) for t in range(C)])

    for step in range(2):
        q, kn, vn = rn(B, Hq, D), rn(B, Hkv, 1, D), rn(B, Hkv, 1, D)
        kf0, vb0, lens0 = kf.clone(), vbuf.clone(), lens.cpu().numpy().copy()
        out = _launch.rotatek_decode_varlen(q, R, dm, kf, vbuf, s_p, s_v, mask, ks, vbuf[:, :, s_p:s_p + s_v],
                                            G, lens, c["policy"], k_new=kn, v_new=vn)
        torch.cuda.synchronize()
        kf_want, vb_want = kf0.clone(), vb0.clone()
        att = np.zeros((B, C), dtype=np.uint8)
        m = np.ones((B, C), dtype=np.uint8) if mask is None else mask.cpu().numpy()
        want_lens = lens0.copy()
        for b in range(B):
            pos = min(C, max(int(lens0[b]), 0))
            att[b, :pos] = m[b, :pos]
            if pos < C:
                kf_want[b, :, pos] = kn[b, :, 0]
                vb_want[b, :, int(vrow[pos])] = vn[b, :, 0]
                att[b, pos] = 1
                want_lens[b] = pos + 1
        assert torch.equal(kf, kf_want), step
        assert torch.equal(vbuf, vb_want), step
        np.testing.assert_array_equal(lens.cpu().numpy(), want_lens)
        vf = vb_want[:, :, torch.as_tensor(vrow, device="cuda")]
        want = od.rotatek_decode(_np(q), _np(R), _np(dm), _np(kf_want), _np(vf), att, _np(ks),
                                 _np(vb_want[:, :, s_p:s_p + s_v]), G)
        got = _np(out)[:, None]  # [B, H_q, D] against the oracle's [B, 1, H_q, D]
        assert got.shape == want.shape
        assert np.isfinite(got).all()
        err = float(np.abs(got - want).max())
        assert err <= TOL[dtype], (step, err)
