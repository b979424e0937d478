"""GPU parity of the decode kernels at head sizes other than 128.

The reference's kernels take any head size: they pad D to a power-of-two
block and mask the channels past D (fused_decode.py:128, 341-342;
full_channel_flash_decoding.py:61, 175-185; gqa_decode.py:92, 243-274), with
scale 1/sqrt(D).  Here the same kernels mask the channels past D: 16-byte row
loads where D is a multiple of 8, element-wise loads otherwise.  Every case
is checked against the float64 oracle at the decode bars (fp16 2e-3, bf16
1e-2, fp32 1e-4 max-abs), and the single-launch merge must stay bit-identical
to the two-launch one.
"""
import sys

import numpy as np
import pytest
import torch

from oracle import decode as od
from rotatek_amd import _lib

pytestmark = pytest.mark.gpu

TOL = {torch.float16: 2e-3, torch.bfloat16: 1e-2, torch.float32: 1e-4}


def _np(t):
    return None if t is None else t.detach().float().cpu().numpy().astype(np.float64)


def _say(msg):
    print(f"[case] {msg}", flush=True)
    sys.stdout.flush()


def _inputs(B, Hq, Hkv, D, Dk, S_v, S_f, dtype, seed, strided=False, mask_p=0.2):
    g = torch.Generator(device="cuda").manual_seed(seed)

    def rn(*s, scale=1.0):
        return (torch.randn(*s, generator=g, device="cuda") * scale).to(dtype)

    R = torch.linalg.qr(torch.randn(B, Hkv, D, D, generator=g, device="cuda"))[0][..., :Dk].contiguous()
    R = R.to(dtype) if dtype != torch.float32 else R
    if strided:
        # channel stride 2 everywhere: the element-wise kernels
        V = rn(B, Hkv, S_v + S_f, 2 * D)[..., ::2]
        kf = rn(B, Hkv, S_f, 2 * D)[..., ::2]
        q = rn(B, Hq, 2 * D)[..., ::2]
    else:
        V = rn(B, Hkv, S_v + S_f, D)
        kf = rn(B, Hkv, S_f, D)
        q = rn(B, Hq, D)
    return dict(q_full=q, R_partial=R, delta_mu=rn(B, Hkv, D, scale=0.5), k_full=kf, v_full=V[:, :, S_v:],
                mask_full=(torch.rand(B, S_f, generator=g, device="cuda") >= mask_p).to(torch.uint8),
                k_sparse=rn(B, Hkv, S_v, Dk, scale=2.0), v_sparse=V[:, :, :S_v], num_kv_groups=Hq // Hkv)


def _oracle(inp):
    a = {k: (_np(v) if torch.is_tensor(v) else v) for k, v in inp.items()}
    return od.rotatek_decode(a["q_full"], a["R_partial"], a["delta_mu"], a["k_full"], a["v_full"],
                             a["mask_full"], a["k_sparse"], a["v_sparse"], a["num_kv_groups"])


def _decode(inp, family):
    from rotatek_amd.kernels.fused_decode import rotatek_decode_fused
    from rotatek_amd.kernels.gqa_decode import rotatek_decode_gqa
    fn = rotatek_decode_gqa if family == "gqa" else rotatek_decode_fused
    out = fn(**inp)[0]
    torch.cuda.synchronize()
    return out


CASES = [
    # B, Hq, Hkv, D, Dk, S_v, S_f
    (2, 8, 8, 64, 16, 1000, 129),    # D = 64: half the channel slots
    (1, 28, 4, 64, 32, 2049, 100),   # ... G = 7
    (2, 8, 4, 80, 24, 517, 64),      # D = 80: a partial 32-channel block
    (1, 28, 4, 80, 40, 900, 33),
    (2, 4, 4, 96, 32, 640, 70),      # D = 96
    (1, 16, 2, 96, 72, 700, 40),     # ... R staged whole (Dk > 64)
    (2, 4, 4, 112, 96, 300, 20),
    (1, 8, 8, 40, 8, 333, 31),       # D = 40
    (1, 4, 4, 8, 8, 129, 17),        # D = 8: one slot
    (2, 4, 4, 64, 64, 0, 300),       # no visual span
    (2, 4, 4, 80, 16, 1025, 0),      # no prompt/text span
    (1, 4, 4, 64, 0, 200, 30),       # no kept channel
]


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("family", ["paper", "gqa"])
@pytest.mark.parametrize("case", CASES)
def test_rotatek_decode_head_dim(case, family, dtype):
    B, Hq, Hkv, D, Dk, S_v, S_f = case
    _say(f"head_dim rotatek {family} {dtype} B={B} Hq={Hq} Hkv={Hkv} D={D} Dk={Dk} S_v={S_v} S_f={S_f}")
    inp = _inputs(B, Hq, Hkv, D, Dk, S_v, S_f, dtype, seed=sum(case) + D)
    out = _decode(inp, family)
    assert out.shape == (B, 1, Hq, D) and out.dtype == dtype
    err = np.abs(_np(out) - _oracle(inp)).max()
    assert err <= TOL[dtype], err


@pytest.mark.parametrize("D,Dk", [(100, 20), (72, 12), (33, 7), (1, 1), (127, 64)])
@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_rotatek_decode_head_dim_not_a_multiple_of_8(D, Dk, dtype):
    """D % 8 != 0: no 16-byte slots, the element-wise kernel; loads past D
    are not issued."""
    _say(f"head_dim {D} (element-wise) {dtype} Dk={Dk}")
    inp = _inputs(2, 8, 4, D, Dk, 700, 45, dtype, seed=D)
    out = _decode(inp, "gqa")
    assert out.shape == (2, 1, 8, D)
    assert np.abs(_np(out) - _oracle(inp)).max() <= TOL[dtype]


@pytest.mark.parametrize("D", [64, 80, 96])
def test_rotatek_decode_head_dim_strided(D):
    """Channel stride 2 (element-wise kernel) at D < 128."""
    _say(f"head_dim {D} strided bf16")
    inp = _inputs(2, 8, 4, D, 32, 900, 50, torch.bfloat16, seed=D + 3, strided=True)
    out = _decode(inp, "gqa")
    assert np.abs(_np(out) - _oracle(inp)).max() <= TOL[torch.bfloat16]


@pytest.mark.parametrize("D,Dk", [(64, 16), (80, 32), (96, 40), (36, 12), (30, 6)])
@pytest.mark.parametrize("family", ["paper", "gqa"])
def test_rotatek_decode_head_dim_fp32(D, Dk, family):
    """fp32 (the VALU kernel): D a multiple of 4 takes 16-byte rows, others
    element-wise loads."""
    _say(f"head_dim {D} fp32 {family} Dk={Dk}")
    inp = _inputs(1, 8, 4, D, Dk, 1100, 60, torch.float32, seed=D + Dk)
    out = _decode(inp, family)
    assert out.dtype == torch.float32 and out.shape == (1, 1, 8, D)
    assert np.abs(_np(out) - _oracle(inp)).max() <= TOL[torch.float32]


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16, torch.float32])
@pytest.mark.parametrize("D", [64, 80, 96, 50])
@pytest.mark.parametrize("family", ["paper", "gqa"])
def test_dense_decode_head_dim(D, family, dtype):
    """The full-channel baseline (both families; the paper family at G > 1
    keeps one unit per query head) against the oracle's dense attention."""
    from rotatek_amd.kernels.full_channel_flash_decoding import full_channel_decode
    from rotatek_amd.kernels.gqa_decode import full_channel_decode_gqa
    _say(f"head_dim dense {family} {dtype} D={D}")
    g = torch.Generator(device="cuda").manual_seed(D)
    q = torch.randn(2, 8, D, generator=g, device="cuda").to(dtype)
    k = torch.randn(2, 2, 1500, D, generator=g, device="cuda").to(dtype)
    v = torch.randn(2, 2, 1500, D, generator=g, device="cuda").to(dtype)
    fn = full_channel_decode_gqa if family == "gqa" else full_channel_decode
    out = fn(q, k, v, num_kv_groups=4)
    torch.cuda.synchronize()
    assert out.shape == (2, 1, 8, D)
    want = od.full_channel_decode(_np(q), _np(k), _np(v), 4)
    assert np.abs(_np(out) - want).max() <= TOL[dtype]


@pytest.mark.parametrize("D", [64, 80])
def test_head_dim_merges_bit_identical(D):
    """Single-launch and two-launch merges agree bit for bit at D < 128."""
    _say(f"head_dim {D} merge modes")
    inp = _inputs(1, 32, 32, D, 16, 6000, 200, torch.float16, seed=D + 9)
    try:
        _lib.set_decode_merge(_lib.MERGE_TWO_LAUNCHES)
        two = _decode(inp, "paper")
        _lib.set_decode_merge(_lib.MERGE_SINGLE_LAUNCH)
        one = _decode(inp, "paper")
    finally:
        _lib.set_decode_merge(_lib.MERGE_AUTO)
    assert torch.equal(one, two)
    assert np.abs(_np(one) - _oracle(inp)).max() <= TOL[torch.float16]


def test_head_dim_channels_past_d_are_not_read():
    """Inputs that are views of wider tensors whose extra channels hold inf
    and NaN: a kernel that read or attended channels past D would return
    non-finite outputs."""
    _say("head_dim 64 views of 128-wide tensors with poisoned channels")
    D, Dk, B, Hq, Hkv, S_v, S_f = 64, 16, 2, 8, 4, 800, 90
    ref = _inputs(B, Hq, Hkv, D, Dk, S_v, S_f, torch.bfloat16, seed=5)
    wide = {}
    for name in ("q_full", "delta_mu", "k_full", "v_full", "v_sparse"):
        t = ref[name]
        w = torch.full(t.shape[:-1] + (128,), float("inf"), dtype=t.dtype, device="cuda")
        w[..., D + 1::2] = float("nan")
        w[..., :D] = t
        wide[name] = w[..., :D]
    inp = dict(ref, **wide)
    out = _decode(inp, "gqa")
    assert torch.isfinite(out.float()).all()
    assert np.abs(_np(out) - _oracle(ref)).max() <= TOL[torch.bfloat16]


@pytest.mark.parametrize("D", [64, 80])
def test_span_cache_decode_step_head_dim(D):
    """The span cache at D < 128: decode_step (fused append through
    rk_rotatek_decode_varlen) over five steps, each against the oracle over
    the spans as they grow, then a plain append (rk_append_kv)."""
    from rotatek_amd.cache import DynamicCache
    _say(f"span cache decode_step head_dim {D}")
    B, Hkv, G, S_p, S_v, S_t, Dk = 2, 4, 2, 5, 700, 9, 16
    dt = torch.bfloat16
    g = torch.Generator(device="cuda").manual_seed(D)

    def rn(*s):
        return torch.randn(*s, generator=g, device="cuda").to(dt)

    cache = DynamicCache(reserve_tokens=8)
    R = torch.linalg.qr(torch.randn(B, Hkv, D, D, generator=g, device="cuda"))[0][..., :Dk].contiguous().to(dt)
    ks, kp, kt = rn(B, Hkv, S_v, Dk), rn(B, Hkv, S_p, D), rn(B, Hkv, S_t, D)
    V = rn(B, Hkv, S_p + S_v + S_t, D)
    dm = rn(B, Hkv, D)
    cache.store_pruned(ks, kp, kt, torch.ones(B, Hkv, D, dtype=torch.bool, device="cuda"), V, 0)
    cache.rotatek_rotations.append(R)
    cache.rotatek_means.append(dm)
    kfull, vfull = torch.cat([kp, kt], 2), torch.cat([V[:, :, :S_p], V[:, :, S_p + S_v:]], 2)
    for step in range(5):
        q, kn, vn = rn(B, Hkv * G, D), rn(B, Hkv, 1, D), rn(B, Hkv, 1, D)
        out = cache.decode_step(q, kn, vn, 0, G)[0]
        torch.cuda.synchronize()
        kfull, vfull = torch.cat([kfull, kn], 2), torch.cat([vfull, vn], 2)
        want = od.rotatek_decode(_np(q), _np(R), _np(dm), _np(kfull), _np(vfull), None, _np(ks),
                                 _np(V[:, :, S_p:S_p + S_v]), G)
        assert out.shape == (B, 1, Hkv * G, D)
        assert np.abs(_np(out) - want).max() <= TOL[dt], step
    cache.sync_lengths()
    assert cache.get_seq_length(0) == S_p + S_v + S_t + 5
    kn, vn = rn(B, Hkv, 1, D), rn(B, Hkv, 1, D)
    cache.append_(0, kn, vn)
    torch.cuda.synchronize()
    cache.sync_lengths()
    assert cache.get_seq_length(0) == S_p + S_v + S_t + 6
    assert torch.equal(cache.key_cache_text[0][:, :, -1:], kn)
