"""GPU parity of the ThinK / SparK baseline kernels at head dims below 128
(rotatek/baselines/think.py:35-36 and spark.py:34-36 take D from the Keys'
last dim): channel slots past D take no part in the selection, and nothing
is read or written past D.

On grid inputs (values m/8: every square and sum exact in fp32) the masks,
compact Keys and pruned means equal the oracle bit for bit (oracle/
baselines.py, itself D-generic), at D in {64, 80, 96} (16-byte rows) and
{40, 5} (element-wise rows, D % 8 != 0), for prune counts 0, D/4, D/2,
D - 1 and D; on random inputs through strided views the selection agrees
with the oracle's scores up to one storage ulp.  The recovery and the
one-hot selection rotation are bit-exact at the same head dims.
"""
import sys

import numpy as np
import pytest
import torch

from oracle import baselines as ob

pytestmark = pytest.mark.gpu

DT = {torch.float16: "float16", torch.bfloat16: "bfloat16"}
ULP = {torch.float16: 2.0 ** -10, torch.bfloat16: 2.0 ** -7}
DIMS = [64, 80, 96, 40, 5]


def _say(msg):
    print(f"[case] {msg}", flush=True)
    sys.stdout.flush()


def _np(t):
    return t.detach().cpu().to(torch.float64).numpy()


def _grid(shape, dtype, seed):
    g = torch.Generator().manual_seed(seed)
    return (torch.randint(-15, 16, shape, generator=g).to(torch.float32) / 8).to(dtype).cuda()


def _rand(shape, dtype, seed):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(shape, generator=g)
    x[..., ::9] *= 6.0
    return x.to(dtype).cuda()


def _same(a, b, what):
    a, b = np.asarray(a, np.float64), np.asarray(b, np.float64)
    assert a.shape == b.shape, (what, a.shape, b.shape)
    np.testing.assert_array_equal(a, b, err_msg=what)


def _prunes(D):
    return sorted({0, D // 4, D // 2, D - 1, D})


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("D", DIMS)
def test_think_grid_head_dim(dtype, D):
    from rotatek_amd.baselines import think_score_and_compact
    B, H, G, S, W = 2, 4, 7, 700, 16
    K = _grid((B, H, S, D), dtype, 1 + D)
    Q = _grid((B, H * G, W, D), dtype, 2 + D)
    for prune in _prunes(D):
        _say(f"think grid {dtype} D={D} prune={prune}")
        Kc, mask = think_score_and_compact(K, Q, H, prune)
        torch.cuda.synchronize()
        Kc_o, mask_o, _ = ob.think_score_and_compact(_np(K), _np(Q), H, prune, DT[dtype])
        _same(mask.cpu().numpy(), mask_o, f"keep_mask D={D} prune={prune}")
        _same(_np(Kc), Kc_o, f"K_compact D={D} prune={prune}")


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("D", [80, 40])
def test_think_random_strided_head_dim(dtype, D):
    """A channel stride of 2 (element path) gives what the contiguous copy
    gives, and the selection agrees with the oracle's scores."""
    from rotatek_amd.baselines import think_score_and_compact
    B, H, G, S, W, prune = 2, 4, 2, 1500, 32, D // 2
    _say(f"think random strided {dtype} D={D}")
    K = _rand((B, H, S, 2 * D), dtype, 3)[..., ::2]
    Q = _rand((B, H * G, W, D), dtype, 4)
    Kc, mask = think_score_and_compact(K, Q, H, prune)
    Kc2, mask2 = think_score_and_compact(K.contiguous(), Q, H, prune)
    torch.cuda.synchronize()
    assert torch.equal(mask, mask2) and torch.equal(Kc, Kc2)
    m = mask.cpu().numpy()
    assert (m.sum(-1) == D - prune).all()
    _, _, scores = ob.think_score_and_compact(_np(K), _np(Q), H, prune, DT[dtype])
    s = np.where(np.isnan(scores), np.inf, scores)
    kept_min = np.where(m, s, np.inf).min(-1)
    pruned_max = np.where(~m, s, -np.inf).max(-1)
    assert np.all(pruned_max <= kept_min + ULP[dtype] * np.abs(kept_min))


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("D", DIMS)
def test_spark_grid_head_dim(dtype, D):
    from rotatek_amd.baselines import spark_prune
    B, H, G, S, W = 2, 2, 4, 513, 8
    K = _grid((B, H, S, D), dtype, 5 + D)
    Q = _grid((B, H * G, W, D), dtype, 6 + D)
    qg = ob.group_queries(_np(Q), G, DT[dtype])
    for prune in _prunes(D):
        _say(f"spark grid {dtype} D={D} prune={prune}")
        Kc, mask, pm = spark_prune(K, Q, G, prune)
        torch.cuda.synchronize()
        Kc_o, mask_o, pm_o, _ = ob.per_token_channel_prune(qg, _np(K), prune, DT[dtype])
        _same(mask.cpu().numpy(), mask_o, f"keep_mask D={D} prune={prune}")
        _same(_np(Kc), Kc_o, f"K_compact D={D} prune={prune}")
        _same(_np(pm), pm_o, f"pruned_mean D={D} prune={prune}")   # NaN == NaN at prune 0


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("D", [96, 40])
def test_spark_random_strided_head_dim(dtype, D):
    from rotatek_amd.baselines import spark_prune
    B, H, G, S, W, prune = 2, 2, 7, 900, 16, (3 * D) // 4
    _say(f"spark random strided {dtype} D={D}")
    K = _rand((B, H, S, 2 * D), dtype, 7)[..., 1::2]
    Q = _rand((B, H * G, W, D), dtype, 8)
    Kc, mask, pm = spark_prune(K, Q, G, prune)
    Kc2, mask2, pm2 = spark_prune(K.contiguous(), Q, G, prune)
    torch.cuda.synchronize()
    assert torch.equal(mask, mask2) and torch.equal(Kc, Kc2) and torch.equal(pm, pm2)
    m = mask.cpu().numpy()
    assert (m.sum(-1) == D - prune).all()
    Kn = _np(K)
    _same(_np(Kc), Kn[m].reshape(B, H, S, D - prune), "K_compact")


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("D", [64, 80, 40])
def test_recover_head_dim(dtype, D):
    """[prompt | recovered | text] rows of width D, into a fresh buffer and
    a strided slice, equal the oracle's assembly bit for bit."""
    from rotatek_amd.baselines import recover_spark, recover_think, spark_prune, think_score_and_compact
    B, H, G, S, W, s_p, s_t = 2, 2, 2, 640, 8, 7, 3
    _say(f"recover {dtype} D={D}")
    K = _rand((B, H, S, D), dtype, 11)
    Q = _rand((B, H * G, W, D), dtype, 12)
    P = _rand((B, H, s_p, D), dtype, 13)
    T = _rand((B, H, s_t, D), dtype, 14)
    rows = s_p + S + s_t
    Kc, tm = think_score_and_compact(K, Q, H, D // 2)
    Kc2, sm, pm = spark_prune(K, Q, G, (3 * D) // 4)
    for layout in ("fresh", "strided"):
        out_t = None if layout == "fresh" else torch.full((B, H, rows, 2 * D), 7.0, dtype=dtype, device="cuda")[..., ::2]
        out_s = None if layout == "fresh" else torch.full((B, H, rows, 2 * D), 7.0, dtype=dtype, device="cuda")[..., ::2]
        Rt = recover_think(Kc, tm, out=out_t, k_prompt=P, k_text=T)
        Rs = recover_spark(Kc2, sm, pm, out=out_s, k_prompt=P, k_text=T)
        torch.cuda.synchronize()
        assert Rt.shape == (B, H, rows, D) and Rs.shape == (B, H, rows, D)
        _same(_np(Rt), ob.assemble(_np(P), ob.recover_think(_np(Kc), tm.cpu().numpy()), _np(T)), f"think {layout}")
        _same(_np(Rs), ob.assemble(_np(P), ob.recover_spark(_np(Kc2), sm.cpu().numpy(), _np(pm)), _np(T)),
              f"spark {layout}")


@pytest.mark.parametrize("D", [80, 5])
def test_selection_rotation_head_dim(D):
    from rotatek_amd.baselines import selection_rotation, think_score_and_compact
    _say(f"selection rotation D={D}")
    B, H, keep = 2, 3, max(D // 2, 1)
    K = _rand((B, H, 300, D), torch.bfloat16, 15)
    Q = _rand((B, 2 * H, 8, D), torch.bfloat16, 16)
    _, mask = think_score_and_compact(K, Q, H, D - keep)
    R = selection_rotation(mask, keep, torch.float32)
    torch.cuda.synchronize()
    m = mask.cpu().numpy()
    want = np.zeros((B, H, D, keep))
    for b in range(B):
        for h in range(H):
            for j, c in enumerate(np.flatnonzero(m[b, h])):
                want[b, h, c, j] = 1.0
    _same(_np(R), want, "R")
