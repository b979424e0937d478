"""Seeded random shapes for the ThinK / SparK baselines against the oracle.

The baseline launches split the token span of each head across workgroups
(score partials, compaction chunks) and size their grids by (B*H, S), so the
shape decides which workgroups hold partial or empty chunks.  Each draw here
takes grid inputs (values m/8: every square and sum is exact in fp32, so the
selection, the compact Keys and the pruned means are bit-exact whatever the
summation order), B 1-3, H 1-4, S from 0 to 2049 tokens, query windows of
1-32 rows, any prune count 0..128 and both 16-bit dtypes.  ThinK takes
groups of 1-7 query heads; SparK groups of 1, 2 or 4 (a group mean over a
count that is not a power of two rounds, after which its squares no longer
sum exactly).  Every case prints its parameters before it touches the GPU.
"""
import sys

import numpy as np
import pytest
import torch

from oracle import baselines as ob

pytestmark = pytest.mark.gpu

D = 128
DT = {torch.float16: "float16", torch.bfloat16: "bfloat16"}


def _np(t):
    return t.detach().cpu().to(torch.float64).numpy()


def _grid(shape, dtype, seed):
    g = torch.Generator().manual_seed(seed)
    return (torch.randint(-15, 16, shape, generator=g).to(torch.float32) / 8).to(dtype).cuda()


def _same(a, b, what):
    a, b = np.asarray(a, np.float64), np.asarray(b, np.float64)
    assert a.shape == b.shape, (what, a.shape, b.shape)
    np.testing.assert_array_equal(a, b, err_msg=what)


def _cases(n, seed, groups):
    rng = np.random.default_rng(seed)
    return [dict(i=i, B=int(rng.integers(1, 4)), H=int(rng.integers(1, 5)), G=int(rng.choice(groups)),
                 S=int(rng.choice([0, 1, 7, 33, 255, 700, 2049])), W=int(rng.choice([1, 3, 8, 32])),
                 prune=int(rng.choice([0, 1, 17, 64, 96, 127, 128])),
                 dtype=[torch.float16, torch.bfloat16][int(rng.integers(0, 2))]) for i in range(n)]


@pytest.mark.parametrize("case", _cases(20, 41, [1, 2, 3, 4, 7]), ids=lambda c: f"t{c['i']}")
def test_think_random_shapes(case):
    from rotatek_amd.baselines import think_score_and_compact
    c = case
    B, H, G, S, W, prune, dtype = c["B"], c["H"], c["G"], c["S"], c["W"], c["prune"], c["dtype"]
    print(f"[case] think random {c}", flush=True)
    sys.stdout.flush()
    K = _grid((B, H, S, D), dtype, 100 + c["i"])
    Q = _grid((B, H * G, W, D), dtype, 200 + c["i"])
    Kc, mask = think_score_and_compact(K, Q, H, prune)
    torch.cuda.synchronize()
    Kc_o, mask_o, _ = ob.think_score_and_compact(_np(K), _np(Q), H, prune, DT[dtype])
    _same(mask.cpu().numpy(), mask_o, "keep_mask")
    _same(_np(Kc), Kc_o, "K_compact")


@pytest.mark.parametrize("case", _cases(20, 43, [1, 2, 4]), ids=lambda c: f"s{c['i']}")
def test_spark_random_shapes(case):
    from rotatek_amd.baselines import spark_prune
    c = case
    B, H, G, S, W, prune, dtype = c["B"], c["H"], c["G"], c["S"], c["W"], c["prune"], c["dtype"]
    print(f"[case] spark random {c}", flush=True)
    sys.stdout.flush()
    K = _grid((B, H, S, D), dtype, 300 + c["i"])
    Q = _grid((B, H * G, W, D), dtype, 400 + c["i"])
    Kc, mask, pm = spark_prune(K, Q, G, prune)
    torch.cuda.synchronize()
    qg = ob.group_queries(_np(Q), G, DT[dtype])
    Kc_o, mask_o, pm_o, _ = ob.per_token_channel_prune(qg, _np(K), prune, DT[dtype])
    _same(mask.cpu().numpy(), mask_o, "keep_mask")
    _same(_np(Kc), Kc_o, "K_compact")
    _same(_np(pm), pm_o, "pruned_mean")  # NaN == NaN at prune 0
