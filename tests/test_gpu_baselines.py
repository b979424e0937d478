"""GPU parity of the ThinK / SparK baseline kernels (rotatek_amd.baselines)
against the CPU oracle (oracle/baselines.py) and against torch's own GPU ops.

Bars: on grid inputs (values m/8, where every square and sum is exact in
fp32) masks, compact Keys and pruned means are bit-exact, against the oracle
and against the reference's torch op chain run on the GPU (which pins the
tie rules and the mean factor of torch's GPU kernels); on random inputs the
selection agrees with the oracle's scores up to one storage ulp and the
compact Keys / pruned means are exact for the selection made; the recovery is
bit-exact; decode over recovered Keys is within the decode tolerance
(2e-3 fp16 / 1e-2 bf16 max-abs) of the oracle.
"""
import sys

import numpy as np
import pytest
import torch

from oracle import baselines as ob
from oracle import decode as od
from oracle.numerics import round_to

pytestmark = pytest.mark.gpu

D = 128
DT = {torch.float16: "float16", torch.bfloat16: "bfloat16"}
ULP = {torch.float16: 2.0 ** -10, torch.bfloat16: 2.0 ** -7}
TOL = {torch.float16: 2e-3, torch.bfloat16: 1e-2}


def _say(msg):
    print(f"[case] {msg}", flush=True)
    sys.stdout.flush()


def _np(t):
    return t.detach().cpu().to(torch.float64).numpy()


def _grid(shape, dtype, seed):
    g = torch.Generator().manual_seed(seed)
    return (torch.randint(-15, 16, shape, generator=g).to(torch.float32) / 8).to(dtype).cuda()


def _rand(shape, dtype, seed, outliers=True):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(shape, generator=g)
    if outliers:
        x[..., ::9] *= 6.0
    return x.to(dtype).cuda()


def _assert_same(a, b, what):
    a, b = np.asarray(a, np.float64), np.asarray(b, np.float64)
    assert a.shape == b.shape, (what, a.shape, b.shape)
    np.testing.assert_array_equal(a, b, err_msg=what)


def _selection_consistent(mask, scores, ulp: float):
    """Every kept score >= every pruned score, up to one ulp of the scores."""
    s = np.where(np.isnan(scores), np.inf, scores)
    m = mask.astype(bool)
    kept_min = np.where(m, s, np.inf).min(axis=-1)
    pruned_max = np.where(~m, s, -np.inf).max(axis=-1)
    slack = ulp * np.maximum(np.abs(kept_min), np.abs(pruned_max))
    slack = np.where(np.isfinite(slack), slack, 0.0)
    assert np.all(pruned_max <= kept_min + slack)


# ------------------------------------------------------------------ ThinK
THINK_SHAPES = [(2, 4, 7, 1000, 32), (1, 2, 1, 1, 5), (3, 1, 4, 4097, 32), (2, 2, 2, 0, 32)]


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("shape", THINK_SHAPES)
@pytest.mark.parametrize("prune", [0, 64, 96, 128])
def test_think_grid_matches_oracle(dtype, shape, prune):
    from rotatek_amd.baselines import think_score_and_compact
    B, H, G, S, W = shape
    _say(f"think grid {dtype} shape={shape} prune={prune}")
    K = _grid((B, H, S, D), dtype, 1)
    Q = _grid((B, H * G, W, D), dtype, 2)
    Kc, mask = think_score_and_compact(K, Q, H, prune)
    torch.cuda.synchronize()
    Kc_o, mask_o, _ = ob.think_score_and_compact(_np(K), _np(Q), H, prune, DT[dtype])
    _assert_same(mask.cpu().numpy(), mask_o, "keep_mask")
    _assert_same(_np(Kc), Kc_o, "K_compact")


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("layout", ["slice", "strided"])
def test_think_random_and_views(dtype, layout):
    """Random Keys read through a token slice (16-byte path) or a channel
    stride of 2 (element path): the selection matches the oracle's scores and
    the compact Keys are the kept channels."""
    from rotatek_amd.baselines import think_score_and_compact
    B, H, G, S, W, prune = 2, 4, 7, 3000, 32, 96
    _say(f"think random {dtype} {layout}")
    if layout == "slice":
        big = _rand((B, H, S + 10, D), dtype, 3)
        K = big[:, :, 5:5 + S]
    else:
        big = _rand((B, H, S, 2 * D), dtype, 3)
        K = big[..., ::2]
    Q = _rand((B, H * G, W, D), dtype, 4)
    Kc, mask = think_score_and_compact(K, Q, H, prune)
    Kc2, mask2 = think_score_and_compact(K.contiguous(), Q, H, prune)
    torch.cuda.synchronize()
    assert torch.equal(mask, mask2) and torch.equal(Kc, Kc2)
    Kn, m = _np(K), mask.cpu().numpy()
    _, _, scores = ob.think_score_and_compact(Kn, _np(Q), H, prune, DT[dtype])
    assert (m.sum(-1) == D - prune).all()
    _selection_consistent(m, scores, ULP[dtype])
    for b in range(B):
        for h in range(H):
            _assert_same(_np(Kc[b, h]), Kn[b, h][:, m[b, h]], f"compact {b},{h}")


# ------------------------------------------------------------------ SparK
SPARK_SHAPES = [(2, 4, 1, 700, 32), (1, 2, 2, 1, 3), (2, 1, 4, 2049, 32), (1, 2, 2, 0, 8)]


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("shape", SPARK_SHAPES)
@pytest.mark.parametrize("prune", [0, 32, 96, 127, 128])
def test_spark_grid_matches_oracle(dtype, shape, prune):
    from rotatek_amd.baselines import spark_prune
    B, H, G, S, W = shape
    _say(f"spark grid {dtype} shape={shape} prune={prune}")
    K = _grid((B, H, S, D), dtype, 5)
    Q = _grid((B, H * G, W, D), dtype, 6)
    Kc, mask, pm = spark_prune(K, Q, G, prune)
    torch.cuda.synchronize()
    qg = ob.group_queries(_np(Q), G, DT[dtype])
    Kc_o, mask_o, pm_o, _ = ob.per_token_channel_prune(qg, _np(K), prune, DT[dtype])
    _assert_same(mask.cpu().numpy(), mask_o, "keep_mask")
    _assert_same(_np(Kc), Kc_o, "K_compact")
    _assert_same(_np(pm), pm_o, "pruned_mean")       # NaN == NaN for prune 0


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("layout", ["contiguous", "strided"])
def test_spark_random_and_views(dtype, layout):
    from rotatek_amd.baselines import spark_prune
    B, H, G, S, W, prune = 2, 4, 7, 1500, 32, 96
    _say(f"spark random {dtype} {layout}")
    if layout == "contiguous":
        K = _rand((B, H, S, D), dtype, 7)
    else:
        K = _rand((B, H, S, 2 * D), dtype, 7)[..., 1::2]
    Q = _rand((B, H * G, W, D), dtype, 8)
    Kc, mask, pm = spark_prune(K, Q, G, prune)
    torch.cuda.synchronize()
    Kn, m = _np(K), mask.cpu().numpy()
    qg = ob.group_queries(_np(Q), G, DT[dtype])
    _, _, _, scores = ob.per_token_channel_prune(qg, Kn, prune, DT[dtype])
    assert (m.sum(-1) == D - prune).all()
    _selection_consistent(m, scores, 2 * ULP[dtype])
    _assert_same(_np(Kc), Kn[m].reshape(B, H, S, D - prune), "K_compact")
    want = round_to(np.where(~m, Kn, 0).sum(-1) / prune, DT[dtype])[..., None]
    err = np.abs(_np(pm) - want)
    assert np.all(err <= ULP[dtype] * np.maximum(np.abs(want), 1e-30)), err.max()


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("prune", [32, 96, 127])
def test_spark_nonfinite_matches_oracle(dtype, prune):
    """Keys holding NaN, +-inf and -0 and a query channel of zeros (so
    inf * 0 scores NaN): NaN scores rank above +inf and equal one another
    (lowest channel first), +inf above every finite score, -0 with +0; the
    pruned mean carries NaN / inf as torch's does."""
    from rotatek_amd.baselines import spark_prune
    B, H, G, S, W = 2, 2, 2, 333, 16
    _say(f"spark non-finite {dtype} prune={prune}")
    K = _grid((B, H, S, D), dtype, 21).float()
    g = torch.Generator().manual_seed(22)
    for val in (float("nan"), float("inf"), float("-inf"), -0.0):
        tok = torch.randint(0, S, (40,), generator=g)
        ch = torch.randint(0, D, (40,), generator=g)
        K[0, :, tok, ch] = val
        K[1, 1, tok[:10], ch[:10]] = val
    K[1, 0, 7, :40] = float("nan")          # a token with more NaN scores than some keeps
    K[1, 0, 9, ::2] = float("inf")
    K = K.to(dtype)
    Q = _grid((B, H * G, W, D), dtype, 23).float()
    Q[0, :G, :, 5] = 0.0                    # head 0 of batch 0: q_norm 0 on channel 5
    Q = Q.to(dtype)
    Kc, mask, pm = spark_prune(K, Q, G, prune)
    torch.cuda.synchronize()
    qg = ob.group_queries(_np(Q), G, DT[dtype])
    Kc_o, mask_o, pm_o, _ = ob.per_token_channel_prune(qg, _np(K), prune, DT[dtype])
    _assert_same(mask.cpu().numpy(), mask_o, "keep_mask")
    _assert_same(_np(Kc), Kc_o, "K_compact")
    _assert_same(_np(pm), pm_o, "pruned_mean")


# --------------------------------------------------- torch's GPU semantics
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_think_and_spark_equal_torch_gpu_op_chain(dtype):
    """The reference's op chains (think.py:37-58, spark.py:37-60 with the
    group mean of kv_pruning_utils.py:76-79) run with torch's GPU kernels on
    grid inputs, where every sum is exact: torch's topk / argsort tie order
    and its 16-bit mean factor decide the result, and the HIP kernels must
    reproduce it bit for bit."""
    from rotatek_amd.baselines import spark_prune, think_score_and_compact
    _say(f"torch gpu op chain {dtype}")
    B, H, S, W = 2, 4, 900, 32
    K = _grid((B, H, S, D), dtype, 9)
    Q7 = _grid((B, H * 7, W, D), dtype, 10)     # ThinK: the 1/7 group factor is applied to exact sums
    Q4 = _grid((B, H * 4, W, D), dtype, 11)     # SparK: q_norm sums stay exact with a power-of-two group
    for prune in (64, 96):
        keep = D - prune
        G, Q = 7, Q7
        qn = torch.pow(Q, 2).mean(dim=2).view(B, H, G, D).mean(dim=2)
        kn = torch.pow(K, 2).mean(dim=2)
        pruned_idx = torch.topk(qn * kn, prune, dim=-1, largest=False, sorted=False).indices
        pm_t = torch.zeros(B, H, D, dtype=torch.bool, device="cuda")
        pm_t.scatter_(-1, pruned_idx, True)
        keep_t = ~pm_t
        Kc, mask = think_score_and_compact(K, Q, H, prune)
        assert torch.equal(mask, keep_t), "ThinK mask differs from torch.topk's choice"
        idx = torch.topk(keep_t.int(), keep, dim=-1, largest=True, sorted=True).indices.sort(dim=-1).values
        assert torch.equal(Kc, torch.gather(K, -1, idx.unsqueeze(2).expand(-1, -1, S, -1)))

        G, Q = 4, Q4
        qg = Q.view(B, H, G, W, D).mean(2)
        qnorm = torch.norm(qg, dim=-2, p=2).unsqueeze(-2)
        order = torch.argsort(torch.pow(K, 2) * qnorm, dim=-1, descending=True)
        kept = order[..., :keep].sort(dim=-1).values
        mask_t = torch.zeros_like(K, dtype=torch.bool).scatter_(-1, kept, True)
        mean_t = torch.gather(K, -1, order[..., keep:]).mean(dim=-1, keepdim=True)
        Kc2, mask2, pm2 = spark_prune(K, Q, G, prune)
        assert torch.equal(mask2, mask_t), "SparK mask differs from torch.argsort's order"
        assert torch.equal(Kc2, torch.gather(K, -1, kept))
        assert torch.equal(pm2, mean_t)


# --------------------------------------------------------------- recovery
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("spans", [(0, 0), (7, 3)])
@pytest.mark.parametrize("out_layout", ["fresh", "slice", "strided"])
def test_recover_matches_oracle(dtype, spans, out_layout):
    from rotatek_amd.baselines import recover_spark, recover_think, spark_prune, think_score_and_compact
    s_p, s_t = spans
    B, H, G, S, W = 2, 4, 2, 1200, 16
    _say(f"recover {dtype} spans={spans} out={out_layout}")
    K = _rand((B, H, S, D), dtype, 11)
    Q = _rand((B, H * G, W, D), dtype, 12)
    P = _rand((B, H, s_p, D), dtype, 13) if s_p else None
    T = _rand((B, H, s_t, D), dtype, 14) if s_t else None
    rows = s_p + S + s_t

    def out_buf():
        if out_layout == "fresh":
            return None
        if out_layout == "slice":
            return torch.full((B, H, rows + 9, D), 7.0, dtype=dtype, device="cuda")[:, :, 4:4 + rows]
        return torch.full((B, H, rows, 2 * D), 7.0, dtype=dtype, device="cuda")[..., ::2]

    Kc, tm = think_score_and_compact(K, Q, H, 100)
    Rt = recover_think(Kc, tm, out=out_buf(), k_prompt=P, k_text=T)
    Kc2, sm, pm = spark_prune(K, Q, G, 90)
    Rs = recover_spark(Kc2, sm, pm, out=out_buf(), k_prompt=P, k_text=T)
    torch.cuda.synchronize()
    Pn = _np(P) if s_p else np.zeros((B, H, 0, D))
    Tn = _np(T) if s_t else np.zeros((B, H, 0, D))
    _assert_same(_np(Rt), ob.assemble(Pn, ob.recover_think(_np(Kc), tm.cpu().numpy()), Tn), "think")
    _assert_same(_np(Rs), ob.assemble(Pn, ob.recover_spark(_np(Kc2), sm.cpu().numpy(), _np(pm)), Tn), "spark")


def test_selection_rotation_is_one_hot_of_the_mask():
    from rotatek_amd.baselines import selection_rotation, think_score_and_compact
    _say("selection rotation")
    B, H = 2, 4
    K = _rand((B, H, 300, D), torch.bfloat16, 15)
    Q = _rand((B, 2 * H, 8, D), torch.bfloat16, 16)
    _, mask = think_score_and_compact(K, Q, H, 100)
    for dt in (torch.bfloat16, torch.float16, torch.float32):
        R = selection_rotation(mask, 28, dt)
        torch.cuda.synchronize()
        m = mask.cpu().numpy()
        want = np.zeros((B, H, D, 28))
        for b in range(B):
            for h in range(H):
                for j, c in enumerate(np.flatnonzero(m[b, h])):
                    want[b, h, c, j] = 1.0
        _assert_same(_np(R), want, f"R {dt}")


# ---------------------------------------------------------- pruner + cache
def _model_states(B, H, G, s_p, s_v, s_t, dtype, seed, make=_rand):
    """(Keys with outlier channels, queries, unit-scale Values): the decode
    bars are absolute, so the Values (and hence the outputs) stay O(1)."""
    S = s_p + s_v + s_t
    if make is _rand:
        return (_rand((B, H, S, D), dtype, seed), _rand((B, H * G, S, D), dtype, seed + 1, outliers=False),
                _rand((B, H, S, D), dtype, seed + 2, outliers=False))
    return (make((B, H, S, D), dtype, seed), make((B, H * G, S, D), dtype, seed + 1),
            make((B, H, S, D), dtype, seed + 2))


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_pruner_update_think_and_spark(dtype):
    """ChannelPruner.update_think / update_spark (kv_pruning_utils.py:44-90):
    spans, the 32-query window, the ratio and the returned tuple as the
    reference, bit-exact against the oracle on grid inputs."""
    from rotatek_amd.pruning import ChannelPruner
    B, H, G, s_p, s_v, s_t = 2, 4, 4, 9, 800, 40
    _say(f"pruner think/spark {dtype}")
    k, q, v = _model_states(B, H, G, s_p, s_v, s_t, dtype, 20, make=_grid)
    pr = ChannelPruner(ratio=0.75, prompt_seqlen=s_p, query_seqlen=s_t)
    Kc, kp, kt, mask, vv = pr.update_think(k, q, v, None, G)
    torch.cuda.synchronize()
    assert kp.shape[2] == s_p and kt.shape[2] == s_t and vv is v
    assert pr.current_think_mask is mask
    Kc_o, mask_o, _ = ob.think_score_and_compact(_np(k[:, :, s_p:s_p + s_v]), _np(q[:, :, -32:]), H, 96,
                                                DT[dtype])
    _assert_same(mask.cpu().numpy(), mask_o, "think mask")
    _assert_same(_np(Kc), Kc_o, "think K_compact")
    Kc, kp, kt, dummy, vv = pr.update_spark(k, q, v, None, G)
    torch.cuda.synchronize()
    assert bool(dummy.all()) and dummy.shape == (B, H, D)
    qg = ob.group_queries(_np(q[:, :, -32:]), G, DT[dtype])
    Kc_o, mask_o, pm_o, _ = ob.per_token_channel_prune(qg, _np(k[:, :, s_p:s_p + s_v]), 96, DT[dtype])
    _assert_same(pr.current_spark_mask.cpu().numpy(), mask_o, "spark mask")
    _assert_same(_np(Kc), Kc_o, "spark K_compact")
    _assert_same(_np(pr.current_spark_pruned_mean), pm_o, "spark pruned mean")


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("method", ["think", "spark"])
def test_cache_decode_over_recovered_keys(dtype, method):
    """DynamicCache.decode_recovered (recover + cat + dense decode, as the
    adapters' decode branch) and, for ThinK, decode_think_fused, against the
    oracle's dense decode over the oracle-assembled Keys, over several
    appended decode tokens."""
    from rotatek_amd.cache import DynamicCache
    from rotatek_amd.pruning import ChannelPruner
    B, H, G, s_p, s_v, s_t = 2, 4, 7, 12, 1500, 20
    _say(f"cache decode recovered {method} {dtype}")
    k, q, v = _model_states(B, H, G, s_p, s_v, s_t, dtype, 30)
    pr = ChannelPruner(ratio=0.75, prompt_seqlen=s_p, query_seqlen=s_t)
    cache = DynamicCache(reserve_tokens=8)
    out = (pr.update_think if method == "think" else pr.update_spark)(k, q, v, None, G)
    cache.store_pruned(*out, 0)
    if method == "think":
        cache.think_mask.append(pr.current_think_mask)
    else:
        cache.spark_mask.append(pr.current_spark_mask)
        cache.spark_pruned_mean.append(pr.current_spark_pruned_mean)
    Kc = out[0]
    for step in range(3):
        kn, vn = _rand((B, H, 1, D), dtype, 40 + step), _rand((B, H, 1, D), dtype, 50 + step, outliers=False)
        cache.update(kn, vn, 0)
        qd = _rand((B, H * G, D), dtype, 60 + step, outliers=False)
        got = cache.decode_recovered(qd, 0, G)
        torch.cuda.synchronize()
        if method == "think":
            rec = ob.recover_think(_np(Kc), pr.current_think_mask.cpu().numpy())
        else:
            rec = ob.recover_spark(_np(Kc), pr.current_spark_mask.cpu().numpy(),
                                   _np(pr.current_spark_pruned_mean))
        keys = ob.assemble(_np(cache.key_cache_prompt[0]), rec, _np(cache.key_cache_text[0]))
        want = od.full_channel_decode(_np(qd), keys, _np(cache.value_cache[0]), G)
        err = np.abs(_np(got) - want).max()
        assert err <= TOL[dtype], (step, err)
        if method == "think":
            for policy in (0, 1):  # paper, gqa
                fused, _, _ = cache.decode_think_fused(qd, 0, G, policy=policy)
                torch.cuda.synchronize()
                err = np.abs(_np(fused) - want).max()
                assert err <= TOL[dtype], ("fused", policy, step, err)
