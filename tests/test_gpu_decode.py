"""GPU parity of the HIP decode kernels against the CPU oracle.

Tolerances (north star): max-abs 2e-3 for fp16 and 1e-2 for bf16 outputs
against the float64 oracle evaluated on the very same (already rounded)
inputs.  The bf16 bar is 1e-2 or the output's own rounding (2^-7 |out|),
whichever is larger; the outputs here are O(1), where the flat 1e-2 holds.
Every case prints its name before touching the GPU.
"""
import math
import sys

import numpy as np
import pytest
import torch

from oracle import decode as od

pytestmark = pytest.mark.gpu

TOL = {torch.float16: 2e-3, torch.bfloat16: 1e-2}


def _np(t):
    return None if t is None else t.detach().float().cpu().numpy().astype(np.float64)


def _say(msg):
    print(f"[case] {msg}", flush=True)
    sys.stdout.flush()


def _rand_inputs(B, Hq, Hkv, Dk, S_v, S_f, dtype, seed=0, mask_p=0.0, bias=True, view_v=True):
    g = torch.Generator(device="cuda").manual_seed(seed)
    dev = "cuda"

    def rn(*s, scale=1.0):
        return (torch.randn(*s, generator=g, device=dev) * scale).to(dtype)

    D = 128
    q = rn(B, Hq, D)
    R = torch.linalg.qr(torch.randn(B, Hkv, D, D, generator=g, device=dev))[0][..., :Dk].contiguous().to(dtype)
    dm = rn(B, Hkv, D, scale=0.5) if bias else None
    if view_v:
        V = rn(B, Hkv, S_v + S_f, D)
        vs, vf = V[:, :, :S_v], V[:, :, S_v:]
    else:
        vs, vf = rn(B, Hkv, S_v, D), rn(B, Hkv, S_f, D)
    kf = rn(B, Hkv, S_f, D)
    ks = rn(B, Hkv, S_v, Dk, scale=2.0)
    mask = (torch.rand(B, S_f, generator=g, device=dev) >= mask_p).to(torch.uint8)
    return dict(q_full=q, R_partial=R, delta_mu=dm, k_full=kf, v_full=vf, mask_full=mask,
                k_sparse=ks, v_sparse=vs, num_kv_groups=Hq // Hkv)


def _oracle(inp, heads=None):
    a = {k: (_np(v) if torch.is_tensor(v) else v) for k, v in inp.items()}
    return od.rotatek_decode(a["q_full"], a["R_partial"], a["delta_mu"], a["k_full"], a["v_full"],
                             a["mask_full"], a["k_sparse"], a["v_sparse"], a["num_kv_groups"])


def _decode(inp, family):
    from rotatek_amd.kernels.fused_decode import rotatek_decode_fused
    from rotatek_amd.kernels.gqa_decode import rotatek_decode_gqa
    fn = rotatek_decode_gqa if family == "gqa" else rotatek_decode_fused
    out, a, b = fn(**inp)
    assert a is None and b is None
    torch.cuda.synchronize()
    return out


CASES = [
    # B, Hq, Hkv, Dk, S_v, S_f
    (1, 4, 4, 32, 300, 50),
    (2, 8, 8, 32, 1000, 129),
    (2, 8, 4, 32, 517, 64),
    (1, 28, 4, 32, 2049, 100),      # G = 7
    (1, 16, 1, 32, 700, 33),        # G = 16
    (1, 40, 2, 32, 300, 20),        # G = 20 -> two head blocks
    (2, 4, 4, 16, 333, 31),
    (2, 4, 4, 64, 1025, 0),         # no prompt/text
    (2, 4, 2, 128, 640, 7),
    (2, 8, 8, 96, 700, 40),         # 65-128 kept channels: R staged whole in LDS
    (1, 28, 4, 100, 900, 33),       # ... G = 7, Dk not a multiple of 8
    (2, 4, 4, 72, 500, 9),          # ... just past 64
    (1, 4, 4, 40, 250, 17),         # Dk not a power of two
    (1, 4, 4, 8, 129, 1),
    (2, 4, 4, 32, 0, 300),          # no visual span
    (1, 2, 2, 32, 1, 1),
]


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("family", ["paper", "gqa"])
@pytest.mark.parametrize("case", CASES)
def test_rotatek_decode_matches_oracle(case, family, dtype):
    B, Hq, Hkv, Dk, S_v, S_f = case
    _say(f"rotatek {family} {dtype} B={B} Hq={Hq} Hkv={Hkv} Dk={Dk} S_v={S_v} S_f={S_f}")
    inp = _rand_inputs(B, Hq, Hkv, Dk, S_v, S_f, dtype, seed=hash(case) % 1000, mask_p=0.2)
    out = _decode(inp, family)
    assert out.shape == (B, 1, Hq, 128) and out.dtype == dtype
    want = _oracle(inp)
    err = np.abs(_np(out) - want).max()
    assert err <= TOL[dtype], err


@pytest.mark.parametrize("Dk", [48, 96])
@pytest.mark.parametrize("family", ["paper", "gqa"])
def test_rotation_in_the_other_16bit_type(Dk, family):
    """R_partial in bf16 under fp16 q/K/V (and the reverse): up to 64 kept
    channels R is staged as is, past 64 only in the compute type, so the
    element-wise R path runs there."""
    for dt, rdt in ((torch.float16, torch.bfloat16), (torch.bfloat16, torch.float16)):
        _say(f"rotatek {family} q {dt} R {rdt} Dk={Dk}")
        inp = _rand_inputs(2, 8, 4, Dk, 600, 50, dt, seed=Dk + 1)
        inp["R_partial"] = inp["R_partial"].to(rdt)
        out = _decode(inp, family)
        assert np.abs(_np(out) - _oracle(inp)).max() <= TOL[dt]


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_no_bias_contiguous_values_and_all_masked(dtype):
    _say(f"rotatek no-bias/all-masked {dtype}")
    inp = _rand_inputs(2, 8, 4, 32, 400, 60, dtype, seed=3, bias=False, view_v=False)
    inp["mask_full"][0] = 0
    out = _decode(inp, "gqa")
    assert np.abs(_np(out) - _oracle(inp)).max() <= TOL[dtype]


def test_empty_spans_give_zeros():
    _say("rotatek empty spans")
    inp = _rand_inputs(2, 4, 4, 32, 0, 0, torch.float16)
    out = _decode(inp, "paper")
    assert torch.count_nonzero(out) == 0
    inp = _rand_inputs(2, 4, 4, 32, 0, 20, torch.float16)
    inp["mask_full"].zero_()
    assert torch.count_nonzero(_decode(inp, "gqa")) == 0


def test_strided_inputs_take_the_scalar_path():
    """Non-unit channel strides (a transposed view) select the element-wise
    load variant; results must not change."""
    _say("rotatek strided inputs")
    inp = _rand_inputs(1, 4, 2, 32, 300, 40, torch.float16, seed=9)
    ref = _decode(inp, "gqa")
    ks = inp["k_sparse"]
    inp2 = dict(inp)
    inp2["k_sparse"] = ks.transpose(-1, -2).contiguous().transpose(-1, -2)   # stride_d = S_v
    assert inp2["k_sparse"].stride(-1) != 1
    out = _decode(inp2, "gqa")
    assert torch.equal(out, ref)


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_dense_decode_matches_oracle(dtype):
    from rotatek_amd.kernels.full_channel_flash_decoding import full_channel_decode
    from rotatek_amd.kernels.gqa_decode import full_channel_decode_gqa
    for (B, Hq, Hkv, S) in [(2, 8, 8, 1000), (1, 28, 4, 3001), (2, 8, 2, 64), (1, 4, 4, 1)]:
        _say(f"dense {dtype} B={B} Hq={Hq} Hkv={Hkv} S={S}")
        g = torch.Generator(device="cuda").manual_seed(S)
        q = torch.randn(B, Hq, 128, generator=g, device="cuda").to(dtype)
        k = torch.randn(B, Hkv, S, 128, generator=g, device="cuda").to(dtype)
        v = torch.randn(B, Hkv, S, 128, generator=g, device="cuda").to(dtype)
        want = od.full_channel_decode(_np(q), _np(k), _np(v), Hq // Hkv)
        for fn in (full_channel_decode, full_channel_decode_gqa):
            out = fn(q, k, v, num_kv_groups=Hq // Hkv)
            torch.cuda.synchronize()
            assert out.shape == (B, 1, Hq, 128)
            assert np.abs(_np(out) - want).max() <= TOL[dtype]


def test_rotatek_with_identity_rotation_equals_dense():
    """Dk = D, R = I, delta_mu = 0: RotateK over (visual, full) equals the
    dense kernel over the concatenated Keys (HIP vs HIP, same dtype)."""
    from rotatek_amd.kernels.gqa_decode import full_channel_decode_gqa, rotatek_decode_gqa
    _say("rotatek identity == dense")
    B, Hq, Hkv, S_v, S_f = 2, 8, 4, 900, 100
    g = torch.Generator(device="cuda").manual_seed(5)
    dt = torch.float16
    q = torch.randn(B, Hq, 128, generator=g, device="cuda").to(dt)
    K = torch.randn(B, Hkv, S_v + S_f, 128, generator=g, device="cuda").to(dt)
    V = torch.randn(B, Hkv, S_v + S_f, 128, generator=g, device="cuda").to(dt)
    R = torch.eye(128, device="cuda", dtype=dt).expand(B, Hkv, 128, 128).contiguous()
    out, _, _ = rotatek_decode_gqa(q, R, torch.zeros(B, Hkv, 128, device="cuda", dtype=dt),
                                   K[:, :, S_v:], V[:, :, S_v:], torch.ones(B, S_f, device="cuda", dtype=torch.uint8),
                                   K[:, :, :S_v], V[:, :, :S_v], Hq // Hkv)
    dense = full_channel_decode_gqa(q, K, V, Hq // Hkv)
    torch.cuda.synchronize()
    assert (out.float() - dense.float()).abs().max().item() <= 2e-3


def test_repeated_calls_are_bitwise_stable():
    """The workspace is reused uninitialised across calls and shapes: every
    call must fully overwrite what it reads back."""
    _say("repeated calls / workspace reuse")
    inp = _rand_inputs(2, 8, 4, 32, 3000, 300, torch.float16, seed=11)
    a = _decode(inp, "gqa")
    other = _rand_inputs(1, 4, 4, 64, 5000, 17, torch.float16, seed=12)
    _decode(other, "paper")
    for _ in range(3):
        assert torch.equal(_decode(inp, "gqa"), a)


def test_split_granularity_does_not_change_results_beyond_rounding():
    from rotatek_amd import _lib
    _say("split granularity sweep")
    inp = _rand_inputs(1, 8, 8, 32, 5000, 700, torch.float16, seed=12)
    want = _oracle(inp)
    try:
        for lo, hi in [(64 << 10, 64 << 10), (1 << 20, 1 << 20), (16 << 20, 16 << 20)]:
            _lib.set_decode_tuning(lo, hi, 4)
            out = _decode(inp, "paper")
            assert np.abs(_np(out) - want).max() <= 2e-3
    finally:
        _lib.set_decode_tuning(64 << 10, 512 << 10, -1)


def test_graph_capture_replays_match_eager():
    from rotatek_amd.kernels.gqa_decode import rotatek_decode_gqa
    _say("hipGraph capture")
    inp = _rand_inputs(2, 8, 4, 32, 2000, 200, torch.float16, seed=13)
    eager = rotatek_decode_gqa(**inp)[0].clone()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        for _ in range(3):
            rotatek_decode_gqa(**inp)
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        out = rotatek_decode_gqa(**inp)[0]
    for i in range(5):
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager), i
        junk = torch.randn(1000, device="cuda") * 2     # eager work between replays
        torch.cuda.synchronize()
        del junk
    # the inputs can change between replays
    inp["q_full"].mul_(-1.0)
    eager2 = rotatek_decode_gqa(**inp)[0].clone()
    graph.replay()
    torch.cuda.synchronize()
    assert torch.equal(out, eager2)


def _sample_oracle(inp, pairs):
    """Oracle on selected (b, kv) groups only (host memory stays small)."""
    G = inp["num_kv_groups"]
    res = {}
    for (b, kv) in pairs:
        sub = {}
        for k in ("R_partial", "delta_mu", "k_full", "v_full", "k_sparse", "v_sparse"):
            sub[k] = _np(inp[k][b:b + 1, kv:kv + 1])
        sub["q_full"] = _np(inp["q_full"][b:b + 1, kv * G:(kv + 1) * G])
        sub["mask_full"] = _np(inp["mask_full"][b:b + 1])
        res[(b, kv)] = od.rotatek_decode(sub["q_full"], sub["R_partial"], sub["delta_mu"], sub["k_full"],
                                         sub["v_full"], sub["mask_full"], sub["k_sparse"], sub["v_sparse"],
                                         G)[0, 0]
    return res


def _torch_fp32_reference(args, b):
    """The decode of batch row b as plain torch fp32 ops on the device
    (softmax over the visual and prompt/text logits, then P V): an
    independent reference for every (head) of a full-size shape.  [H_q, D]."""
    G = args["num_kv_groups"]
    q = args["q_full"][b].float()
    R = args["R_partial"][b].float().contiguous()
    Hkv, D = R.shape[0], q.shape[-1]
    qg = q.view(Hkv, G, D)
    scale = 1.0 / math.sqrt(D)
    s_vis = torch.matmul(torch.matmul(qg, R), args["k_sparse"][b].float().transpose(-1, -2).contiguous())
    if args["delta_mu"] is not None:
        s_vis = s_vis + (qg * args["delta_mu"][b].float()[:, None, :]).sum(-1, keepdim=True)
    s_full = torch.matmul(qg, args["k_full"][b].float().transpose(-1, -2).contiguous())
    s_full = s_full.masked_fill(args["mask_full"][b][None, None, :] == 0, float("-inf"))
    p = torch.softmax(torch.cat([s_vis * scale, s_full * scale], dim=-1), dim=-1)
    S_v = s_vis.shape[-1]
    out = torch.matmul(p[..., :S_v].contiguous(), args["v_sparse"][b].float().contiguous()) + \
        torch.matmul(p[..., S_v:].contiguous(), args["v_full"][b].float().contiguous())
    return out.reshape(Hkv * G, D)


@pytest.mark.parametrize("cfg", ["cfg1", "cfg2", "cfg3", "kp"])
def test_benchmark_configs_full_size(cfg):
    """Full BASELINE shapes (and the reference kernel harness's shape, kp):
    every output against a plain torch fp32 reference on the device, that
    reference and the HIP output on sampled (b, kv) groups against the
    oracle, and paper == gqa (bit for bit for MHA)."""
    from rotatek_amd import synth
    c = synth.CONFIGS[cfg]
    _say(f"full-size {cfg}")
    inp = synth.make_decode_inputs(c, "cuda", seed=1)
    args = synth.decode_args(inp)
    out = _decode(args, "gqa")
    assert torch.isfinite(out.float()).all()
    rng = np.random.default_rng(0)
    pairs = {(int(rng.integers(c.B)), int(rng.integers(c.H_kv))) for _ in range(6)}
    pairs |= {(0, 0), (c.B - 1, c.H_kv - 1)}
    want = _sample_oracle(args, sorted(pairs))
    G = c.G
    tf32 = torch.backends.cuda.matmul.allow_tf32
    torch.backends.cuda.matmul.allow_tf32 = False
    try:
        refs = {}
        for b in range(c.B):                     # every batch row, every head
            ref = _torch_fp32_reference(args, b)
            refs[b] = ref
            err = (out[b, 0].float() - ref).abs().max().item()
            assert err <= TOL[c.dtype], (b, err)
    finally:
        torch.backends.cuda.matmul.allow_tf32 = tf32
    for (b, kv), w in want.items():
        got = _np(out[b, 0, kv * G:(kv + 1) * G])
        assert np.abs(got - w).max() <= TOL[c.dtype], (b, kv)
        # the torch reference itself against the oracle
        assert np.abs(_np(refs[b][kv * G:(kv + 1) * G]) - w).max() <= 1e-4, (b, kv)
    out_p = _decode(args, "paper")
    if c.G == 1:
        assert torch.equal(out_p, out)
    else:
        assert (out_p.float() - out.float()).abs().max().item() <= TOL[c.dtype]


LONG_CASES = [
    # dtype, family, B, Hq, Hkv, S_v, S_f
    (torch.bfloat16, "gqa", 1, 8, 2, 4_000_003, 100_001),
    (torch.float16, "paper", 1, 4, 4, 1_000_003, 30_001),
]


@pytest.mark.parametrize("case", LONG_CASES, ids=["bf16-gqa-4M", "f16-mha-1M"])
def test_long_context(case):
    """Millions of tokens per head (a V head spans 0.5 G elements, the
    kernels' offsets are 32-bit within a head).  Needle tokens at the first
    and last rows of both spans carry large logits for one query head of
    each group, so that head's output is a mix of those four V rows and an
    offset error at the far end of a span shows at O(1); every output is
    checked against the plain torch fp32 reference on the device (relative
    to its magnitude, since the other heads average millions of rows)."""
    dtype, family, B, Hq, Hkv, S_v, S_f = case
    G, Dk = Hq // Hkv, 32
    _say(f"long context {dtype} {family} B={B} Hq={Hq} Hkv={Hkv} S_v={S_v} S_f={S_f}")
    g = torch.Generator(device="cuda").manual_seed(11)

    def rn(*shape, scale=1.0):
        return (torch.randn(*shape, generator=g, device="cuda") * scale).to(dtype)

    q = rn(B, Hq, 128)
    R = torch.linalg.qr(torch.randn(B, Hkv, 128, 128, generator=g, device="cuda"))[0][..., :Dk].contiguous()
    ks = rn(B, Hkv, S_v, Dk, scale=0.5)
    V = rn(B, Hkv, S_v + S_f, 128)
    kf = rn(B, Hkv, S_f, 128, scale=0.5)
    qh = q.float().view(B, Hkv, G, 128)[:, :, 0]                  # the first query head of each group
    qt = torch.einsum("bhd,bhdk->bhk", qh, R)
    # needle logits of 20 (e^20 outweighs millions of O(1)-logit tokens)
    for t in (0, S_v - 1):
        ks[:, :, t] = (qt * (20.0 / qt.norm(dim=-1, keepdim=True) ** 2 * 128 ** 0.5)).to(dtype)
    for t in (0, S_f - 1):
        kf[:, :, t] = (qh * (20.0 / qh.norm(dim=-1, keepdim=True) ** 2 * 128 ** 0.5)).to(dtype)
    args = dict(q_full=q, R_partial=R.to(dtype), delta_mu=rn(B, Hkv, 128, scale=0.1), k_full=kf,
                v_full=V[:, :, S_v:], mask_full=torch.ones(B, S_f, dtype=torch.uint8, device="cuda"),
                k_sparse=ks, v_sparse=V[:, :, :S_v], num_kv_groups=G)
    out = _decode(args, family)
    assert torch.isfinite(out.float()).all()
    tf32 = torch.backends.cuda.matmul.allow_tf32
    torch.backends.cuda.matmul.allow_tf32 = False
    try:
        for b in range(B):
            ref = _torch_fp32_reference(args, b)
            got = out[b, 0].float()
            scale = ref.abs().amax(dim=-1, keepdim=True)
            err = ((got - ref).abs() / scale).max().item()
            assert err <= 2e-2, (b, err)
            # the needle heads: a mix of the four needle rows, O(1)
            assert scale.view(Hkv, G)[:, 0].min().item() > 0.3, scale.view(Hkv, G)[:, 0]
    finally:
        torch.backends.cuda.matmul.allow_tf32 = tf32


# ---------------------------------------------------------------- fp32
# The reference kernels load any float input as fp32 and compute in fp32
# (fused_decode.py:133,166,174; full_channel_flash_decoding.py:65,84,92);
# the HIP fp32 path does the same on the VALU.  Bar: max-abs 1e-4 against
# the float64 oracle on the same fp32 inputs (outputs are O(0.1); a dropped
# bias or a wrong scale is off by 1e-2 or more).
TOL32 = 1e-4

FP32_CASES = [
    # B, Hq, Hkv, Dk, S_v, S_f
    (1, 32, 32, 32, 2304, 128),     # config 0
    (2, 8, 2, 32, 1000, 77),        # GQA
    (1, 4, 4, 40, 300, 0),          # no prompt/text, Dk % 8 != 0
    (2, 4, 4, 32, 0, 257),          # no visual span
    (1, 28, 4, 128, 513, 65),
    (1, 2, 2, 6, 5, 3),             # Dk not a multiple of 4 (element loads)
    (1, 24, 2, 32, 700, 40),        # G = 12: head blocks of 8 and 4 query heads
    (2, 16, 1, 64, 400, 30),        # G = 16: two blocks of 8
]


@pytest.mark.parametrize("family", ["paper", "gqa"])
@pytest.mark.parametrize("case", FP32_CASES)
def test_fp32_decode_matches_oracle(case, family):
    B, Hq, Hkv, Dk, S_v, S_f = case
    _say(f"rotatek fp32 {family} B={B} Hq={Hq} Hkv={Hkv} Dk={Dk} S_v={S_v} S_f={S_f}")
    inp = _rand_inputs(B, Hq, Hkv, Dk, S_v, S_f, torch.float32, seed=sum(case), mask_p=0.2)
    out = _decode(inp, family)
    assert out.dtype == torch.float32 and out.shape == (B, 1, Hq, 128)
    err = np.abs(_np(out) - _oracle(inp)).max()
    assert err <= TOL32, err


@pytest.mark.parametrize("case", [(2, 28, 4, 32, 1500, 61), (1, 24, 2, 64, 900, 33)])
def test_fp32_grouped_merges_are_bit_identical(case):
    """fp32 units of up to 8 query heads of one KV head (each K / V row
    read once for the unit's heads): the single-launch merge equals the
    merge kernel bit for bit, and both match the oracle."""
    from rotatek_amd import _lib
    B, Hq, Hkv, Dk, S_v, S_f = case
    _say(f"fp32 grouped merges B={B} Hq={Hq} Hkv={Hkv} Dk={Dk}")
    p = _lib.plan_decode(B, Hq, Hkv, Dk, S_v, S_f, 4, _lib.RK_POLICY_GQA)
    assert p["heads_per_unit"] == min(Hq // Hkv, 8) and p["units"] == B * Hkv * -(-(Hq // Hkv) // 8)
    inp = _rand_inputs(B, Hq, Hkv, Dk, S_v, S_f, torch.float32, seed=sum(case), mask_p=0.2)
    try:
        _lib.set_decode_merge(_lib.MERGE_TWO_LAUNCHES)
        two = _decode(inp, "gqa")
        _lib.set_decode_merge(_lib.MERGE_SINGLE_LAUNCH)
        one = _decode(inp, "gqa")
    finally:
        _lib.set_decode_merge(_lib.MERGE_AUTO)
    assert torch.equal(one, two)
    assert np.abs(_np(two) - _oracle(inp)).max() <= TOL32


def test_fp32_config0_end_to_end():
    """BASELINE config 0 (B=1, 32 heads, 2304 visual + 128 text tokens, fp32,
    seeded orthogonal R_k, top 32 channels by mean |K R_k|): the kept channels,
    selected by the HIP prefill kernels at fp32 (synth's default for fp32:
    channel scores, top-k, gather, truncated write), and the decode against
    the oracle."""
    from rotatek_amd import synth
    from rotatek_amd.kernels.fused_decode import rotatek_decode_fused
    from oracle import prefill as op
    cfg = synth.CONFIGS["cfg0"]
    _say("config 0 fp32 end to end")
    inp = synth.make_decode_inputs(cfg, "cuda", seed=0, with_raw=True)
    # selection rule: the kept indices are the oracle's top 32 of mean |K R_k|
    # on every head whose 32nd and 33rd scores are apart by more than the
    # fp32 scoring error (a closer boundary may go either way)
    Rk = synth.random_rotations(cfg.B, cfg.H_kv, cfg.D, 2).numpy().astype(np.float32).astype(np.float64)
    scores = np.abs(_np(inp["k_vis_raw"]) @ Rk).mean(axis=-2)
    idx_o, _ = op.topk_channels(scores, cfg.keep)
    top = -np.sort(-scores, axis=-1)
    clear = (top[..., cfg.keep - 1] - top[..., cfg.keep]) > 1e-4 * top[..., cfg.keep - 1]
    assert clear.sum() >= cfg.H_kv // 2
    assert np.array_equal(inp["keep_idx"].cpu().numpy()[clear], idx_o[clear])
    args = synth.decode_args(inp)
    out, _, _ = rotatek_decode_fused(**args)
    torch.cuda.synchronize()
    want = _oracle(dict(args))
    err = np.abs(_np(out) - want).max()
    assert err <= TOL32, err


def test_fp32_strided_and_bf16_rotation():
    _say("rotatek fp32 strided views, bf16 R and delta_mu")
    inp = _rand_inputs(2, 8, 4, 32, 700, 90, torch.float32, seed=9, view_v=False)
    inp["R_partial"] = inp["R_partial"].to(torch.bfloat16)
    inp["delta_mu"] = inp["delta_mu"].to(torch.bfloat16)
    big = torch.randn(2, 4, 700, 48, device="cuda")
    big[..., :32] = inp["k_sparse"]
    inp["k_sparse"] = big[..., :32]            # row stride 48: element loads
    out = _decode(inp, "gqa")
    assert np.abs(_np(out) - _oracle(inp)).max() <= TOL32


@pytest.mark.parametrize("G", [1, 4])
def test_fp32_dense_matches_oracle(G):
    from rotatek_amd.kernels.full_channel_flash_decoding import full_channel_decode
    _say(f"dense fp32 G={G}")
    g = torch.Generator(device="cuda").manual_seed(G)
    q = torch.randn(2, 8, 128, generator=g, device="cuda")
    k = torch.randn(2, 8 // G, 1500, 128, generator=g, device="cuda")
    v = torch.randn(2, 8 // G, 1500, 128, generator=g, device="cuda")
    out = full_channel_decode(q, k, v, num_kv_groups=G)
    torch.cuda.synchronize()
    want = od.full_channel_decode(_np(q), _np(k), _np(v), G)
    assert out.dtype == torch.float32
    assert np.abs(_np(out) - want).max() <= TOL32


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("family", ["paper", "gqa"])
def test_zero_kept_channels(dtype, family):
    """channel_ratio >= 1 keeps no channel: R_partial [B,H,D,0], k_sparse
    [B,H,S_v,0] (no storage), delta_mu = the Key mean.  Visual logits are the
    bias q . delta_mu alone, as in the reference's kernels."""
    _say(f"rotatek Dk=0 {family} {dtype}")
    inp = _rand_inputs(2, 8, 4, 32, 500, 40, dtype, seed=13)
    inp["R_partial"] = inp["R_partial"][..., :0]
    inp["k_sparse"] = torch.empty(2, 4, 500, 0, device="cuda", dtype=dtype)
    out = _decode(inp, family)
    want = _oracle(inp)
    assert np.abs(_np(out) - want).max() <= (TOL32 if dtype == torch.float32 else TOL[dtype])


def test_pruner_ratio_one_decodes():
    """ChannelPruner with channel_ratio 1.0 (keep 0) feeds the decode."""
    from rotatek_amd.kernels.gqa_decode import rotatek_decode_gqa
    from rotatek_amd.pruning import ChannelPruner
    _say("pruner ratio 1.0 -> decode")
    g = torch.Generator(device="cuda").manual_seed(2)
    B, H, G, S = 1, 2, 4, 300
    K = torch.randn(B, H, S, 128, generator=g, device="cuda").to(torch.bfloat16)
    Q = torch.randn(B, H * G, S, 128, generator=g, device="cuda").to(torch.bfloat16)
    V = torch.randn(B, H, S, 128, generator=g, device="cuda").to(torch.bfloat16)
    pr = ChannelPruner(1.0, 10, 20, solver="power_iter", query_aware=True)
    kept, kp, kt, mask, v = pr.update_rotatek(K, Q, V, None, G)
    assert kept.shape[-1] == 0 and pr.current_rotatek_R_partial.shape[-1] == 0
    q = torch.randn(B, H * G, 128, generator=g, device="cuda").to(torch.bfloat16)
    kf, vf = torch.cat([kp, kt], -2), torch.cat([V[:, :, :10], V[:, :, -20:]], -2)
    mask_full = torch.ones(B, 30, dtype=torch.uint8, device="cuda")
    args = dict(q_full=q, R_partial=pr.current_rotatek_R_partial, delta_mu=pr.current_rotatek_delta_mu,
                k_full=kf, v_full=vf, mask_full=mask_full, k_sparse=kept, v_sparse=V[:, :, 10:-20],
                num_kv_groups=G)
    out, _, _ = rotatek_decode_gqa(**args)
    torch.cuda.synchronize()
    assert np.abs(_np(out) - _oracle(args)).max() <= TOL[torch.bfloat16]


@pytest.mark.parametrize("dtype", [torch.float16, torch.float32])
@pytest.mark.parametrize("family", ["paper", "gqa"])
def test_more_units_than_the_reported_grid_y(dtype, family):
    """66560 work units (B=2080, 32 MHA heads): the unit-major grid puts the
    unit in blockIdx.y, past the 65536 that hipDeviceProp_t.maxGridSize[1]
    reports (the dispatch packet's 32-bit grid size takes it; the reference
    launches B * H programs along its first grid axis).  Sampled batch rows,
    the last one included, against the oracle on their own slices."""
    B, H, Dk, S_v, S_f = 2080, 32, 8, 40, 8
    _say(f"66560 units {family} {dtype}")
    g = torch.Generator(device="cuda").manual_seed(66560)

    def rn(*s, scale=1.0):
        return (torch.randn(*s, generator=g, device="cuda") * scale).to(dtype)

    # one orthogonal basis for every head (a batched QR of 66560 matrices
    # would dominate the test)
    R1 = torch.linalg.qr(torch.randn(128, 128, generator=g, device="cuda"))[0][:, :Dk]
    R = R1.to(dtype).expand(B, H, 128, Dk).contiguous()
    V = rn(B, H, S_v + S_f, 128)
    inp = dict(q_full=rn(B, H, 128), R_partial=R, delta_mu=rn(B, H, 128, scale=0.5), k_full=rn(B, H, S_f, 128),
               v_full=V[:, :, S_v:], mask_full=torch.ones(B, S_f, dtype=torch.uint8, device="cuda"),
               k_sparse=rn(B, H, S_v, Dk, scale=2.0), v_sparse=V[:, :, :S_v], num_kv_groups=1)
    from rotatek_amd import _lib
    p = _lib.plan_decode(B, H, H, Dk, S_v, S_f, torch.tensor([], dtype=dtype).element_size(),
                         _lib.RK_POLICY_GQA if family == "gqa" else _lib.RK_POLICY_PAPER)
    assert p["units"] == B * H > 65536
    out = _decode(inp, family)
    assert torch.isfinite(out.float()).all()
    for b in (0, 1037, B - 1):
        sl = {k: (v[b:b + 1] if torch.is_tensor(v) else v) for k, v in inp.items()}
        err = np.abs(_np(out[b:b + 1]) - _oracle(sl)).max()
        assert err <= (TOL32 if dtype == torch.float32 else TOL[dtype]), (b, err)


@pytest.mark.parametrize("family", ["paper", "gqa"])
def test_fp16_queries_past_the_split_range(family):
    """fp16 queries of order 3e4: entries of q R reach ~1e5, past fp16's
    65504, where a plain fp16 hi + lo split would overflow to inf.  The
    reference's paper kernel forms q R and the scores in fp32
    (fused_decode.py:133-139, 166-167); the kernel scales q R by a power of
    two before the split and the score multiplier back, so the output
    matches the float64 oracle (softmax over scores of order 1e5: nearly one
    row).  The scaling is exact and off (factor 1) below 2^15."""
    B, Hq, Hkv, Dk, S_v, S_f = 2, 8, 4, 32, 300, 40
    _say(f"fp16 q past the split range {family}")
    inp = _rand_inputs(B, Hq, Hkv, Dk, S_v, S_f, torch.float16, seed=30000)
    g = torch.Generator(device="cuda").manual_seed(30001)
    q = (torch.randn(B, Hq, 128, generator=g, device="cuda") * 3e4).clamp(-6e4, 6e4)
    inp["q_full"] = q.to(torch.float16)
    qr = torch.einsum("bhd,bhdk->bhk", inp["q_full"].float(),
                      inp["R_partial"].float().repeat_interleave(Hq // Hkv, dim=1))
    assert qr.abs().max().item() > 65504  # the case the split must survive
    out = _decode(inp, family)
    assert torch.isfinite(out.float()).all()
    assert np.abs(_np(out) - _oracle(inp)).max() <= TOL[torch.float16]
