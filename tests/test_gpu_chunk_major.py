"""GPU checks of the decode planner's launch layouts for one round of short
workgroups: chunk-major workgroup ids (all chunks of a unit on one XCD),
32-token visual chunks, the enlarged first-dispatched chunks where
workgroups stream <= 128 KB at two workgroups per CU, and one workgroup per
CU where that is still one round.

Each shape runs under four planner settings (unit-major; chunk-major with
equal chunks and with enlarged first chunks, both at two workgroups per CU;
the default) and every output is checked against the float64 oracle (on
sampled (b, kv) groups at full size) at the north-star bars; the layouts
differ only in where chunk boundaries fall, so the outputs also agree with
each other within those bars.  The plan fields are asserted, so each case
provably runs the layout it names.
"""
import sys

import numpy as np
import pytest
import torch

from oracle import decode as od
from rotatek_amd import _lib

pytestmark = pytest.mark.gpu

TOL = {torch.float16: 2e-3, torch.bfloat16: 1e-2}
# (skew permille, workgroups per CU; -1 = the default choice)
MODES = {"unit_major": (0, -1), "chunk_major": (1000, 2), "skewed": (1300, 2), "default": (1300, -1)}


def _set_mode(name):
    skew, wgs = MODES[name]
    _lib.set_decode_skew(skew)
    _lib.set_decode_tuning(0, 0, wgs)


def _say(msg):
    print(f"[case] {msg}", flush=True)
    sys.stdout.flush()


def _np(t):
    return t.detach().float().cpu().numpy().astype(np.float64)


@pytest.fixture(autouse=True)
def _restore_planner():
    yield
    _set_mode("default")


def _inputs(B, Hq, Hkv, Dk, S_v, S_f, dtype, seed):
    g = torch.Generator(device="cuda").manual_seed(seed)

    def rn(*s, scale=1.0):
        return (torch.randn(*s, generator=g, device="cuda") * scale).to(dtype)

    R = torch.linalg.qr(torch.randn(B, Hkv, 128, 128, generator=g, device="cuda"))[0][..., :Dk]
    V = rn(B, Hkv, S_v + S_f, 128)
    return dict(q_full=rn(B, Hq, 128), R_partial=R.contiguous().to(dtype), delta_mu=rn(B, Hkv, 128, scale=0.5),
                k_full=rn(B, Hkv, S_f, 128), v_full=V[:, :, S_v:],
                mask_full=(torch.rand(B, S_f, generator=g, device="cuda") >= 0.1).to(torch.uint8),
                k_sparse=rn(B, Hkv, S_v, Dk, scale=2.0), v_sparse=V[:, :, :S_v], num_kv_groups=Hq // Hkv)


def _oracle_groups(inp, groups):
    G = inp["num_kv_groups"]
    out = {}
    for b, kv in groups:
        sl = slice(kv * G, (kv + 1) * G)
        a = {k: (_np(v[b:b + 1, kv:kv + 1]) if torch.is_tensor(v) and v.dim() == 4 else v) for k, v in inp.items()}
        want = od.rotatek_decode(_np(inp["q_full"][b:b + 1, sl]), a["R_partial"], _np(inp["delta_mu"][b:b + 1, kv:kv + 1]),
                                 a["k_full"], a["v_full"], _np(inp["mask_full"][b:b + 1]), a["k_sparse"],
                                 a["v_sparse"], G)
        out[(b, kv)] = want[0, 0]  # [G, D]
    return out


CASES = [
    # B, Hq, Hkv, Dk, S_v, S_f, dtype, family, expected (chunk_major, skewed at two per CU,
    # one workgroup per CU by default)
    (8, 28, 4, 32, 4097, 61, torch.bfloat16, "gqa", (1, True, True)),     # config 4 layer, 4097 tokens
    (8, 28, 4, 64, 12001, 61, torch.bfloat16, "gqa", (1, False, False)),  # config 4 layer, 12001 tokens
    (1, 32, 32, 32, 15360, 640, torch.float16, "paper", (1, False, False)),  # config 1
    (3, 12, 4, 32, 2049, 17, torch.float16, "gqa", (1, False, False)),    # 12 units, 132 workgroups
    (2, 8, 8, 16, 3001, 129, torch.bfloat16, "paper", (1, False, False)),  # 208 workgroups: one per CU
    (2, 16, 16, 32, 2500, 60, torch.float16, "paper", (1, True, True)),   # 416 workgroups of <= 128 KB
    (1, 32, 32, 32, 8000, 640, torch.float16, "paper", (1, False, True)),  # one-head units, 177 KB: one per CU
    (1, 32, 32, 32, 12000, 640, torch.bfloat16, "paper", (1, False, True)),  # ... 256 KB at <= 32 channels
]


@pytest.mark.parametrize("case", CASES, ids=[f"B{c[0]}_Hq{c[1]}_Hkv{c[2]}_k{c[3]}_S{c[4]}" for c in CASES])
def test_layouts_match_oracle(case):
    from rotatek_amd.kernels.fused_decode import rotatek_decode_fused
    from rotatek_amd.kernels.gqa_decode import rotatek_decode_gqa
    B, Hq, Hkv, Dk, S_v, S_f, dtype, family, (cm, skewed, one_slot) = case
    fn = rotatek_decode_gqa if family == "gqa" else rotatek_decode_fused
    pol = _lib.RK_POLICY_GQA if Hq != Hkv else _lib.RK_POLICY_PAPER
    inp = _inputs(B, Hq, Hkv, Dk, S_v, S_f, dtype, seed=S_v + Dk)
    groups = sorted({(0, 0), (B - 1, Hkv - 1), (B // 2, Hkv // 2)})
    want = _oracle_groups(inp, groups)
    outs = {}
    plans = {}
    for name in MODES:
        _set_mode(name)
        p = plans[name] = _lib.plan_decode(B, Hq, Hkv, Dk, S_v, S_f, 2, pol)
        _say(f"{name}: B={B} Hq={Hq} Hkv={Hkv} Dk={Dk} S_v={S_v} S_f={S_f} {dtype} {family} plan "
             f"grid={p['grid']} chunk_major={p['chunk_major']} n_fast={p['n_fast']} "
             f"chunk_fast={p['chunk_fast']} chunk_vis={p['chunk_vis']}")
        if name == "unit_major":
            assert p["chunk_major"] == 0
        elif name == "chunk_major":
            assert p["chunk_major"] == cm and p["n_fast"] == 0
        elif name == "skewed":
            assert p["chunk_major"] == cm and (p["n_fast"] > 0) == skewed
        elif one_slot:
            assert p["chunk_major"] == 1 and p["n_fast"] == 0 and p["grid"] <= 256 < plans["skewed"]["grid"]
        else:
            assert p == plans["skewed"]
        outs[name] = fn(**inp)[0][:, 0]  # [B, H_q, D]
        torch.cuda.synchronize()
        got = _np(outs[name])
        assert np.isfinite(got).all()
        G = Hq // Hkv
        for (b, kv), w in want.items():
            err = np.abs(got[b, kv * G:(kv + 1) * G] - w).max()
            assert err <= TOL[dtype], (name, b, kv, err)
    for name in ("chunk_major", "skewed", "default"):
        assert (outs[name].float() - outs["unit_major"].float()).abs().max().item() <= TOL[dtype]


@pytest.mark.parametrize("layout", ["skewed", "default"])
@pytest.mark.parametrize("mode", ["eager", "graph"])
def test_fused_append_chunk_major(mode, layout):
    """The span cache's decode step (fused append) on a chunk-major grid,
    skewed at two workgroups per CU and one workgroup per CU (the default
    here): every step against the oracle on the grown spans, eager and
    replayed from one graph."""
    from rotatek_amd.cache import DynamicCache
    B, Hkv, G, S_p, S_v, S_t, Dk, steps = 8, 4, 7, 30, 4097, 30, 32, 4
    dt = torch.bfloat16
    _set_mode(layout)
    p = _lib.plan_decode(B, Hkv * G, Hkv, Dk, S_v, S_p + S_t + steps, 2, _lib.RK_POLICY_GQA)
    _say(f"fused append chunk-major {mode} {layout}: plan grid={p['grid']} chunk_major={p['chunk_major']} "
         f"n_fast={p['n_fast']}")
    if layout == "skewed":
        assert p["chunk_major"] == 1 and p["n_fast"] > 0
    else:
        assert p["chunk_major"] == 1 and p["n_fast"] == 0 and p["grid"] == 256
    g = torch.Generator(device="cuda").manual_seed(5)

    def rn(*s):
        return torch.randn(*s, generator=g, device="cuda").to(dt)

    cache = DynamicCache(reserve_tokens=steps)
    R = torch.linalg.qr(torch.randn(B, Hkv, 128, 128, generator=g, device="cuda"))[0][..., :Dk].contiguous().to(dt)
    dm = rn(B, Hkv, 128)
    ks, kp, kt = rn(B, Hkv, S_v, Dk), rn(B, Hkv, S_p, 128), rn(B, Hkv, S_t, 128)
    v = rn(B, Hkv, S_p + S_v + S_t, 128)
    cache.store_pruned(ks, kp, kt, torch.ones(B, Hkv, 128, dtype=torch.bool, device="cuda"), v, 0)
    cache.rotatek_rotations.append(R)
    cache.rotatek_means.append(dm)
    q, kn, vn = rn(steps, B, Hkv * G, 128), rn(steps, B, Hkv, 1, 128), rn(steps, B, Hkv, 1, 128)
    if mode == "graph":
        qs, kns, vns = q[:1].clone(), kn[:1].clone(), vn[:1].clone()
        out = torch.empty(1, B, Hkv * G, 128, device="cuda", dtype=dt)
        graph = cache.capture_decode(qs, kns, vns, out, G)
    for t in range(steps):
        if mode == "eager":
            got = cache.decode_step(q[t], kn[t], vn[t], 0, G)[0][:, 0]
        else:
            qs.copy_(q[t:t + 1])
            kns.copy_(kn[t:t + 1])
            vns.copy_(vn[t:t + 1])
            graph.replay()
            got = out[0]
        torch.cuda.synchronize()
        for b, kv in ((0, 0), (5, 3), (7, 1)):
            k_full = np.concatenate([_np(kp[b, kv]), _np(kt[b, kv])] + [_np(kn[i, b, kv]) for i in range(t + 1)])
            v_full = np.concatenate([_np(v[b, kv, :S_p]), _np(v[b, kv, S_p + S_v:])] +
                                    [_np(vn[i, b, kv]) for i in range(t + 1)])
            want = od.rotatek_decode(_np(q[t, b, kv * G:(kv + 1) * G])[None], _np(R[b, kv])[None, None],
                                     _np(dm[b, kv])[None, None], k_full[None, None], v_full[None, None], None,
                                     _np(ks[b, kv])[None, None], _np(v[b, kv, S_p:S_p + S_v])[None, None], G)
            err = np.abs(_np(got[b, kv * G:(kv + 1) * G]) - want[0, 0]).max()
            assert err <= TOL[dt], (mode, t, b, kv, err)
