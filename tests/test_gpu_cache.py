"""GPU checks of the span cache (rotatek_amd.cache) and the two entry points
behind it, rk_append_kv and rk_rotatek_decode_varlen.

* ``DynamicCache`` holds exactly what the reference's ``torch.cat`` cache
  (cache_utils.py:48-55, 76-83) holds after any sequence of updates
  (bit-exact), including across a capacity reallocation;
* ``decode_rotatek`` from the buffers equals the oracle on the adapter's
  concatenated ``k_full`` / ``v_full`` (llama_visionzip.py:197-215), per
  step, within the north-star tolerance;
* per-row lengths act as a mask of the tail rows;
* a captured HIP graph of append + decode replays over growing steps and
  matches the eager result each step.
"""
import sys

import numpy as np
import pytest
import torch

from oracle import decode as od

pytestmark = pytest.mark.gpu

D = 128
TOL = {torch.float16: 2e-3, torch.bfloat16: 1e-2}


def _say(msg):
    print(f"[case] {msg}", flush=True)
    sys.stdout.flush()


def _np(t):
    return None if t is None else t.detach().float().cpu().numpy().astype(np.float64)


def _prefill(B, Hkv, Dk, s_p, s_v, s_t, dtype, seed):
    g = torch.Generator(device="cuda").manual_seed(seed)

    def rn(*s, scale=1.0):
        return (torch.randn(*s, generator=g, device="cuda") * scale).to(dtype)

    R = torch.linalg.qr(torch.randn(B, Hkv, D, D, generator=g, device="cuda"))[0][..., :Dk]
    return dict(k_pruned=rn(B, Hkv, s_v, Dk, scale=2.0), k_prompt=rn(B, Hkv, s_p, D),
                k_text=rn(B, Hkv, s_t, D), v=rn(B, Hkv, s_p + s_v + s_t, D),
                R=R.contiguous().to(dtype), dm=rn(B, Hkv, D, scale=0.5), gen=g, rn=rn)


class _CatCache:
    """The reference's storage rule: torch.cat per decode token."""

    def __init__(self, p):
        self.k_prompt, self.k_text, self.v, self.k_pruned = p["k_prompt"], p["k_text"], p["v"], p["k_pruned"]

    def update(self, k, v):
        self.k_text = torch.cat([self.k_text, k], dim=-2)
        self.v = torch.cat([self.v, v], dim=-2)

    def rotatek_args(self, q, R, dm, G):
        s_p, s_v = self.k_prompt.shape[-2], self.k_pruned.shape[-2]
        kf = torch.cat([self.k_prompt, self.k_text], dim=-2)
        vf = torch.cat([self.v[:, :, :s_p], self.v[:, :, s_p + s_v:]], dim=-2)
        mask = torch.ones(q.shape[0], kf.shape[-2], dtype=torch.uint8, device=q.device)
        return dict(q_full=q, R_partial=R, delta_mu=dm, k_full=kf, v_full=vf, mask_full=mask,
                    k_sparse=self.k_pruned, v_sparse=self.v[:, :, s_p:s_p + s_v], num_kv_groups=G)


def _oracle(args):
    a = {k: (_np(v) if torch.is_tensor(v) else v) for k, v in args.items()}
    return od.rotatek_decode(a["q_full"], a["R_partial"], a["delta_mu"], a["k_full"], a["v_full"],
                             a["mask_full"], a["k_sparse"], a["v_sparse"], a["num_kv_groups"])


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("policy", [0, 1])
def test_span_cache_updates_and_decode_match_reference(dtype, policy):
    from rotatek_amd.cache import DynamicCache
    B, Hq, Hkv, Dk, s_p, s_v, s_t = 2, 8, 4, 32, 30, 517, 3
    _say(f"span cache update+decode {dtype} policy={policy}")
    p = _prefill(B, Hkv, Dk, s_p, s_v, s_t, dtype, seed=11)
    cache = DynamicCache(reserve_tokens=4)          # forces one reallocation below
    ref = _CatCache(p)
    kt, vv = cache.store_pruned(p["k_pruned"], p["k_prompt"], p["k_text"], None, p["v"], 0)
    cache.rotatek_rotations.append(p["R"])
    cache.rotatek_means.append(p["dm"])
    assert torch.equal(kt, p["k_text"]) and torch.equal(vv, p["v"])
    for step in range(7):
        k, v = p["rn"](B, Hkv, 1, D), p["rn"](B, Hkv, 1, D)
        text, value, pruned, prompt, mask = cache.update(k, v, 0)
        ref.update(k, v)
        assert torch.equal(text, ref.k_text) and torch.equal(value, ref.v)
        assert torch.equal(prompt, ref.k_prompt) and torch.equal(pruned, ref.k_pruned) and mask is None
        assert cache.get_seq_length(0) == s_p + s_v + s_t + step + 1
        q = p["rn"](B, Hq, D)
        out, a, b = cache.decode_rotatek(q, 0, Hq // Hkv, policy=policy)
        torch.cuda.synchronize()
        assert a is None and b is None and out.shape == (B, 1, Hq, D)
        want = _oracle(ref.rotatek_args(q, p["R"], p["dm"], Hq // Hkv))
        assert want.shape == out.shape
        err = np.abs(_np(out) - want).max()
        assert err <= TOL[dtype], (step, err)
    assert torch.equal(cache.lengths(0).cpu(), torch.full((B,), s_p + s_t + 7, dtype=torch.int32))
    assert cache._seen_tokens == s_p + s_v + s_t + 7


def test_unified_cache_matches_cat_and_dense_decode():
    from rotatek_amd.cache import DynamicCache
    from rotatek_amd.kernels.full_channel_flash_decoding import full_channel_decode
    _say("unified cache")
    dtype, B, Hq, Hkv, S = torch.float16, 2, 8, 8, 200
    g = torch.Generator(device="cuda").manual_seed(5)
    k0 = torch.randn(B, Hkv, S, D, generator=g, device="cuda").to(dtype)
    v0 = torch.randn(B, Hkv, S, D, generator=g, device="cuda").to(dtype)
    cache = DynamicCache(reserve_tokens=2)
    cache.store_unified(k0, v0, 0)
    kr, vr = k0, v0
    for step in range(5):
        k = torch.randn(B, Hkv, 1, D, generator=g, device="cuda").to(dtype)
        v = torch.randn(B, Hkv, 1, D, generator=g, device="cuda").to(dtype)
        ku, vu = cache.update_unified(k, v, 0)
        kr, vr = torch.cat([kr, k], dim=-2), torch.cat([vr, v], dim=-2)
        assert torch.equal(ku, kr) and torch.equal(vu, vr)
        assert cache.get_seq_length(0) == S + step + 1
        q = torch.randn(B, Hq, D, generator=g, device="cuda").to(dtype)
        got = full_channel_decode(q=q, k=ku, v=vu, num_kv_groups=1)
        want = full_channel_decode(q=q, k=kr, v=vr, num_kv_groups=1)
        torch.cuda.synchronize()
        assert torch.equal(got, want)


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_per_row_lengths_mask_the_tail(dtype):
    from rotatek_amd._lib import RK_POLICY_GQA
    from rotatek_amd.kernels import _launch
    B, Hq, Hkv, Dk, s_p, s_v, cap = 3, 8, 2, 32, 17, 301, 150
    _say(f"varlen per-row lengths {dtype}")
    p = _prefill(B, Hkv, Dk, s_p, s_v, cap, dtype, seed=3)
    kf = torch.cat([p["k_prompt"], p["k_text"]], dim=-2)           # [B,H,s_p+cap,D]
    vbuf = p["v"]                                                   # [B,H,s_p+s_v+cap,D]
    lens = torch.tensor([0, 40, s_p + cap], dtype=torch.int32, device="cuda")
    q = p["rn"](B, Hq, D)
    out = _launch.rotatek_decode_varlen(q, p["R"], p["dm"], kf, vbuf, s_p, s_v, None, p["k_pruned"],
                                        vbuf[:, :, s_p:s_p + s_v], Hq // Hkv, lens, RK_POLICY_GQA)
    torch.cuda.synchronize()
    vf = torch.cat([vbuf[:, :, :s_p], vbuf[:, :, s_p + s_v:]], dim=-2)
    mask = (torch.arange(s_p + cap, device="cuda")[None, :] < lens[:, None].long()).to(torch.uint8)
    want = _oracle(dict(q_full=q, R_partial=p["R"], delta_mu=p["dm"], k_full=kf, v_full=vf,
                        mask_full=mask, k_sparse=p["k_pruned"], v_sparse=vbuf[:, :, s_p:s_p + s_v],
                        num_kv_groups=Hq // Hkv))
    assert want.shape == (B, 1, Hq, D)
    assert np.abs(_np(out)[:, None] - want).max() <= TOL[dtype]


def test_append_into_a_full_buffer_leaves_it_unchanged():
    from rotatek_amd.cache import DynamicCache
    _say("append into full buffer")
    dtype, B, Hkv, s_p, s_v, s_t = torch.float16, 2, 2, 5, 9, 3
    p = _prefill(B, Hkv, 16, s_p, s_v, s_t, dtype, seed=1)
    cache = DynamicCache(reserve_tokens=0)
    cache.store_pruned(p["k_pruned"], p["k_prompt"], p["k_text"], None, p["v"], 0)
    sp = cache._spans[0]
    k_before, v_before = sp.k.clone(), sp.v.clone()
    cache.append_(0, p["rn"](B, Hkv, 1, D), p["rn"](B, Hkv, 1, D))
    torch.cuda.synchronize()
    assert torch.equal(sp.k, k_before) and torch.equal(sp.v, v_before)
    assert torch.equal(sp.lens.cpu(), torch.full((B,), s_p + s_t, dtype=torch.int32))


@pytest.mark.parametrize("policy", [0, 1])
def test_graph_of_append_and_decode_replays_across_steps(policy):
    from rotatek_amd.cache import DynamicCache
    B, Hq, Hkv, Dk, s_p, s_v, s_t, steps = 2, 28, 4, 32, 30, 4097, 30, 6
    dtype = torch.bfloat16
    _say(f"graph append+decode over {steps} steps policy={policy}")
    p = _prefill(B, Hkv, Dk, s_p, s_v, s_t, dtype, seed=21)
    cache = DynamicCache(reserve_tokens=steps + 2)
    cache.store_pruned(p["k_pruned"], p["k_prompt"], p["k_text"], None, p["v"], 0)
    cache.rotatek_rotations.append(p["R"])
    cache.rotatek_means.append(p["dm"])
    ref = _CatCache(p)
    G = Hq // Hkv
    k_in = torch.zeros(B, Hkv, 1, D, dtype=dtype, device="cuda")
    v_in = torch.zeros_like(k_in)
    q_in = torch.zeros(B, Hq, D, dtype=dtype, device="cuda")
    out = torch.empty(B, Hq, D, dtype=dtype, device="cuda")
    # warm-up outside the graph (workspace allocation), then undo its append
    lens0 = cache.lengths(0).clone()
    cache.append_(0, k_in, v_in)
    cache.decode_rotatek(q_in, 0, G, policy=policy, out=out)
    torch.cuda.synchronize()
    cache.lengths(0).copy_(lens0)
    graph = torch.cuda.CUDAGraph()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        with torch.cuda.graph(graph, stream=s):
            cache.append_(0, k_in, v_in)
            cache.decode_rotatek(q_in, 0, G, policy=policy, out=out)
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    cache.lengths(0).copy_(lens0)            # capture does not run the kernels; keep it explicit
    for step in range(steps):
        k, v, q = p["rn"](B, Hkv, 1, D), p["rn"](B, Hkv, 1, D), p["rn"](B, Hq, D)
        k_in.copy_(k)
        v_in.copy_(v)
        q_in.copy_(q)
        graph.replay()
        torch.cuda.synchronize()
        ref.update(k, v)
        eager, _, _ = cache.decode_rotatek(q, 0, G, policy=policy)
        torch.cuda.synchronize()
        assert torch.equal(out, eager[:, 0]), step
        want = _oracle(ref.rotatek_args(q, p["R"], p["dm"], G))
        assert np.abs(_np(out)[:, None] - want).max() <= TOL[dtype], step
    cache.sync_lengths()
    assert torch.equal(cache.key_cache_text[0], ref.k_text) and torch.equal(cache.value_cache[0], ref.v)
    assert cache.get_seq_length(0) == s_p + s_v + s_t + steps


def test_capture_decode_over_layers_matches_eager():
    from rotatek_amd.cache import DynamicCache
    L, B, Hq, Hkv, Dk, s_p, s_v, s_t, steps = 3, 2, 8, 2, 16, 7, 333, 5, 4
    dtype = torch.bfloat16
    _say(f"capture_decode over {L} layers, {steps} replays")
    cache = DynamicCache(reserve_tokens=steps)
    refs, ps = [], []
    for layer in range(L):
        p = _prefill(B, Hkv, Dk, s_p, s_v, s_t, dtype, seed=40 + layer)
        cache.store_pruned(p["k_pruned"], p["k_prompt"], p["k_text"], None, p["v"], layer)
        cache.rotatek_rotations.append(p["R"])
        cache.rotatek_means.append(p["dm"])
        refs.append(_CatCache(p))
        ps.append(p)
    q = torch.zeros(L, B, Hq, D, dtype=dtype, device="cuda")
    kn = torch.zeros(L, B, Hkv, 1, D, dtype=dtype, device="cuda")
    vn = torch.zeros_like(kn)
    out = torch.empty(L, B, Hq, D, dtype=dtype, device="cuda")
    graph = cache.capture_decode(q, kn, vn, out, Hq // Hkv)
    torch.cuda.synchronize()
    for step in range(steps):
        for layer in range(L):
            rn = ps[layer]["rn"]
            q[layer].copy_(rn(B, Hq, D))
            kn[layer].copy_(rn(B, Hkv, 1, D))
            vn[layer].copy_(rn(B, Hkv, 1, D))
            refs[layer].update(kn[layer].clone(), vn[layer].clone())
        graph.replay()
        torch.cuda.synchronize()
        for layer in range(L):
            want = _oracle(refs[layer].rotatek_args(q[layer], ps[layer]["R"], ps[layer]["dm"], Hq // Hkv))
            assert np.abs(_np(out[layer])[:, None] - want).max() <= TOL[dtype], (step, layer)
    cache.sync_lengths()
    for layer in range(L):
        assert torch.equal(cache.key_cache_text[layer], refs[layer].k_text)
        assert torch.equal(cache.value_cache[layer], refs[layer].v)


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("policy", [0, 1])
def test_fused_append_decode_step_matches_reference(dtype, policy):
    """decode_step = append then decode, in the decode's own two launches."""
    from rotatek_amd.cache import DynamicCache
    B, Hq, Hkv, Dk, s_p, s_v, s_t = 2, 28, 4, 32, 30, 700, 30
    _say(f"fused append+decode {dtype} policy={policy}")
    p = _prefill(B, Hkv, Dk, s_p, s_v, s_t, dtype, seed=17)
    cache = DynamicCache(reserve_tokens=5)
    cache.store_pruned(p["k_pruned"], p["k_prompt"], p["k_text"], None, p["v"], 0)
    cache.rotatek_rotations.append(p["R"])
    cache.rotatek_means.append(p["dm"])
    ref = _CatCache(p)
    for step in range(5):
        k, v, q = p["rn"](B, Hkv, 1, D), p["rn"](B, Hkv, 1, D), p["rn"](B, Hq, D)
        out, _, _ = cache.decode_step(q, k, v, 0, Hq // Hkv, policy=policy)
        torch.cuda.synchronize()
        ref.update(k, v)
        want = _oracle(ref.rotatek_args(q, p["R"], p["dm"], Hq // Hkv))
        assert np.abs(_np(out) - want).max() <= TOL[dtype], step
        assert torch.equal(cache.lengths(0).cpu(), torch.full((B,), s_p + s_t + step + 1, dtype=torch.int32))
    cache.sync_lengths()
    assert torch.equal(cache.key_cache_text[0], ref.k_text) and torch.equal(cache.value_cache[0], ref.v)
    # the buffers are now full: a further step neither stores nor attends the token
    sp = cache._spans[0]
    k_before, v_before = sp.k.clone(), sp.v.clone()
    k, v, q = p["rn"](B, Hkv, 1, D), p["rn"](B, Hkv, 1, D), p["rn"](B, Hq, D)
    out, _, _ = cache.decode_step(q, k, v, 0, Hq // Hkv, policy=policy)
    torch.cuda.synchronize()
    assert torch.equal(sp.k, k_before) and torch.equal(sp.v, v_before)
    want = _oracle(ref.rotatek_args(q, p["R"], p["dm"], Hq // Hkv))
    assert np.abs(_np(out) - want).max() <= TOL[dtype]


def test_fused_append_with_ragged_lengths():
    from rotatek_amd._lib import RK_POLICY_GQA
    from rotatek_amd.kernels import _launch
    dtype, B, Hq, Hkv, Dk, s_p, s_v, cap = torch.float16, 3, 8, 2, 32, 9, 200, 40
    _say("fused append, ragged per-row lengths")
    p = _prefill(B, Hkv, Dk, s_p, s_v, cap, dtype, seed=23)
    kf = torch.cat([p["k_prompt"], p["k_text"]], dim=-2).contiguous()
    vbuf = p["v"].clone()
    lens = torch.tensor([0, 20, s_p + cap], dtype=torch.int32, device="cuda")   # last row is full
    kn, vn, q = p["rn"](B, Hkv, 1, D), p["rn"](B, Hkv, 1, D), p["rn"](B, Hq, D)
    kf0, vb0, lens0 = kf.clone(), vbuf.clone(), lens.clone()
    out = _launch.rotatek_decode_varlen(q, p["R"], p["dm"], kf, vbuf, s_p, s_v, None, p["k_pruned"],
                                        vbuf[:, :, s_p:s_p + s_v], Hq // Hkv, lens, RK_POLICY_GQA,
                                        k_new=kn, v_new=vn)
    torch.cuda.synchronize()
    # expected buffers: token written at row lens0[b] of rows that had room
    kf_want, vb_want = kf0.clone(), vb0.clone()
    for b in range(B):
        pos = int(lens0[b])
        if pos < s_p + cap:
            kf_want[b, :, pos] = kn[b, :, 0]
            row = pos + (s_v if pos >= s_p else 0)
            vb_want[b, :, row] = vn[b, :, 0]
    assert torch.equal(kf, kf_want) and torch.equal(vbuf, vb_want)
    assert lens.tolist() == [1, 21, s_p + cap]
    vf = torch.cat([vb_want[:, :, :s_p], vb_want[:, :, s_p + s_v:]], dim=-2)
    mask = (torch.arange(s_p + cap, device="cuda")[None, :] < lens[:, None].long()).to(torch.uint8)
    want = _oracle(dict(q_full=q, R_partial=p["R"], delta_mu=p["dm"], k_full=kf_want, v_full=vf,
                        mask_full=mask, k_sparse=p["k_pruned"], v_sparse=vb_want[:, :, s_p:s_p + s_v],
                        num_kv_groups=Hq // Hkv))
    assert np.abs(_np(out)[:, None] - want).max() <= TOL[dtype]


def test_graph_survives_workspace_growth_after_capture():
    """A captured decode graph keeps its workspace: a later, larger decode
    grows the shared workspace (the old buffer is retired, not freed), a
    tensor allocated afterwards must not alias it, and the replays still
    match the oracle."""
    from rotatek_amd import _lib
    from rotatek_amd.cache import DynamicCache
    from rotatek_amd.kernels.gqa_decode import rotatek_decode_gqa
    B, Hq, Hkv, Dk, s_p, s_v, s_t, steps = 2, 8, 2, 32, 7, 900, 5, 3
    dtype = torch.bfloat16
    _say("graph replay after the workspace grew")
    p = _prefill(B, Hkv, Dk, s_p, s_v, s_t, dtype, seed=61)
    cache = DynamicCache(reserve_tokens=steps)
    cache.store_pruned(p["k_pruned"], p["k_prompt"], p["k_text"], None, p["v"], 0)
    cache.rotatek_rotations.append(p["R"])
    cache.rotatek_means.append(p["dm"])
    ref = _CatCache(p)
    q = torch.zeros(1, B, Hq, D, dtype=dtype, device="cuda")
    kn = torch.zeros(1, B, Hkv, 1, D, dtype=dtype, device="cuda")
    vn = torch.zeros_like(kn)
    out = torch.empty(1, B, Hq, D, dtype=dtype, device="cuda")
    # start from a workspace sized for this cache alone (earlier tests may
    # have grown the shared one past the large decode below)
    idx = torch.cuda.current_device()
    if idx in _lib._WORKSPACE:
        _lib._RETIRED.append(_lib._WORKSPACE.pop(idx))
    graph = cache.capture_decode(q, kn, vn, out, Hq // Hkv)
    torch.cuda.synchronize()
    old_ws = _lib._WORKSPACE[idx].data_ptr()
    # a much larger decode grows the workspace past the captured buffer
    g = torch.Generator(device="cuda").manual_seed(3)
    big = dict(q_full=torch.randn(16, 32, D, generator=g, device="cuda").to(dtype),
               R_partial=torch.randn(16, 8, D, Dk, generator=g, device="cuda").to(dtype),
               delta_mu=None,
               k_full=torch.randn(16, 8, 4000, D, generator=g, device="cuda").to(dtype),
               v_full=torch.randn(16, 8, 4000, D, generator=g, device="cuda").to(dtype),
               mask_full=torch.ones(16, 4000, dtype=torch.uint8, device="cuda"),
               k_sparse=torch.randn(16, 8, 30000, Dk, generator=g, device="cuda").to(dtype),
               v_sparse=torch.randn(16, 8, 30000, D, generator=g, device="cuda").to(dtype),
               num_kv_groups=4)
    rotatek_decode_gqa(**big)
    torch.cuda.synchronize()
    assert _lib._WORKSPACE[torch.cuda.current_device()].data_ptr() != old_ws
    del big
    torch.cuda.empty_cache()
    filler = torch.full((1 << 22,), 7.0, device="cuda")   # may land where a freed buffer was
    for step in range(steps):
        kq, kk, kv = p["rn"](B, Hq, D), p["rn"](B, Hkv, 1, D), p["rn"](B, Hkv, 1, D)
        q[0].copy_(kq)
        kn[0].copy_(kk)
        vn[0].copy_(kv)
        graph.replay()
        torch.cuda.synchronize()
        ref.update(kk, kv)
        want = _oracle(ref.rotatek_args(kq, p["R"], p["dm"], Hq // Hkv))
        assert np.abs(_np(out[0])[:, None] - want).max() <= TOL[dtype], step
    assert bool((filler == 7.0).all())
