"""GPU checks of the decode merge: the single-launch merge (the last
workgroup of each unit merges the unit's records behind a ticket) against
the two-launch merge (a second kernel).

Both fold the records in the same order, so the outputs must be
bit-identical, on every shape, family, dtype and span layout, and across
repeated calls and graph replays on one workspace.  Record memory is
poisoned with NaN between calls, so a merge that read anything but this
call's records could not pass, and the counters must be back at zero after
every call.  The fused append's length advance (behind the per-row
ticket) must match the two-launch one step for step.
"""
import sys

import numpy as np
import pytest
import torch

from oracle import decode as od
from rotatek_amd import _lib

pytestmark = pytest.mark.gpu

TOL = {torch.float16: 2e-3, torch.bfloat16: 1e-2}


def _say(msg):
    print(f"[case] {msg}", flush=True)
    sys.stdout.flush()


def _np(t):
    return None if t is None else t.detach().float().cpu().numpy().astype(np.float64)


@pytest.fixture(autouse=True)
def _restore_merge_mode():
    yield
    _lib.set_decode_merge(_lib.MERGE_AUTO)


def _inputs(B, Hq, Hkv, Dk, S_v, S_f, dtype, seed, mask_p=0.2):
    g = torch.Generator(device="cuda").manual_seed(seed)

    def rn(*s, scale=1.0):
        return (torch.randn(*s, generator=g, device="cuda") * scale).to(dtype)

    R = torch.linalg.qr(torch.randn(B, Hkv, 128, 128, generator=g, device="cuda"))[0][..., :Dk]
    V = rn(B, Hkv, S_v + S_f, 128)
    return dict(q_full=rn(B, Hq, 128), R_partial=R.contiguous().to(dtype), delta_mu=rn(B, Hkv, 128, scale=0.5),
                k_full=rn(B, Hkv, S_f, 128), v_full=V[:, :, S_v:],
                mask_full=(torch.rand(B, S_f, generator=g, device="cuda") >= mask_p).to(torch.uint8),
                k_sparse=rn(B, Hkv, S_v, Dk, scale=2.0), v_sparse=V[:, :, :S_v], num_kv_groups=Hq // Hkv)


def _decode(inp, family, mode):
    from rotatek_amd.kernels.fused_decode import rotatek_decode_fused
    from rotatek_amd.kernels.gqa_decode import rotatek_decode_gqa
    _lib.set_decode_merge(mode)
    fn = rotatek_decode_gqa if family == "gqa" else rotatek_decode_fused
    out = fn(**inp)[0]
    torch.cuda.synchronize()
    return out


def _poison_records(device):
    """NaN over the workspace past the counters (a fill kernel)."""
    ws = _lib._WORKSPACE[device.index if device.index is not None else torch.cuda.current_device()]
    n = ws.numel() - _lib.DECODE_TICKET_BYTES
    if n > 0:
        ws[_lib.DECODE_TICKET_BYTES:].view(torch.float32)[: n // 4].fill_(float("nan"))


def _tickets_zero(ws):
    """Unit and batch-row tickets of workspace ``ws`` are back at zero."""
    return int(torch.count_nonzero(ws[:_lib.DECODE_TICKET_BYTES]).item()) == 0


def _counters_zero(device):
    return _tickets_zero(_lib._WORKSPACE[device.index if device.index is not None else torch.cuda.current_device()])


CASES = [
    # B, Hq, Hkv, Dk, S_v, S_f
    (1, 32, 32, 32, 15360, 640),     # config 1 shape
    (8, 28, 4, 32, 12001, 61),       # a config 4 layer
    (8, 28, 4, 64, 4097, 60),
    (2, 8, 8, 32, 1000, 129),
    (1, 40, 2, 32, 300, 20),         # two head blocks
    (2, 4, 4, 32, 0, 300),           # no visual span
    (2, 4, 4, 64, 1025, 0),          # no prompt/text span
    (1, 2, 2, 32, 1, 1),
]


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("family", ["paper", "gqa"])
@pytest.mark.parametrize("case", CASES)
def test_single_launch_merge_is_bit_identical(case, family, dtype):
    B, Hq, Hkv, Dk, S_v, S_f = case
    _say(f"merge modes {family} {dtype} B={B} Hq={Hq} Hkv={Hkv} Dk={Dk} S_v={S_v} S_f={S_f}")
    inp = _inputs(B, Hq, Hkv, Dk, S_v, S_f, dtype, seed=sum(case))
    two = _decode(inp, family, _lib.MERGE_TWO_LAUNCHES)
    _poison_records(two.device)
    one = _decode(inp, family, _lib.MERGE_SINGLE_LAUNCH)
    assert torch.equal(one, two)
    assert _counters_zero(one.device)
    if S_v + S_f <= 2000:
        want = od.rotatek_decode(*[_np(inp[k]) for k in ("q_full", "R_partial", "delta_mu", "k_full", "v_full",
                                                          "mask_full", "k_sparse", "v_sparse")],
                                 inp["num_kv_groups"])
        assert np.abs(_np(one) - want).max() <= TOL[dtype]


def test_alternating_inputs_on_one_workspace():
    """Two input sets of one shape alternate through the single-launch merge,
    records poisoned between calls: every call equals the two-launch result
    of its own inputs (a stale record from the other set would show)."""
    _say("merge alternating inputs")
    sets = [_inputs(4, 28, 4, 32, 3001, 70, torch.bfloat16, seed=s) for s in (11, 12)]
    want = [_decode(x, "gqa", _lib.MERGE_TWO_LAUNCHES) for x in sets]
    for i in range(40):
        _poison_records(want[0].device)
        got = _decode(sets[i % 2], "gqa", _lib.MERGE_SINGLE_LAUNCH)
        assert torch.equal(got, want[i % 2]), i
    assert _counters_zero(want[0].device)


def test_shapes_of_different_unit_counts_share_a_workspace():
    """Shapes of 8, 32 and 16 units take turns on one workspace through the
    single-launch merge: each call equals the two-launch merge of its own
    inputs and leaves the tickets at zero (unit and batch-row tickets sit
    at fixed offsets, so one shape's counters never overlap another's)."""
    shapes = [(1, 8, 8, 32, 4000, 64), (1, 32, 32, 32, 8000, 640), (2, 8, 8, 32, 3001, 129)]
    sets = [_inputs(*s, torch.float16, seed=sum(s)) for s in shapes]
    want = [_decode(x, "paper", _lib.MERGE_TWO_LAUNCHES) for x in sets]
    for i, j in enumerate([0, 1, 0, 2, 1, 2, 0, 1, 1, 2]):
        _say(f"merge shape turns: call {i} shape {shapes[j]}")
        _poison_records(want[0].device)
        got = _decode(sets[j], "paper", _lib.MERGE_SINGLE_LAUNCH)
        assert torch.equal(got, want[j]), (i, shapes[j])
        assert _counters_zero(got.device)


def test_dense_baseline_single_launch():
    _say("merge dense baseline paper G=4 / gqa")
    from rotatek_amd.kernels.full_channel_flash_decoding import full_channel_decode
    from rotatek_amd.kernels.gqa_decode import full_channel_decode_gqa
    g = torch.Generator(device="cuda").manual_seed(5)
    q = torch.randn(2, 16, 128, generator=g, device="cuda").half()
    k = torch.randn(2, 4, 3000, 128, generator=g, device="cuda").half()
    v = torch.randn(2, 4, 3000, 128, generator=g, device="cuda").half()
    for fn in (full_channel_decode, full_channel_decode_gqa):
        outs = []
        for mode in (_lib.MERGE_TWO_LAUNCHES, _lib.MERGE_SINGLE_LAUNCH):
            _lib.set_decode_merge(mode)
            outs.append(fn(q, k, v, num_kv_groups=4))
            torch.cuda.synchronize()
            _poison_records(q.device)
        assert torch.equal(outs[0], outs[1])
    assert _counters_zero(q.device)


@pytest.mark.parametrize("G", [7, 1])
@pytest.mark.parametrize("mode", ["eager", "graph"])
def test_fused_append_length_advance(mode, G):
    """decode_step (fused append) under both merges over 6 steps: the same
    outputs, lengths and appended rows, eager or replayed from a graph; G = 1
    merges one query head per unit by a slice."""
    _say(f"merge fused append {mode} G={G}")
    from rotatek_amd.cache import DynamicCache
    B, Hkv, S_p, S_v, S_t, Dk = 3, 4, 5, 2000, 9, 32
    dt = torch.bfloat16
    results = []
    for merge in (_lib.MERGE_TWO_LAUNCHES, _lib.MERGE_SINGLE_LAUNCH):
        _lib.set_decode_merge(merge)
        g = torch.Generator(device="cuda").manual_seed(77)

        def rn(*s):
            return torch.randn(*s, generator=g, device="cuda").to(dt)

        cache = DynamicCache(reserve_tokens=8)
        R = torch.linalg.qr(torch.randn(B, Hkv, 128, 128, generator=g, device="cuda"))[0][..., :Dk].contiguous().to(dt)
        cache.store_pruned(rn(B, Hkv, S_v, Dk), rn(B, Hkv, S_p, 128), rn(B, Hkv, S_t, 128),
                           torch.ones(B, Hkv, 128, dtype=torch.bool, device="cuda"),
                           rn(B, Hkv, S_p + S_v + S_t, 128), 0)
        cache.rotatek_rotations.append(R)
        cache.rotatek_means.append(rn(B, Hkv, 128))
        steps = 6
        q = rn(steps, B, Hkv * G, 128)
        kn, vn = rn(steps, B, Hkv, 1, 128), rn(steps, B, Hkv, 1, 128)
        outs = []
        if mode == "eager":
            for t in range(steps):
                outs.append(cache.decode_step(q[t], kn[t], vn[t], 0, G)[0][:, 0].clone())
        else:
            qs, ks, vs = q[:1].clone(), kn[:1].clone(), vn[:1].clone()
            out = torch.empty(1, B, Hkv * G, 128, device="cuda", dtype=dt)
            graph = cache.capture_decode(qs, ks, vs, out, G)
            for t in range(steps):
                qs.copy_(q[t:t + 1])
                ks.copy_(kn[t:t + 1])
                vs.copy_(vn[t:t + 1])
                graph.replay()
                torch.cuda.synchronize()
                outs.append(out[0].clone())
        torch.cuda.synchronize()
        lens = cache.lengths(0).clone()
        results.append((torch.stack(outs), lens, cache._spans[0].k.clone(), cache._spans[0].v.clone()))
    (o2, l2, k2, v2), (o1, l1, k1, v1) = results
    assert torch.equal(l1, l2) and int(l1[0]) == S_p + S_t + 6
    assert torch.equal(o1, o2)
    rows = S_p + S_t + 6
    assert torch.equal(k1[:, :, :rows], k2[:, :, :rows])
    assert torch.equal(v1[:, :, :rows + S_v], v2[:, :, :rows + S_v])


def _abi_decode(inp, ws, policy=_lib.RK_POLICY_GQA):
    """rk_rotatek_decode through the C ABI on a caller-owned workspace."""
    import ctypes
    names = ("q_full", "R_partial", "delta_mu", "k_full", "v_full", "mask_full", "k_sparse", "v_sparse")
    d = [_lib.desc(inp[k]) for k in names]
    out = torch.empty_like(inp["q_full"])
    do = _lib.desc(out)
    st = _lib.load().rk_rotatek_decode(*[ctypes.byref(x) for x in d], inp["num_kv_groups"], ctypes.byref(do),
                                       policy, ws.data_ptr(), ws.numel(), _lib.stream_handle(out.device))
    torch.cuda.synchronize()
    assert st == 0, _lib.strerror(st)
    return out


@pytest.mark.parametrize("case", [(1, 32, 32, 32, 15360, 640), (8, 28, 4, 32, 12001, 61)])
def test_uninitialised_workspace_with_garbage_counters(case):
    """A caller-owned workspace that was never passed to
    rk_decode_workspace_init, its counter region full of garbage: the first
    single-launch decode on it already equals the two-launch merge (the
    library zeroes the counters of an address it has not seen), so does the
    next one, and the tickets are zero after each.  After
    rk_decode_workspace_release the address is treated as new again."""
    B, Hq, Hkv, Dk, S_v, S_f = case
    _say(f"garbage counters B={B} Hq={Hq} Hkv={Hkv}")
    inp = _inputs(B, Hq, Hkv, Dk, S_v, S_f, torch.bfloat16, seed=sum(case) + 1)
    want = _decode(inp, "gqa", _lib.MERGE_TWO_LAUNCHES)[:, 0]
    need = _lib.plan_decode(B, Hq, Hkv, Dk, S_v, S_f, 2, _lib.RK_POLICY_GQA,
                            torch.cuda.get_device_properties(0).multi_processor_count)["workspace_bytes"]
    ws = torch.full((need + 4096,), 0x5A, dtype=torch.uint8, device="cuda")
    _lib.set_decode_merge(_lib.MERGE_SINGLE_LAUNCH)
    for round_ in range(2):
        for call in range(2):
            got = _abi_decode(inp, ws)
            assert torch.equal(got, want), (round_, call)
            assert _tickets_zero(ws)
        _lib.load().rk_decode_workspace_release(ws.data_ptr())
        ws.fill_(0x5A)
        torch.cuda.synchronize()
