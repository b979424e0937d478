"""GPU check of the allocation-free decode entry point
(rk_rotatek_decode_noalloc, a fixed device scratch array in place of the
workspace): through the C ABI it must equal rk_rotatek_decode bit for bit,
on two calls in a row, the second with a smaller input, under both merges;
an oversized problem is refused with RK_ERR_SCRATCH before any launch.
"""
import ctypes
import sys

import pytest
import torch

from rotatek_amd import _lib

pytestmark = pytest.mark.gpu


def _say(msg):
    print(f"[case] {msg}", flush=True)
    sys.stdout.flush()


def _inputs(B, Hq, Hkv, Dk, S_v, S_f, dtype, seed):
    g = torch.Generator(device="cuda").manual_seed(seed)

    def rn(*s, scale=1.0):
        return (torch.randn(*s, generator=g, device="cuda") * scale).to(dtype)

    R = torch.linalg.qr(torch.randn(B, Hkv, 128, 128, generator=g, device="cuda"))[0][..., :Dk]
    V = rn(B, Hkv, S_v + S_f, 128)
    return [rn(B, Hq, 128), R.contiguous().to(dtype), rn(B, Hkv, 128, scale=0.5), rn(B, Hkv, S_f, 128),
            V[:, :, S_v:], (torch.rand(B, S_f, generator=g, device="cuda") >= 0.2).to(torch.uint8),
            rn(B, Hkv, S_v, Dk, scale=2.0), V[:, :, :S_v]]


def _run(entry, tensors, G, policy):
    """out via the C ABI: entry 'workspace' (rk_rotatek_decode) or 'noalloc'."""
    lib = _lib.load()
    q = tensors[0]
    out = torch.empty_like(q)
    d = [_lib.desc(t) for t in tensors]
    do = _lib.desc(out)
    stream = _lib.stream_handle(q.device)
    if entry == "noalloc":
        st = lib.rk_rotatek_decode_noalloc(*[ctypes.byref(x) for x in d], G, ctypes.byref(do), policy, stream)
    else:
        need = ctypes.c_size_t(0)
        _lib.check(lib.rk_rotatek_decode_check(*[ctypes.byref(x) for x in d], G, ctypes.byref(do), policy, 0,
                                               ctypes.byref(need)), "check")
        ws = _lib.workspace(q.device, need.value)
        st = lib.rk_rotatek_decode(*[ctypes.byref(x) for x in d], G, ctypes.byref(do), policy, ws.data_ptr(),
                                   ws.numel(), stream)
    torch.cuda.synchronize()
    return st, out


@pytest.mark.parametrize("merge", [_lib.MERGE_TWO_LAUNCHES, _lib.MERGE_SINGLE_LAUNCH])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_noalloc_matches_workspace_entry(dtype, merge):
    _lib.set_decode_merge(merge)
    try:
        # a larger call, then a smaller one: the second must not see the first's records
        for i, (B, Hq, Hkv, S_v, S_f) in enumerate([(8, 28, 4, 12001, 61), (2, 8, 8, 900, 33)]):
            _say(f"noalloc {dtype} merge={merge} call {i}: B={B} Hq={Hq} Hkv={Hkv} S_v={S_v} S_f={S_f}")
            t = _inputs(B, Hq, Hkv, 32, S_v, S_f, dtype, seed=100 + i)
            G = Hq // Hkv
            st_w, want = _run("workspace", t, G, _lib.RK_POLICY_GQA)
            st_n, got = _run("noalloc", t, G, _lib.RK_POLICY_GQA)
            assert st_w == 0 and st_n == 0, (st_w, st_n)
            assert torch.equal(got, want)
    finally:
        _lib.set_decode_merge(_lib.MERGE_AUTO)


def test_noalloc_fp32_and_paper_family():
    _say("noalloc fp32, paper family")
    t = _inputs(1, 8, 8, 32, 700, 50, torch.float32, seed=7)
    st_w, want = _run("workspace", t, 1, _lib.RK_POLICY_PAPER)
    st_n, got = _run("noalloc", t, 1, _lib.RK_POLICY_PAPER)
    assert st_w == 0 and st_n == 0
    assert torch.equal(got, want)


def test_noalloc_rejects_oversized_problem():
    """A plan whose partials exceed the scratch is refused before any launch."""
    _say("noalloc oversized plan")
    B, Hq, Hkv, S_v, S_f = 64, 64, 64, 40000, 100
    need = _lib.plan_decode(B, Hq, Hkv, 32, S_v, S_f, 2, _lib.RK_POLICY_PAPER,
                            torch.cuda.get_device_properties(0).multi_processor_count)["workspace_bytes"]
    assert need > _lib.NOALLOC_SCRATCH_BYTES
    # descriptors only (no device memory behind K/V): the size check comes first
    def t(shape, dt=_lib.RK_BF16):
        d = _lib.RkTensor()
        d.data, d.dtype, d.ndim = 0, dt, len(shape)
        acc = 1
        for i in reversed(range(len(shape))):
            d.shape[i], d.stride[i] = shape[i], acc
            acc *= shape[i]
        return d
    ds = [t((B, Hq, 128)), t((B, Hkv, 128, 32)), t((B, Hkv, 128)), t((B, Hkv, S_f, 128)), t((B, Hkv, S_f, 128)),
          t((B, S_f), _lib.RK_U8), t((B, Hkv, S_v, 32)), t((B, Hkv, S_v, 128))]
    o = t((B, Hq, 128))
    st = _lib.load().rk_rotatek_decode_noalloc(*[ctypes.byref(x) for x in ds], 1, ctypes.byref(o),
                                               _lib.RK_POLICY_PAPER, None)
    assert st == _lib.RK_ERR_SCRATCH
    with pytest.raises(ValueError, match="allocation-free"):
        _lib.check(st, "noalloc")


def _graph_replays_match(tensors, G, n_replays=4):
    """Capture one allocation-free decode in a CUDA graph and replay it
    n_replays times, with eager decodes of other inputs and synchronisations
    between the replays; every replay must equal rk_rotatek_decode bit for
    bit.  Returns the number of replays checked."""
    q = tensors[0]
    out = torch.empty_like(q)
    d = [_lib.desc(t) for t in tensors]
    do = _lib.desc(out)
    lib = _lib.load()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=s):
        st = lib.rk_rotatek_decode_noalloc(*[ctypes.byref(x) for x in d], G, ctypes.byref(do),
                                           _lib.RK_POLICY_GQA, _lib.stream_handle(q.device))
    assert st == 0, _lib.strerror(st)
    st_w, want = _run("workspace", tensors, G, _lib.RK_POLICY_GQA)
    assert st_w == 0
    other = _inputs(1, 4, 4, 32, 300, 20, tensors[0].dtype, seed=999)
    for i in range(n_replays):
        out.fill_(float("nan"))
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, want), f"replay {i}"
        _run("noalloc", other, 1, _lib.RK_POLICY_GQA)  # eager work between replays, same scratch
    return n_replays


@pytest.mark.parametrize("merge", [_lib.MERGE_TWO_LAUNCHES, _lib.MERGE_SINGLE_LAUNCH])
def test_noalloc_captured_after_an_eager_call(merge):
    _lib.set_decode_merge(merge)
    try:
        _say(f"noalloc captured after eager, merge={merge}")
        t = _inputs(2, 16, 4, 32, 3000, 45, torch.bfloat16, seed=31)
        _run("noalloc", t, 4, _lib.RK_POLICY_GQA)
        assert _graph_replays_match(t, 4) == 4
    finally:
        _lib.set_decode_merge(_lib.MERGE_AUTO)


_FIRST_CALL_SCRIPT = r"""
import ctypes, sys, torch
sys.path.insert(0, sys.argv[1])
import tests.test_zz_no_alloc as m
from rotatek_amd import _lib
_lib.set_decode_merge(int(sys.argv[2]))
t = m._inputs(2, 16, 4, 32, 3000, 45, torch.bfloat16, seed=32)
print("replays", m._graph_replays_match(t, 4), flush=True)
"""


@pytest.mark.parametrize("merge", [_lib.MERGE_TWO_LAUNCHES, _lib.MERGE_SINGLE_LAUNCH])
def test_noalloc_captured_as_the_first_call_on_the_device(merge):
    """In a fresh process the first allocation-free decode on the device is
    the one being captured: the scratch address is taken then, and with the
    single-launch merge the counters' fill kernel is recorded into the graph
    ahead of the decode."""
    import os
    import subprocess
    _say(f"noalloc captured as the first call (subprocess), merge={merge}")
    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    res = subprocess.run([sys.executable, "-c", _FIRST_CALL_SCRIPT, root, str(merge)], capture_output=True,
                         text=True, timeout=300)
    assert res.returncode == 0, res.stdout[-2000:] + res.stderr[-4000:]
    assert "replays 4" in res.stdout
