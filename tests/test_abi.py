"""CPU checks of the C ABI boundary (no GPU needed).

* the library loads and exports every function include/rotatek_hip.h
  declares;
* the host-side validators return the status codes that mirror the
  reference's ``ValueError`` guards (fused_decode.py:323-338,
  full_channel_flash_decoding.py:173-178) for descriptors without device
  memory;
* the split planner covers every token exactly once.
"""
import ctypes
import os
import re

import pytest

from rotatek_amd import _lib

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "rotatek_hip.h")


def _declared_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(rk_[a-z0-9_]+)\s*\(", text)))


def test_library_exports_every_declared_symbol():
    lib = _lib.load()
    names = _declared_functions()
    assert len(names) >= 9
    missing = [n for n in names if not hasattr(lib, n)]
    assert not missing, missing


def test_abi_version_and_strerror():
    lib = _lib.load()
    assert lib.rk_abi_version() == _lib.ABI_VERSION == 3
    assert _lib.strerror(0) == "success"
    assert "H_kv" in _lib.strerror(-5)
    assert _lib.strerror(-999) == "unknown status"


def test_descriptor_matches_the_header_layout():
    """desc() packs rk_tensor in one step: its bytes equal a field-by-field
    fill (data, dtype code, ndim, then shape and element strides, zeros past
    ndim) for every rank, dtype, view and empty tensor; a NULL data pointer
    for empty tensors; rank > 4 and unknown dtypes raise ValueError."""
    import torch

    assert ctypes.sizeof(_lib.RkTensor) == 80
    n = 0
    for dt in (torch.float16, torch.bfloat16, torch.float32, torch.float64, torch.uint8, torch.int32,
               torch.int64):
        for shape in [(), (5,), (3, 4), (2, 3, 4), (2, 3, 4, 5), (0, 4), (2, 0, 3, 1)]:
            t = torch.zeros(shape, dtype=dt)
            views = [t]
            if t.dim() > 1:
                views.append(t.transpose(0, -1))
            if t.dim() > 0 and t.shape[-1] > 1:
                views.append(t[..., ::2])
            for v in views:
                want = _lib.RkTensor()
                want.data = v.data_ptr() if v.numel() > 0 else 0
                want.dtype = _lib._DTYPES[dt]
                want.ndim = v.dim()
                for i in range(v.dim()):
                    want.shape[i] = v.shape[i]
                    want.stride[i] = v.stride(i)
                assert bytes(_lib.desc(v)) == bytes(want), (dt, shape, v.stride())
                n += 1
    assert n > 100
    assert _lib.desc(None) is None
    with pytest.raises(ValueError):
        _lib.desc(torch.zeros(1, 1, 1, 1, 1))
    with pytest.raises(ValueError):
        _lib.desc(torch.zeros(2, dtype=torch.complex64))


def _t(shape, dtype=_lib.RK_F16, strides=None):
    d = _lib.RkTensor()
    d.data = 0
    d.dtype = dtype
    d.ndim = len(shape)
    if strides is None:
        strides, acc = [], 1
        for s in reversed(shape):
            strides.insert(0, acc)
            acc *= s
    for i, (s, st) in enumerate(zip(shape, strides)):
        d.shape[i] = s
        d.stride[i] = st
    return d


def _rot_check(B=2, Hq=8, Hkv=4, D=128, Dk=32, S_v=100, S_f=20, G=None, mask_dtype=_lib.RK_U8,
               q_shape=None, R_shape=None, dtype=_lib.RK_F16, out=True, policy=1):
    G = Hq // Hkv if G is None else G
    q = _t(q_shape or (B, Hq, D), dtype)
    R = _t(R_shape or (B, Hkv, D, Dk), dtype)
    dm = _t((B, Hkv, D), dtype)
    kf = _t((B, Hkv, S_f, D), dtype)
    vf = _t((B, Hkv, S_f, D), dtype)
    mask = _t((B, S_f), mask_dtype)
    ks = _t((B, Hkv, S_v, Dk), dtype)
    vs = _t((B, Hkv, S_v, D), dtype)
    o = _t((B, Hq, D), dtype) if out else None
    need = ctypes.c_size_t(0)
    args = [ctypes.byref(x) for x in (q, R, dm, kf, vf, mask, ks, vs)]
    st = _lib.load().rk_rotatek_decode_check(*args, G, ctypes.byref(o) if o else None, policy, 256,
                                             ctypes.byref(need))
    return st, need.value


def test_rotatek_check_ok_and_workspace():
    st, need = _rot_check()
    assert st == 0 and need > 0


@pytest.mark.parametrize("kw,code", [
    (dict(q_shape=(2, 8)), -2),                 # q rank != 3
    (dict(R_shape=(2, 4, 128)), -2),            # R rank != 4
    (dict(mask_dtype=_lib.RK_F16), -3),         # mask not uint8
    (dict(G=3), -5),                            # H_q / G != H_kv
    (dict(D=64), 0),                            # any head_dim 1..128
    (dict(D=80), 0),
    (dict(D=1), 0),
    (dict(D=129), -6),                          # head_dim past 128
    (dict(D=0), -6),
    (dict(dtype=_lib.RK_F64), -3),              # fp64 not supported
    (dict(Dk=129), -7),
    (dict(Dk=0), 0),                            # every channel pruned: bias-only visual logits
    (dict(policy=7), -10),
])
def test_rotatek_check_errors(kw, code):
    st, _ = _rot_check(**kw)
    assert st == code, (st, _lib.strerror(st))


@pytest.mark.parametrize("which,ss", [
    ("v_sparse", ((1 << 31) - 8 - 127) // (63 + 32) + 1),  # span fits 2^31, span + 32 rows does not
    ("k_sparse", 1 << 26),                                   # token stride at the bound
    ("k_full", 1 << 26),
    ("v_full", ((1 << 31) - 8 - 127) // (15 + 32) + 1),
])
def test_rotatek_check_refuses_strides_beyond_32bit_offsets(which, ss):
    """A K/V descriptor whose within-head span plus 32 rows reaches 2^31
    elements, or whose token stride reaches 2^26, is refused with
    RK_ERR_STRIDE by the host-side check (the kernels form 32-bit byte
    offsets of rows up to 31 past a block's first row before clamping
    them), so the launching entry, which runs the same validation first,
    never launches such a call."""
    B, Hq, Hkv, D, Dk, S_v, S_f = 1, 4, 4, 128, 32, 64, 16
    names = ("q_full", "R_partial", "delta_mu", "k_full", "v_full", "mask_full", "k_sparse", "v_sparse")
    shapes = dict(q_full=(B, Hq, D), R_partial=(B, Hkv, D, Dk), delta_mu=(B, Hkv, D), k_full=(B, Hkv, S_f, D),
                  v_full=(B, Hkv, S_f, D), mask_full=(B, S_f), k_sparse=(B, Hkv, S_v, Dk),
                  v_sparse=(B, Hkv, S_v, D))
    d = {k: _t(shapes[k], _lib.RK_U8 if k == "mask_full" else _lib.RK_F16) for k in names}
    t = d[which]
    t.stride[2] = ss
    t.stride[1] = ss * t.shape[2]
    t.stride[0] = t.stride[1] * t.shape[1]
    o = _t((B, Hq, D))
    need = ctypes.c_size_t(0)
    st = _lib.load().rk_rotatek_decode_check(*[ctypes.byref(d[k]) for k in names], 1, ctypes.byref(o), 0, 256,
                                             ctypes.byref(need))
    assert st == _lib.RK_ERR_STRIDE, _lib.strerror(st)
    # one element of stride less (v_sparse: the largest span that fits) is accepted
    if which == "v_sparse":
        t.stride[2] = ss - 1
        t.stride[1] = t.stride[2] * t.shape[2]
        t.stride[0] = t.stride[1] * t.shape[1]
        st = _lib.load().rk_rotatek_decode_check(*[ctypes.byref(d[k]) for k in names], 1, ctypes.byref(o), 0,
                                                 256, ctypes.byref(need))
        assert st == 0, _lib.strerror(st)


def test_dense_check_refuses_strides_beyond_32bit_offsets():
    q, o = _t((1, 4, 128)), _t((1, 4, 128))
    k = _t((1, 4, 16, 128), strides=(4 * 16 << 26, 16 << 26, 1 << 26, 1))
    v = _t((1, 4, 16, 128))
    need = ctypes.c_size_t(0)
    st = _lib.load().rk_full_channel_decode_check(ctypes.byref(q), ctypes.byref(k), ctypes.byref(v), 1,
                                                  ctypes.byref(o), 0, 256, ctypes.byref(need))
    assert st == _lib.RK_ERR_STRIDE, _lib.strerror(st)


def test_rotatek_check_fp32():
    """fp32 q/K/V/out (the reference's kernels accept it) plan one unit per
    query head; mixing fp32 q with 16-bit K/V is a dtype error."""
    st, need = _rot_check(dtype=_lib.RK_F32)
    assert st == 0 and need > 0
    p = _lib.plan_decode(2, 8, 4, 32, 100, 20, elem_bytes=4, policy=_lib.RK_POLICY_PAPER)
    assert p["heads_per_unit"] == 1 and p["units"] == 2 * 8
    lib = _lib.load()
    B, Hq, Hkv, D = 2, 8, 4, 128
    q, R = _t((B, Hq, D), _lib.RK_F32), _t((B, Hkv, D, 32), _lib.RK_F32)
    kf, vf = _t((B, Hkv, 10, D)), _t((B, Hkv, 10, D))
    ks, vs = _t((B, Hkv, 50, 32)), _t((B, Hkv, 50, D))
    st = lib.rk_rotatek_decode_check(*[ctypes.byref(x) for x in (q, R)], None,
                                     *[ctypes.byref(x) for x in (kf, vf)], None,
                                     *[ctypes.byref(x) for x in (ks, vs)], 2, None, 1, 256, None)
    assert st == -3


def test_varlen_rejects_fp32():
    """The span cache decode is 16-bit only: fp32 is a dtype error."""
    lib = _lib.load()
    B, Hq, Hkv, D = 1, 4, 4, 128
    f = _lib.RK_F32
    q, R, o = _t((B, Hq, D), f), _t((B, Hkv, D, 32), f), _t((B, Hq, D), f)
    kf, vb = _t((B, Hkv, 10, D), f), _t((B, Hkv, 60, D), f)
    ks, vs = _t((B, Hkv, 50, 32), f), _t((B, Hkv, 50, D), f)
    lens = (ctypes.c_int32 * 1)()
    st = lib.rk_rotatek_decode_varlen(ctypes.byref(q), ctypes.byref(R), None, ctypes.byref(kf), ctypes.byref(vb),
                                      4, 50, None, ctypes.byref(ks), ctypes.byref(vs), 1, None, None,
                                      ctypes.cast(lens, ctypes.c_void_p), ctypes.byref(o), 1, None, 0, None)
    assert st == -3


def test_rotatek_check_shape_mismatch():
    lib = _lib.load()
    B, Hq, Hkv, D = 2, 8, 4, 128
    q, R = _t((B, Hq, D)), _t((B, Hkv, D, 32))
    kf, vf = _t((B, Hkv, 10, D)), _t((B, Hkv, 11, D))        # S_f disagree
    mask = _t((B, 10), _lib.RK_U8)
    ks, vs = _t((B, Hkv, 50, 32)), _t((B, Hkv, 50, D))
    st = lib.rk_rotatek_decode_check(*[ctypes.byref(x) for x in (q, R, R, kf, vf, mask, ks, vs)], 2,
                                     None, 1, 256, None)
    assert st == -4 or st == -2  # delta_mu passed with the wrong rank, or S_f mismatch
    dm = _t((B, Hkv, D))
    st = lib.rk_rotatek_decode_check(*[ctypes.byref(x) for x in (q, R, dm, kf, vf, mask, ks, vs)], 2,
                                     None, 1, 256, None)
    assert st == -4


def test_rotatek_check_null_descriptor():
    lib = _lib.load()
    st = lib.rk_rotatek_decode_check(None, None, None, None, None, None, None, None, 1, None, 1, 256,
                                     None)
    assert st == -1


def test_dense_check():
    lib = _lib.load()
    q, k, v, o = _t((2, 8, 128)), _t((2, 4, 64, 128)), _t((2, 4, 64, 128)), _t((2, 8, 128))
    need = ctypes.c_size_t(0)
    args = [ctypes.byref(x) for x in (q, k, v)]
    assert lib.rk_full_channel_decode_check(*args, 2, ctypes.byref(o), 0, 256, ctypes.byref(need)) == 0
    assert need.value > 0
    assert lib.rk_full_channel_decode_check(*args, 3, None, 0, 256, None) == -5
    kbad = _t((2, 4, 64, 96))
    assert lib.rk_full_channel_decode_check(ctypes.byref(q), ctypes.byref(kbad), ctypes.byref(v), 2,
                                            None, 0, 256, None) == -4
    q2 = _t((2, 8))
    assert lib.rk_full_channel_decode_check(ctypes.byref(q2), ctypes.byref(k), ctypes.byref(v), 2,
                                            None, 0, 256, None) == -2


def test_launch_without_workspace_fails_cleanly():
    """The launch entry validates the workspace before any HIP call."""
    lib = _lib.load()
    q, k, v, o = _t((2, 8, 128)), _t((2, 4, 64, 128)), _t((2, 4, 64, 128)), _t((2, 8, 128))
    st = lib.rk_full_channel_decode(ctypes.byref(q), ctypes.byref(k), ctypes.byref(v), 2,
                                    ctypes.byref(o), 0, None, 0, None)
    # no device here -> NO_DEVICE; with a device -> WORKSPACE
    assert st in (-9, -12)


@pytest.mark.parametrize("shape", [
    (32, 32, 32, 32, 14000, 2000), (1, 32, 32, 32, 15360, 640), (16, 28, 4, 32, 30720, 2048),
    (8, 28, 4, 16, 12001, 61), (1, 4, 4, 64, 1, 1), (3, 8, 2, 128, 0, 77), (2, 8, 8, 8, 300, 0),
    (1, 64, 2, 32, 500, 40), (2, 4, 4, 32, 0, 0), (8, 28, 4, 32, 4097, 61), (8, 28, 4, 64, 4097, 60),
    (3, 12, 4, 32, 2049, 17), (5, 20, 4, 24, 9001, 300), (4, 32, 8, 32, 3001, 100), (2, 16, 16, 32, 2500, 60),
])
@pytest.mark.parametrize("policy", [0, 1])
def test_plan_covers_every_token(shape, policy):
    B, Hq, Hkv, Dk, S_v, S_f = shape
    p = _lib.plan_decode(B, Hq, Hkv, Dk, S_v, S_f, policy=policy)
    G = Hq // Hkv
    if policy == 1:
        assert p["heads_per_unit"] == min(G, 16) and p["units"] == B * Hkv * -(-G // 16)
    else:
        assert p["heads_per_unit"] == 1 and p["units"] == B * Hq
    if S_v > 0:
        # visual chunks: n_fast of chunk_fast tokens, then chunk_vis each;
        # whole 32-token blocks in a chunk-major grid, else 128-token ones
        nf, cf, cv, wg = p["n_fast"], p["chunk_fast"], p["chunk_vis"], p["wg_vis"]
        align = 32 if p["chunk_major"] else 128
        assert cv % align == 0 and cf % align == 0 and 0 <= nf < wg
        assert nf == 0 or (p["chunk_major"] and cf > cv)
        assert nf * cf + (wg - nf) * cv >= S_v and nf * cf + (wg - nf - 1) * cv < S_v
    if S_f > 0:
        wg, ch = p["wg_full"], p["chunk_full"]
        assert ch % 128 == 0 and wg * ch >= S_f and (wg - 1) * ch < S_f
    assert p["wg_vis"] + p["wg_full"] >= 1
    assert p["grid"] == p["units"] * (p["wg_vis"] + p["wg_full"])
    if p["chunk_major"]:
        assert p["grid"] <= 2 * 256


def _check_plan(p, B, Hq, Hkv, Dk, S_v, S_f, policy, elem_bytes, cus):
    """Invariants of any decode plan: units, exact token coverage by the
    chunks, the grid, one round for chunk-major grids, and one workgroup per
    CU for the one-slot plans."""
    G = Hq // Hkv
    if policy == 1:  # blocks of up to 16 query heads (fp32: 8)
        hmax = 8 if elem_bytes == 4 else 16
        assert p["heads_per_unit"] == min(G, hmax) and p["units"] == B * Hkv * -(-G // hmax)
    else:
        assert p["heads_per_unit"] == 1 and p["units"] == B * Hq
    if S_v > 0:
        nf, cf, cv, wg = p["n_fast"], p["chunk_fast"], p["chunk_vis"], p["wg_vis"]
        assert cv > 0 and cv % 32 == 0 and 0 <= nf < wg and (nf == 0 or (p["chunk_major"] and cf > cv))
        assert nf * cf + (wg - nf) * cv >= S_v and nf * cf + (wg - nf - 1) * cv < S_v
    else:
        assert p["wg_vis"] == 0
    if S_f > 0:
        assert p["chunk_full"] % 128 == 0 and p["wg_full"] * p["chunk_full"] >= S_f
        assert (p["wg_full"] - 1) * p["chunk_full"] < S_f
    assert p["wg_vis"] + p["wg_full"] >= 1
    assert p["grid"] == p["units"] * (p["wg_vis"] + p["wg_full"])
    if p["chunk_major"]:
        assert elem_bytes == 2 and S_v > 0 and p["grid"] <= 2 * cus
    assert p["workspace_bytes"] >= p["grid"] * p["heads_per_unit"] * 640


def test_plan_invariants_on_random_shapes():
    """The planner's rules (rounds, span shares, chunk-major short rounds,
    enlarged first chunks, one workgroup per CU for small rounds and for
    fp32) on 600 seeded random shapes, both policies, both element sizes,
    two CU counts and every planner setting, checked for the plan
    invariants; the default plan never exceeds the two-slot plan's grid."""
    import random
    rng = random.Random(2024)
    try:
        for _ in range(600):
            Hkv = rng.choice([1, 2, 4, 8, 32])
            G = rng.choice([1, 1, 2, 4, 7, 8, 16, 20])
            B = rng.choice([1, 2, 3, 8, 16, 32])
            Dk = rng.choice([0, 8, 16, 32, 48, 64, 128])
            S_v = rng.choice([0, 1, 31, 200, 1025, 2304, 4097, 8000, 12001, 30720])
            S_f = rng.choice([0, 1, 60, 128, 640, 2000])
            if S_v + S_f == 0:
                S_f = 5
            policy, eb, cus = rng.choice([0, 1]), rng.choice([2, 2, 4]), rng.choice([256, 304])
            skew = rng.choice([0, 1000, 1300])
            _lib.set_decode_skew(skew)
            _lib.set_decode_tuning(0, 0, 2)
            two = _lib.plan_decode(B, Hkv * G, Hkv, Dk, S_v, S_f, eb, policy, cus)
            _check_plan(two, B, Hkv * G, Hkv, Dk, S_v, S_f, policy, eb, cus)
            _lib.set_decode_tuning(0, 0, -1)
            dflt = _lib.plan_decode(B, Hkv * G, Hkv, Dk, S_v, S_f, eb, policy, cus)
            _check_plan(dflt, B, Hkv * G, Hkv, Dk, S_v, S_f, policy, eb, cus)
            assert dflt["grid"] <= two["grid"]
            if dflt != two:  # a one-per-CU plan: one workgroup per CU, one round
                assert dflt["grid"] <= cus and dflt["n_fast"] == 0
    finally:
        _lib.set_decode_skew(1300)
        _lib.set_decode_tuning(0, 0, -1)


def test_planner_knobs_read_once_per_plan():
    """The planner knobs are process-wide atomics that each plan reads once:
    a byte cap set below the floor plans as the floor, and threads that flip
    the knobs while others plan (ctypes drops the GIL around each call) only
    ever get plans that satisfy the plan invariants."""
    import random
    import threading
    shape = (8, 28, 4, 32, 12001, 61, 2, 1, 256)
    try:
        _lib.set_decode_tuning(1 << 20, 1 << 20, 0)
        want = _lib.plan_decode(*shape)
        _lib.set_decode_tuning(1 << 20, 4096, 0)
        assert _lib.plan_decode(*shape) == want
        _lib.set_decode_tuning(64 << 10, 512 << 10, -1)

        stop, errors = threading.Event(), []

        def flip():
            i = 0
            while not stop.is_set():
                _lib.set_decode_tuning((64 << 10) << (i % 2), (512 << 10) << (i % 3), 2 if i % 2 else -1)
                _lib.set_decode_skew((1000, 1300, 0)[i % 3])
                i += 1

        def plan(seed):
            rng = random.Random(seed)
            try:
                for _ in range(1500):
                    Hkv, G = rng.choice([1, 4, 8]), rng.choice([1, 7])
                    B, Dk = rng.choice([1, 8, 32]), rng.choice([16, 32, 64])
                    S_v, S_f = rng.choice([0, 200, 4097, 12001]), rng.choice([1, 61, 2000])
                    pol, eb = rng.choice([0, 1]), rng.choice([2, 4])
                    p = _lib.plan_decode(B, Hkv * G, Hkv, Dk, S_v, S_f, eb, pol, 256)
                    _check_plan(p, B, Hkv * G, Hkv, Dk, S_v, S_f, pol, eb, 256)
            except AssertionError as e:  # reported from the main thread
                errors.append(e)

        threads = [threading.Thread(target=flip)] + [threading.Thread(target=plan, args=(s,)) for s in range(3)]
        for t in threads:
            t.start()
        for t in threads[1:]:
            t.join()
        stop.set()
        threads[0].join()
        assert not errors, errors[0]
    finally:
        _lib.set_decode_skew(1300)
        _lib.set_decode_tuning(64 << 10, 512 << 10, -1)


# ----------------------------------------------------------------- prefill ABI
def _cov_check(shape=(2, 4, 300, 128), dtype=_lib.RK_BF16, cov_shape=None, mean_shape=None):
    lib = _lib.load()
    k = _t(shape, dtype)
    B, H, _, D = shape
    c = _t(cov_shape or (B, H, D, D), _lib.RK_F32)
    m = _t(mean_shape or (B, H, D), _lib.RK_F32)
    need = ctypes.c_size_t(0)
    st = lib.rk_key_covariance_check(ctypes.byref(k), ctypes.byref(m), ctypes.byref(c), 256, ctypes.byref(need))
    return st, need.value


def test_covariance_check():
    st, need = _cov_check()
    assert st == 0 and need > 0
    assert _cov_check(shape=(2, 4, 300, 64))[0] == 0             # any head_dim 1..128
    assert _cov_check(shape=(2, 4, 300, 1))[0] == 0
    assert _cov_check(shape=(2, 4, 300, 129))[0] == -6
    assert _cov_check(shape=(2, 4, 300, 64), cov_shape=(2, 4, 128, 128))[0] == -4
    assert _cov_check(dtype=_lib.RK_F32)[0] == 0                  # fp32 Keys
    assert _cov_check(dtype=_lib.RK_F64)[0] == -3
    assert _cov_check(cov_shape=(2, 4, 128, 64))[0] == -4
    assert _cov_check(mean_shape=(2, 3, 128))[0] == -4


def test_rotate_and_select_validation():
    lib = _lib.load()
    k = _t((1, 2, 50, 128), _lib.RK_F16)
    R = _t((1, 2, 128, 32), _lib.RK_F16)
    out_bad = _t((1, 2, 50, 16), _lib.RK_F16)
    assert lib.rk_rotate_keys(ctypes.byref(k), ctypes.byref(R), ctypes.byref(out_bad), None) == -4
    out_dt = _t((1, 2, 50, 32), _lib.RK_BF16)
    assert lib.rk_rotate_keys(ctypes.byref(k), ctypes.byref(R), ctypes.byref(out_dt), None) == -3
    sc = _t((1, 2, 128), _lib.RK_F32)
    idx = _t((1, 2, 32), _lib.RK_I64)
    assert lib.rk_topk_channels(ctypes.byref(sc), 32, ctypes.byref(idx), None, None) == -3
    sc = _t((1, 2, 128), _lib.RK_F64)
    assert lib.rk_topk_channels(ctypes.byref(sc), 129, ctypes.byref(idx), None, None) == -7
    Rf = _t((1, 2, 128, 128), _lib.RK_F32)
    mean = _t((1, 2, 128), _lib.RK_F32)
    Ro = _t((1, 2, 128, 32), _lib.RK_F64)      # output must be F16 / BF16 / F32
    dm = _t((1, 2, 128), _lib.RK_F64)
    assert lib.rk_gather_rotation(ctypes.byref(Rf), ctypes.byref(idx), ctypes.byref(mean), ctypes.byref(Ro),
                                  ctypes.byref(dm), None) == -3
    Ro, dm = _t((1, 2, 128, 32), _lib.RK_F32), _t((1, 2, 128), _lib.RK_F32)
    assert lib.rk_gather_rotation(ctypes.byref(Rf), ctypes.byref(idx), ctypes.byref(mean), ctypes.byref(Ro),
                                  ctypes.byref(dm), None) == -1    # fp32 accepted; no device memory
    R80 = _t((1, 2, 80, 32), _lib.RK_F16)
    assert lib.rk_rotate_keys(ctypes.byref(k), ctypes.byref(R80), ctypes.byref(out_dt), None) == -4  # D mismatch
    need = ctypes.c_size_t(0)
    scores = _t((1, 2, 128), _lib.RK_F64)
    assert lib.rk_channel_scores_check(ctypes.byref(k), ctypes.byref(Rf), ctypes.byref(scores), 256,
                                       ctypes.byref(need)) == 0
    assert need.value > 0


# ------------------------------------------------------------- span cache ABI
def _varlen(S_cap=40, gap_at=10, gap=100, v_rows=None, lens=1, B=2, Hq=8, Hkv=4, new=None):
    lib = _lib.load()
    kn = vn = None
    if new is not None:
        kn, vn = (ctypes.byref(_t(s)) if s else None for s in new)
    q, R, dm = _t((B, Hq, 128)), _t((B, Hkv, 128, 32)), _t((B, Hkv, 128))
    kf = _t((B, Hkv, S_cap, 128))
    vb = _t((B, Hkv, S_cap + gap if v_rows is None else v_rows, 128))
    ks, vs, o = _t((B, Hkv, gap, 32)), _t((B, Hkv, gap, 128)), _t((B, Hq, 128))
    return lib.rk_rotatek_decode_varlen(ctypes.byref(q), ctypes.byref(R), ctypes.byref(dm), ctypes.byref(kf),
                                        ctypes.byref(vb), gap_at, gap, None, ctypes.byref(ks),
                                        ctypes.byref(vs), Hq // Hkv, kn, vn, lens, ctypes.byref(o), 1, None, 0,
                                        None)


def test_varlen_decode_validation():
    # argument errors come back before any device query
    assert _varlen(v_rows=139) == -4               # V rows != capacity + gap
    assert _varlen(gap_at=41) == -10               # gap start past the capacity
    assert _varlen(gap=-1, v_rows=39) == -10
    assert _varlen(lens=None) == -1                # device lengths required
    assert _varlen(new=((2, 4, 1, 128), None)) == -1                  # k_new without v_new
    assert _varlen(new=((2, 4, 2, 128), (2, 4, 2, 128))) == -4        # more than one token
    assert _varlen(new=((2, 4, 1, 128), (2, 4, 1, 128))) == -1        # well-formed, but no device memory
    # well-formed, no device / no workspace
    assert _varlen() in (-9, -12)


def test_append_kv_validation():
    lib = _lib.load()
    kn, vn = _t((2, 4, 1, 128)), _t((2, 4, 1, 128))
    kb, vb = _t((2, 4, 64, 128)), _t((2, 4, 64, 128))
    r = ctypes.byref
    assert lib.rk_append_kv(r(kn), r(vn), r(kb), r(vb), None, None) == -1
    two = _t((2, 4, 2, 128))
    assert lib.rk_append_kv(r(two), r(vn), r(kb), r(vb), 1, None) == -4       # more than one token
    vb_short = _t((2, 4, 63, 128))
    assert lib.rk_append_kv(r(kn), r(vn), r(kb), r(vb_short), 1, None) == -4
    kb_bf = _t((2, 4, 64, 128), _lib.RK_BF16)
    assert lib.rk_append_kv(r(kn), r(vn), r(kb_bf), r(vb), 1, None) == -3
    assert lib.rk_append_kv(r(kn), None, r(kb), r(vb), 1, None) == -1          # V given for one side only
    empty_k, empty_b = _t((0, 4, 1, 128)), _t((0, 4, 64, 128))
    assert lib.rk_append_kv(r(empty_k), None, r(empty_b), None, 1, None) == 0   # nothing to do


def test_power_iteration_validation():
    lib = _lib.load()
    r = ctypes.byref
    cov, v0, out = _t((2, 4, 128, 128), _lib.RK_F32), _t((2, 4, 128, 16), _lib.RK_F32), _t((2, 4, 128, 16), _lib.RK_F32)
    assert lib.rk_power_iteration(r(cov), r(v0), r(out), 5, 1e-4, None, None) == -1        # no device memory
    bad = _t((2, 4, 128, 16), _lib.RK_F16)
    assert lib.rk_power_iteration(r(cov), r(bad), r(out), 5, 1e-4, None, None) == -3
    wide = _t((2, 4, 128, 129), _lib.RK_F32)
    assert lib.rk_power_iteration(r(cov), r(wide), r(wide), 5, 1e-4, None, None) == -7     # k > 128
    w96 = _t((2, 4, 128, 96), _lib.RK_F32)
    assert lib.rk_power_iteration(r(cov), r(w96), r(w96), 5, 1e-4, None, None) == -1       # 96 is valid
    c64 = _t((2, 4, 64, 64), _lib.RK_F32)
    assert lib.rk_power_iteration(r(c64), r(v0), r(out), 5, 1e-4, None, None) == -4      # V0 rows != D
    v64, o64 = _t((2, 4, 64, 16), _lib.RK_F32), _t((2, 4, 64, 16), _lib.RK_F32)
    assert lib.rk_power_iteration(r(c64), r(v64), r(o64), 5, 1e-4, None, None) == -1     # D = 64 is valid
    w65 = _t((2, 4, 64, 65), _lib.RK_F32)
    assert lib.rk_power_iteration(r(c64), r(w65), r(w65), 5, 1e-4, None, None) == -7     # k > D
    c129 = _t((2, 4, 129, 129), _lib.RK_F32)
    assert lib.rk_power_iteration(r(c129), r(v0), r(out), 5, 1e-4, None, None) == -6
    o2 = _t((2, 4, 128, 8), _lib.RK_F32)
    assert lib.rk_power_iteration(r(cov), r(v0), r(o2), 5, 1e-4, None, None) == -4
    assert lib.rk_power_iteration(r(cov), r(v0), r(out), -1, 1e-4, None, None) == -10


def test_query_weight_validation():
    lib = _lib.load()
    r = ctypes.byref
    cov, out = _t((2, 4, 128, 128), _lib.RK_F32), _t((2, 4, 128, 128), _lib.RK_F32)
    q = _t((2, 28, 50, 128), _lib.RK_BF16)
    assert lib.rk_query_weight(r(cov), r(q), 7, 32, r(out), None) == -1      # no device memory
    assert lib.rk_query_weight(r(cov), r(q), 5, 32, r(out), None) == -5      # H_q != H_kv * G
    assert lib.rk_query_weight(r(cov), r(q), 7, 33, r(out), None) == -10     # window above 32
    q32 = _t((2, 28, 50, 128), _lib.RK_F32)
    assert lib.rk_query_weight(r(cov), r(q32), 7, 32, r(out), None) == -1    # fp32 queries accepted
    q64 = _t((2, 28, 50, 128), _lib.RK_F64)
    assert lib.rk_query_weight(r(cov), r(q64), 7, 32, r(out), None) == -3


def test_think_validation():
    lib = _lib.load()
    need = ctypes.c_size_t(0)

    def chk(keys=(2, 4, 50, 128), q=(2, 8, 32, 128), heads=4, prune=96, kc=None, mask=(2, 4, 128),
            kdt=_lib.RK_BF16, qdt=_lib.RK_BF16, mdt=_lib.RK_U8):
        kc = kc or (keys[0], keys[1], keys[2], 128 - prune)
        d = [_t(keys, kdt), _t(q, qdt), _t(kc, kdt), _t(mask, mdt)]
        return lib.rk_think_score_and_compact_check(ctypes.byref(d[0]), ctypes.byref(d[1]), heads, prune,
                                                    ctypes.byref(d[2]), ctypes.byref(d[3]), 256,
                                                    ctypes.byref(need))

    assert chk() == 0 and need.value > 0
    assert chk(prune=0) == 0 and chk(prune=128) == 0
    assert chk(prune=129, kc=(2, 4, 50, 1)) == _lib.RK_ERR_KEEP_DIM
    assert chk(heads=3) == _lib.RK_ERR_HEADS
    assert chk(q=(2, 6, 32, 128), heads=4) == _lib.RK_ERR_HEADS
    # any head dim 1..128, the same in keys, queries and the mask
    assert chk(keys=(2, 4, 50, 64), q=(2, 8, 32, 64), kc=(2, 4, 50, 40), prune=24, mask=(2, 4, 64)) == 0
    assert chk(keys=(2, 4, 50, 5), q=(2, 8, 32, 5), kc=(2, 4, 50, 5), prune=0, mask=(2, 4, 5)) == 0
    assert chk(keys=(2, 4, 50, 64), q=(2, 8, 32, 64), kc=(2, 4, 50, 40), prune=24) == _lib.RK_ERR_SHAPE
    assert chk(keys=(2, 4, 50, 64), kc=(2, 4, 50, 40), prune=24, mask=(2, 4, 64)) == _lib.RK_ERR_SHAPE
    assert chk(keys=(2, 4, 50, 64), q=(2, 8, 32, 64), kc=(2, 4, 50, 1), prune=65,
               mask=(2, 4, 64)) == _lib.RK_ERR_KEEP_DIM
    assert chk(keys=(2, 4, 50, 129), q=(2, 8, 32, 129), mask=(2, 4, 129)) == _lib.RK_ERR_HEAD_DIM
    assert chk(qdt=_lib.RK_F16) == _lib.RK_ERR_DTYPE
    assert chk(kc=(2, 4, 50, 33)) == _lib.RK_ERR_SHAPE
    assert chk(mask=(2, 4, 127)) == _lib.RK_ERR_SHAPE
    assert chk(mdt=_lib.RK_I32) == _lib.RK_ERR_DTYPE
    assert chk(kdt=_lib.RK_F32, qdt=_lib.RK_F32) == _lib.RK_ERR_DTYPE


def test_spark_validation():
    lib = _lib.load()
    need = ctypes.c_size_t(0)

    def chk(keys=(2, 4, 50, 128), q=(2, 28, 32, 128), groups=7, prune=96, kc=None, mask=None, pm=None,
            dt=_lib.RK_F16):
        B, H, S = keys[:3]
        kc = kc or (B, H, S, 128 - prune)
        mask = mask or (B, H, S, 128)
        pm = pm or (B, H, S, 1)
        d = [_t(keys, dt), _t(q, dt), _t(kc, dt), _t(mask, _lib.RK_U8), _t(pm, dt)]
        return lib.rk_spark_prune_check(ctypes.byref(d[0]), ctypes.byref(d[1]), groups, prune,
                                        *[ctypes.byref(x) for x in d[2:]], 256, ctypes.byref(need))

    assert chk() == 0 and need.value > 0
    assert chk(groups=1, q=(2, 4, 32, 128)) == 0
    assert chk(groups=6) == _lib.RK_ERR_HEADS
    assert chk(groups=0) == _lib.RK_ERR_HEADS
    assert chk(prune=-1, kc=(2, 4, 50, 129)) == _lib.RK_ERR_KEEP_DIM
    assert chk(mask=(2, 4, 50, 64)) == _lib.RK_ERR_SHAPE
    assert chk(mask=(2, 4, 128)) == _lib.RK_ERR_RANK
    assert chk(pm=(2, 4, 50, 2)) == _lib.RK_ERR_SHAPE
    assert chk(kc=(2, 4, 49, 32)) == _lib.RK_ERR_SHAPE
    assert chk(dt=_lib.RK_F32) == _lib.RK_ERR_DTYPE
    # head dim 80: keys, queries, mask and compact width follow it
    assert chk(keys=(2, 4, 50, 80), q=(2, 28, 32, 80), prune=60, kc=(2, 4, 50, 20), mask=(2, 4, 50, 80)) == 0
    assert chk(keys=(2, 4, 50, 80), q=(2, 28, 32, 80), prune=60, kc=(2, 4, 50, 20)) == _lib.RK_ERR_SHAPE
    assert chk(keys=(2, 4, 50, 80), prune=60, kc=(2, 4, 50, 20), mask=(2, 4, 50, 80)) == _lib.RK_ERR_SHAPE
    assert chk(keys=(2, 4, 50, 0), q=(2, 28, 32, 0), prune=0, kc=(2, 4, 50, 0),
               mask=(2, 4, 50, 0)) == _lib.RK_ERR_HEAD_DIM


def test_recover_validation():
    lib = _lib.load()
    B, H, Sp, Sv, St, Dk = 2, 4, 5, 40, 3, 32
    kp, kc, kt = _t((B, H, Sp, 128)), _t((B, H, Sv, Dk)), _t((B, H, St, 128))
    tm, sm, pm = _t((B, H, 128), _lib.RK_U8), _t((B, H, Sv, 128), _lib.RK_U8), _t((B, H, Sv, 1))
    out, vis = _t((B, H, Sp + Sv + St, 128)), _t((B, H, Sv, 128))
    r = ctypes.byref
    assert lib.rk_think_recover_check(r(kp), r(kc), r(kt), r(tm), r(out)) == 0
    assert lib.rk_think_recover_check(None, r(kc), None, r(tm), r(vis)) == 0
    assert lib.rk_think_recover_check(None, r(kc), None, r(tm), r(out)) == _lib.RK_ERR_SHAPE
    assert lib.rk_think_recover_check(r(kp), r(kc), r(kt), r(sm), r(out)) == _lib.RK_ERR_RANK
    assert lib.rk_spark_recover_check(r(kp), r(kc), r(kt), r(sm), r(pm), r(out)) == 0
    assert lib.rk_spark_recover_check(None, r(kc), None, r(sm), r(pm), r(vis)) == 0
    assert lib.rk_spark_recover_check(None, r(kc), None, r(sm), None, r(vis)) == _lib.RK_ERR_NULL
    bad_pm = _t((B, H, Sv, 1), _lib.RK_BF16)
    assert lib.rk_spark_recover_check(None, r(kc), None, r(sm), r(bad_pm), r(vis)) == _lib.RK_ERR_DTYPE
    wide = _t((B, H, Sv, 129))
    assert lib.rk_think_recover_check(None, wide, None, r(tm), r(vis)) == _lib.RK_ERR_SHAPE
    sel = _t((B, H, 128, Dk), _lib.RK_F32)
    assert lib.rk_channel_selection(r(tm), r(_t((B, H, 128, 0), _lib.RK_F32)), None) == _lib.RK_ERR_KEEP_DIM
    assert lib.rk_channel_selection(r(tm), r(_t((B, H, 64, Dk), _lib.RK_F32)), None) == _lib.RK_ERR_SHAPE
    assert lib.rk_channel_selection(r(tm), r(_t((B, H, 129, Dk), _lib.RK_F32)), None) == _lib.RK_ERR_HEAD_DIM
    assert lib.rk_channel_selection(r(sm), r(sel), None) == _lib.RK_ERR_RANK
    # head dim 64: mask [B,H,64], R [B,H,64,Dk <= 64], recovered rows of 64
    tm64, sm64 = _t((B, H, 64), _lib.RK_U8), _t((B, H, Sv, 64), _lib.RK_U8)
    # (valid shapes pass validation and stop at the descriptors' missing data)
    assert lib.rk_channel_selection(r(tm64), r(_t((B, H, 64, Dk), _lib.RK_F32)), None) == _lib.RK_ERR_NULL
    assert lib.rk_channel_selection(r(tm64), r(_t((B, H, 64, 65), _lib.RK_F32)), None) == _lib.RK_ERR_KEEP_DIM
    kp64, kt64 = _t((B, H, Sp, 64)), _t((B, H, St, 64))
    out64 = _t((B, H, Sp + Sv + St, 64))
    assert lib.rk_think_recover_check(r(kp64), r(kc), r(kt64), r(tm64), r(out64)) == 0
    assert lib.rk_spark_recover_check(r(kp64), r(kc), r(kt64), r(sm64), r(pm), r(out64)) == 0
    assert lib.rk_think_recover_check(r(kp), r(kc), r(kt64), r(tm64), r(out64)) == _lib.RK_ERR_SHAPE
    assert lib.rk_think_recover_check(r(kp64), r(kc), r(kt64), r(tm), r(out64)) == _lib.RK_ERR_SHAPE
    assert lib.rk_think_recover_check(None, r(_t((B, H, Sv, 65))), None, r(tm64),
                                      r(_t((B, H, Sv, 64)))) == _lib.RK_ERR_SHAPE


def test_plan_small_span_does_not_starve_the_other():
    """A prompt/text span too small for a workgroup of its own still gets
    one, but at two slots per unit it must not leave the visual span a
    single workgroup (the reference kernel-benchmark shape: B=32, 8 KV heads
    of 4 query heads, 16000 visual + 80 prompt/text tokens)."""
    p = _lib.plan_decode(32, 32, 8, 32, 16000, 80, policy=1)
    assert p["wg_full"] == 1 and p["wg_vis"] >= 2


def test_plan_gives_every_unit_several_workgroups():
    """With many units the planner adds rounds so each unit streams through
    at least 8 workgroups (while a workgroup keeps >= 64 KB)."""
    p = _lib.plan_decode(32, 32, 8, 32, 16000, 80, policy=1)
    assert p["wg_vis"] + p["wg_full"] >= 8
    # a small problem keeps its workgroups above the minimum size instead
    q = _lib.plan_decode(1, 4, 4, 32, 300, 50, policy=1)
    assert q["wg_vis"] + q["wg_full"] <= 4


def test_plan_keeps_one_round_when_the_extra_slot_saves_little():
    """Config 4 layer (B=8, 4 KV heads of 7, 12001 visual + 61 prompt/text,
    256 CUs): giving the visual span its full share would overflow the
    single round by 32 workgroups for a 6 % shorter workgroup, so the grid
    stays within 2 x 256 slots."""
    p = _lib.plan_decode(8, 28, 4, 32, 12001, 61, policy=1)
    assert p["grid"] <= 2 * 256


def test_plan_chunk_major_short_rounds():
    """One round of short workgroups launches chunk-major with 32-token
    chunks (config 4 layers, config 1); rounds of long workgroups (config 3)
    and multi-round grids (config 2, kp) keep the unit-major launch; at two
    workgroups per CU the first-dispatched chunks are enlarged only where
    workgroups stream <= 128 KB (config 4 at 4097 visual tokens)."""
    cfg4l = _lib.plan_decode(8, 28, 4, 32, 12001, 61, policy=1)
    assert cfg4l["chunk_major"] == 1 and cfg4l["n_fast"] == 0 and cfg4l["grid"] == 512
    try:
        _lib.set_decode_tuning(0, 0, 2)
        cfg4s = _lib.plan_decode(8, 28, 4, 32, 4097, 61, policy=1)
        assert cfg4s["chunk_major"] == 1 and cfg4s["n_fast"] == 256 // cfg4s["units"]
        assert cfg4s["chunk_fast"] > cfg4s["chunk_vis"]
    finally:
        _lib.set_decode_tuning(0, 0, -1)
    assert _lib.plan_decode(1, 32, 32, 32, 15360, 640, policy=0)["chunk_major"] == 1
    for shape, pol in (((16, 28, 4, 32, 30720, 2048), 1), ((32, 32, 32, 32, 14000, 2000), 0),
                       ((32, 32, 8, 32, 16000, 80), 1)):
        p = _lib.plan_decode(*shape, policy=pol)
        assert p["chunk_major"] == 0 and p["n_fast"] == 0 and p["chunk_vis"] % 128 == 0
    # fp32 (the VALU kernel) keeps the unit-major launch
    assert _lib.plan_decode(1, 32, 32, 32, 2304, 128, elem_bytes=4, policy=0)["chunk_major"] == 0
    try:
        _lib.set_decode_skew(1000)      # chunk-major, equal chunks
        p = _lib.plan_decode(8, 28, 4, 32, 4097, 61, policy=1)
        assert p["chunk_major"] == 1 and p["n_fast"] == 0
        _lib.set_decode_skew(0)         # unit-major
        p = _lib.plan_decode(8, 28, 4, 32, 4097, 61, policy=1)
        assert p["chunk_major"] == 0 and p["chunk_vis"] % 128 == 0
    finally:
        _lib.set_decode_skew(1300)


def test_plan_one_workgroup_per_cu_for_small_short_rounds():
    """Where a one-round chunk-major grid at two workgroups per CU would give
    each visual workgroup <= 128 KB, the planner takes one workgroup per CU
    of twice the tokens if that is still one chunk-major round (config 4 at
    4097 visual tokens, every keep; one query head per unit at 4000 tokens),
    and keeps two per CU otherwise: larger chunks (config 4 at 12001, config
    1) or a one-slot plan of two rounds (B=16 at 2049 tokens, which keeps the
    enlarged first-dispatched chunks).  A fixed count restores the two-slot
    plan."""
    for keep in (16, 32, 64):
        p = _lib.plan_decode(8, 28, 4, keep, 4097, 61, policy=1)
        assert p["chunk_major"] == 1 and p["n_fast"] == 0 and p["grid"] == 256, (keep, p)
        # multi-head units: the merge kernel
        assert p["single_launch"] == 0, (keep, p)
    p = _lib.plan_decode(1, 32, 32, 32, 4000, 640, policy=0)
    assert p["chunk_major"] == 1 and p["grid"] == 256 and p["single_launch"] == 1
    # units of one query head take one workgroup per CU up to 256 KB two-slot
    # chunks at <= 32 kept channels (8000 / 12000 tokens: 177 / 256 KB, not
    # 13000: 277 KB), up to 192 KB with more (keep 64, 8000 tokens: 209 KB)
    assert _lib.plan_decode(1, 32, 32, 32, 8000, 640, policy=0)["grid"] == 256
    assert _lib.plan_decode(1, 32, 32, 32, 12000, 640, policy=0)["grid"] == 256
    assert _lib.plan_decode(1, 32, 32, 32, 13000, 640, policy=0)["grid"] == 512
    assert _lib.plan_decode(1, 32, 32, 64, 8000, 640, policy=0)["grid"] == 512
    assert _lib.plan_decode(8, 28, 4, 32, 8001, 61, policy=1)["grid"] == 512   # GQA, 159 KB
    # fp32 (the VALU kernel): one workgroup per CU wherever that is still one
    # round (config 0: 320 -> 224 workgroups), else the two-slot plan
    for S_v, want in ((2304, 224), (1024, 160), (6000, 256), (8192, 448)):
        p = _lib.plan_decode(1, 32, 32, 32, S_v, 128, elem_bytes=4, policy=0)
        assert p["grid"] == want and p["chunk_major"] == 0, (S_v, p)
    assert _lib.plan_decode(2, 32, 32, 32, 1152, 128, elem_bytes=4, policy=0)["grid"] == 384
    # fp32 GQA: units of up to 8 query heads of one KV head (K / V read once
    # per unit), 16-bit: up to 16
    for G in (4, 7, 8, 12, 16):
        p4 = _lib.plan_decode(2, 4 * G, 4, 32, 3000, 64, elem_bytes=4, policy=1)
        assert p4["heads_per_unit"] == min(G, 8) and p4["head_blocks"] == -(-G // 8)
        assert p4["units"] == 2 * 4 * p4["head_blocks"]
        assert _lib.plan_decode(2, 4 * G, 4, 32, 3000, 64, elem_bytes=2, policy=1)["heads_per_unit"] == min(G, 16)
    for shape, pol in (((8, 28, 4, 32, 12001, 61), 1), ((1, 32, 32, 32, 15360, 640), 0)):
        assert _lib.plan_decode(*shape, policy=pol)["grid"] == 512
    p = _lib.plan_decode(16, 28, 4, 32, 2049, 61, policy=1)
    assert p["grid"] > 256 and p["chunk_major"] == 1 and p["n_fast"] == 256 // p["units"]
    try:
        _lib.set_decode_tuning(0, 0, 2)
        assert _lib.plan_decode(8, 28, 4, 32, 4097, 61, policy=1)["grid"] == 512
    finally:
        _lib.set_decode_tuning(0, 0, -1)
    assert _lib.plan_decode(8, 28, 4, 32, 4097, 61, policy=1)["grid"] == 256

