"""The reference's import paths resolve to this package after
``install_as_rotatek()`` (CPU only: nothing is launched)."""
import importlib
import sys

import pytest


@pytest.fixture
def installed():
    saved = {k: v for k, v in sys.modules.items() if k == "rotatek" or k.startswith("rotatek.")}
    import rotatek_amd
    rotatek_amd.install_as_rotatek()
    yield
    for k in [k for k in sys.modules if k == "rotatek" or k.startswith("rotatek.")]:
        del sys.modules[k]
    sys.modules.update(saved)


def test_reference_import_paths_resolve(installed):
    import rotatek_amd
    from rotatek_amd import baselines, kernels, rotation
    ref = {
        ("rotatek.kernels", "rotatek_decode"): kernels.rotatek_decode,
        ("rotatek.kernels", "full_channel_decode"): kernels.full_channel_decode,
        ("rotatek.rotation", "power_iteration_gpu"): rotation.power_iteration_gpu,
        ("rotatek.baselines.think", "think_score_and_compact"): baselines.think_score_and_compact,
        ("rotatek.baselines.spark", "per_token_channel_prune"): baselines.per_token_channel_prune,
        ("rotatek.kernels.fused_decode", "rotatek_decode_fused_triton"):
            importlib.import_module("rotatek_amd.kernels.fused_decode").rotatek_decode_fused_triton,
        ("rotatek.kernels.gqa_decode", "rotatek_decode_gqa"):
            importlib.import_module("rotatek_amd.kernels.gqa_decode").rotatek_decode_gqa,
    }
    for (mod, name), fn in ref.items():
        assert getattr(importlib.import_module(mod), name) is fn, (mod, name)
    assert importlib.import_module("rotatek") is rotatek_amd


def test_pruner_exposes_every_reference_method():
    from rotatek_amd.pruning import ChannelPruner
    for m in ("update_think", "update_spark", "update_rotatek"):
        assert callable(getattr(ChannelPruner, m))


def test_spark_ratio_outside_unit_interval_is_a_value_error():
    from rotatek_amd.baselines import per_token_channel_prune
    import torch
    k = torch.zeros(1, 1, 4, 128)
    with pytest.raises(ValueError):
        per_token_channel_prune(torch.zeros(1, 1, 2, 128), k, 1.5)


@pytest.mark.parametrize("S,prompt,text,want", [
    (10, 3, 2, ([0, 1, 2], [3, 4, 5, 6, 7], [8, 9])),
    (10, 0, 0, ([], list(range(10)), [])),
    (10, 12, 2, (list(range(10)), [], [])),          # prompt clamped to S, nothing left for text
    (10, 4, 9, ([0, 1, 2, 3], [], [4, 5, 6, 7, 8, 9])),  # text clamped to what the prompt leaves
    (10, -3, -1, ([], list(range(10)), [])),          # negative lengths count as 0
    (0, 2, 2, ([], [], [])),
])
def test_split_spans_clamping(S, prompt, text, want):
    """Span split of kv_pruning_utils.py:26-35 on written-out cases."""
    import torch
    from rotatek_amd.pruning import _split_spans

    class Pruner:
        prompt_seqlen, query_seqlen = prompt, text

    x = torch.arange(S).view(1, 1, S, 1)
    got = tuple(t.flatten().tolist() for t in _split_spans(Pruner, x))
    assert got == want


@pytest.mark.parametrize("ratio,want", [(0.0, 128), (0.75, 32), (0.875, 16), (0.5, 64), (1.0, 0),
                                        (1.5, 0), (-0.25, 128), (0.999, 1)])
def test_keep_count(ratio, want):
    """keep = 128 - clamp(int(128 * ratio), 0, 128) (kv_pruning_utils.py:108)."""
    from rotatek_amd.pruning import keep_count
    assert keep_count(128, ratio) == want


@pytest.mark.parametrize("value,want", [("gqa", "rotatek_decode_gqa full_channel_decode_gqa"),
                                        (" Paper ", "rotatek_decode_fused full_channel_decode"),
                                        ("bogus", "ValueError")])
def test_kernel_family_from_environment(value, want):
    """ROTATEK_KERNEL is read once at import; an unknown family raises
    ValueError (rotatek/kernels/__init__.py:15-24).  Fresh interpreter each."""
    import os
    import subprocess
    import sys
    code = ("import rotatek_amd.kernels as k\n"
            "print(k.rotatek_decode.__name__, k.full_channel_decode.__name__)")
    env = dict(os.environ, ROTATEK_KERNEL=value)
    r = subprocess.run([sys.executable, "-c", code], env=env, capture_output=True, text=True,
                       cwd=os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
    if want == "ValueError":
        assert r.returncode != 0 and "ValueError" in r.stderr
    else:
        assert r.returncode == 0, r.stderr
        assert r.stdout.strip() == want


def _decode_args(**over):
    """CPU tensors shaped like a valid decode call (B=1, H_q=4, H_kv=2, Dk=8);
    the guards run before anything touches the device."""
    import torch
    a = dict(q_full=torch.zeros(1, 4, 128), R_partial=torch.zeros(1, 2, 128, 8), delta_mu=torch.zeros(1, 2, 128),
             k_full=torch.zeros(1, 2, 5, 128), v_full=torch.zeros(1, 2, 5, 128),
             mask_full=torch.ones(1, 5, dtype=torch.uint8), k_sparse=torch.zeros(1, 2, 7, 8),
             v_sparse=torch.zeros(1, 2, 7, 128), num_kv_groups=2)
    a.update(over)
    return a


@pytest.mark.parametrize("over", [
    dict(q_full="rank2"),                 # q_full not [B, H_q, D]       (fused_decode.py:323-324)
    dict(R_partial="rank3"),              # R_partial not rank 4         (fused_decode.py:325-326)
    dict(mask_full="bool"),               # mask not uint8               (fused_decode.py:327-328)
    dict(num_kv_groups=3),                # H_q / G != H_kv              (fused_decode.py:335-338)
])
@pytest.mark.parametrize("family", ["paper", "gqa"])
def test_rotatek_decode_guards_are_value_errors(over, family):
    import torch
    from rotatek_amd.kernels.fused_decode import rotatek_decode_fused
    from rotatek_amd.kernels.gqa_decode import rotatek_decode_gqa
    fn = rotatek_decode_fused if family == "paper" else rotatek_decode_gqa
    bad = {"rank2": torch.zeros(4, 128), "rank3": torch.zeros(1, 2, 128), "bool": torch.ones(1, 5, dtype=torch.bool)}
    over = {k: bad.get(v, v) if isinstance(v, str) else v for k, v in over.items()}
    with pytest.raises(ValueError):
        fn(**_decode_args(**over))


@pytest.mark.parametrize("q_shape,kv_dim", [((4, 128), 128), ((1, 4, 128), 64)])
def test_full_channel_decode_guards_are_value_errors(q_shape, kv_dim):
    """q rank != 3 or a K/V head size other than q's (full_channel_flash_decoding.py:173-178)."""
    import torch
    from rotatek_amd.kernels.full_channel_flash_decoding import full_channel_decode
    q = torch.zeros(*q_shape)
    k = torch.zeros(1, 4, 9, kv_dim)
    with pytest.raises(ValueError):
        full_channel_decode(q=q, k=k, v=k, num_kv_groups=1)


def test_decode_on_host_tensors_fails_loudly():
    """Well-formed host tensors are not silently computed on the CPU: the
    HIP kernels are the only implementation."""
    from rotatek_amd.kernels.fused_decode import rotatek_decode_fused
    with pytest.raises(RuntimeError):
        rotatek_decode_fused(**_decode_args())


def test_captured_cache_refuses_to_reallocate():
    """Once a decode graph holds the span buffers, an append past capacity
    raises instead of moving them (host tensors: no GPU needed)."""
    import torch

    from rotatek_amd.cache import DynamicCache
    cache = DynamicCache(reserve_tokens=0)
    B, H, D = 1, 2, 128
    cache._spans.append(__import__("rotatek_amd.cache", fromlist=["_Spans"])._Spans(
        torch.zeros(B, H, 3, D), torch.zeros(B, H, 3, D), torch.zeros(B, dtype=torch.int32), 1, 0, 2, False))
    cache._captured = True
    with pytest.raises(RuntimeError, match="reserve"):
        cache._grow(0, 4)
    with pytest.raises(RuntimeError, match="reserve"):
        cache.reserve(1)
