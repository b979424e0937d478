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
