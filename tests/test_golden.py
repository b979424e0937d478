"""Known-answer fixtures (tests/golden/*.npz, written by
tests/golden/make_golden.py with explicit float64 loops independent of the
oracle).  CPU: the oracle reproduces them.  GPU: the HIP kernels reproduce
them (fp16 and bf16 inputs are exact, outputs within the north-star bars)."""
import os

import numpy as np
import pytest

from oracle import decode as od
from oracle import prefill as op

HERE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
DECODE = ["decode_mha.npz", "decode_gqa.npz", "decode_nobias.npz"]


def _load(name):
    return dict(np.load(os.path.join(HERE, name), allow_pickle=False))


@pytest.mark.parametrize("name", DECODE)
def test_oracle_decode_reproduces_golden(name):
    f = _load(name)
    got = od.rotatek_decode(f["q_full"], f["R_partial"], f.get("delta_mu"), f["k_full"], f["v_full"],
                            f["mask_full"], f["k_sparse"], f["v_sparse"], int(f["num_kv_groups"]))
    np.testing.assert_allclose(got, f["out"], rtol=1e-12, atol=1e-13)
    split = od.rotatek_decode_paper_splitk(f["q_full"], f["R_partial"], f.get("delta_mu"), f["k_full"],
                                           f["v_full"], f["mask_full"], f["k_sparse"], f["v_sparse"],
                                           int(f["num_kv_groups"]))
    np.testing.assert_allclose(split, f["out"], rtol=1e-12, atol=1e-13)


@pytest.mark.parametrize("dtype", ["bfloat16", "float16"])
def test_oracle_covariance_reproduces_golden(dtype):
    f = _load("covariance.npz")
    mean, cov = op.key_covariance(f["keys"], dtype)
    np.testing.assert_array_equal(mean, f["mean"])
    # golden values are small integers: exact in both storage formats
    np.testing.assert_array_equal(cov, f["cov"])


def test_oracle_topk_reproduces_golden():
    f = _load("topk.npz")
    idx, mask = op.topk_channels(f["scores"], int(f["k"]))
    np.testing.assert_array_equal(idx, f["idx"])
    np.testing.assert_array_equal(mask, f["mask"])


# ----------------------------------------------------------------- GPU
@pytest.mark.gpu
@pytest.mark.parametrize("name", DECODE)
@pytest.mark.parametrize("family", ["paper", "gqa"])
@pytest.mark.parametrize("dt", ["float16", "bfloat16"])
def test_hip_decode_reproduces_golden(name, family, dt):
    import torch

    from rotatek_amd.kernels.fused_decode import rotatek_decode_fused
    from rotatek_amd.kernels.gqa_decode import rotatek_decode_gqa
    print(f"[case] golden {name} {family} {dt}", flush=True)
    dtype = getattr(torch, dt)
    f = _load(name)
    args = {}
    for k in ("q_full", "R_partial", "delta_mu", "k_full", "v_full", "k_sparse", "v_sparse"):
        args[k] = torch.tensor(f[k], device="cuda").to(dtype) if k in f else None
    args["mask_full"] = torch.tensor(f["mask_full"], device="cuda")
    args["num_kv_groups"] = int(f["num_kv_groups"])
    fn = rotatek_decode_gqa if family == "gqa" else rotatek_decode_fused
    out = fn(**args)[0]
    torch.cuda.synchronize()
    tol = 2e-3 if dt == "float16" else 1e-2
    assert np.abs(out.float().cpu().numpy() - f["out"]).max() <= tol


@pytest.mark.gpu
@pytest.mark.parametrize("dt", ["float16", "bfloat16"])
def test_hip_covariance_reproduces_golden(dt):
    import torch

    from rotatek_amd import prefill
    print(f"[case] golden covariance {dt}", flush=True)
    f = _load("covariance.npz")
    mean, cov = prefill.key_covariance(torch.tensor(f["keys"], device="cuda").to(getattr(torch, dt)))
    torch.cuda.synchronize()
    np.testing.assert_array_equal(mean.cpu().numpy(), f["mean"])
    np.testing.assert_array_equal(cov.cpu().numpy(), f["cov"])


@pytest.mark.gpu
def test_hip_topk_reproduces_golden():
    import torch

    from rotatek_amd import prefill
    print("[case] golden topk", flush=True)
    f = _load("topk.npz")
    idx, mask = prefill.topk_channels(torch.tensor(f["scores"], device="cuda"), int(f["k"]))
    torch.cuda.synchronize()
    np.testing.assert_array_equal(idx.cpu().numpy(), f["idx"])
    np.testing.assert_array_equal(mask.cpu().numpy(), f["mask"])
