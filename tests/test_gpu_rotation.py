"""GPU parity of the HIP subspace iteration (rk_power_iteration) with the
float64 oracle of rotation.py:21-53 started from the same block V0, with
the reference's torch loop on the device, and with eigh's subspace."""
import sys

import numpy as np
import pytest
import torch

from oracle import prefill as op

pytestmark = pytest.mark.gpu


def _say(msg):
    print(f"[case] {msg}", flush=True)
    sys.stdout.flush()


def _cov(B, H, seed, gap=True):
    g = torch.Generator(device="cuda").manual_seed(seed)
    Q = torch.linalg.qr(torch.randn(B, H, 128, 128, generator=g, device="cuda", dtype=torch.float64))[0]
    lam = torch.linspace(1.0, 0.01, 128, device="cuda", dtype=torch.float64)
    if gap:
        lam[:16] *= 20.0   # separated top block
    lam = lam * (1 + 0.1 * torch.rand(B, H, 128, generator=g, device="cuda", dtype=torch.float64))
    C = (Q * lam[..., None, :]) @ Q.transpose(-1, -2)
    C = 0.5 * (C + C.transpose(-1, -2))
    return C.float().contiguous()


def _power_iter_torch(cov, V, num_iters, eps):
    """The reference's loop (rotation.py:21-53) as torch ops on the device:
    a second, independent implementation to compare the kernel with."""
    eye = torch.eye(V.shape[-1], device=V.device, dtype=V.dtype)
    for _ in range(num_iters):
        V = cov @ V
        G = V.mT @ V
        G = G + (eps * G.diagonal(dim1=-2, dim2=-1).mean(-1)[..., None, None]) * eye
        V = torch.linalg.solve_triangular(torch.linalg.cholesky(G).mT, V, upper=True, left=False)
    return V


@pytest.mark.parametrize("k", [1, 16, 32, 40, 64, 65, 96, 128])
@pytest.mark.parametrize("eps", [1e-4, 1e-6])
def test_power_iteration_matches_oracle_from_same_start(k, eps):
    from rotatek_amd.rotation import power_iteration_hip
    _say(f"power iteration k={k} eps={eps}")
    cov = _cov(2, 3, seed=k)
    g = torch.Generator(device="cuda").manual_seed(0)
    V0 = torch.randn(2, 3, 128, k, generator=g, device="cuda")
    try:
        got = power_iteration_hip(cov, V0, 5, eps)
    except torch.linalg.LinAlgError:
        # past k = 64 the basis reaches the covariance's smallest eigenvalues
        # (down to 0.01 of 20): with the 1e-6 ridge the fp32 Gram matrix may
        # lose definiteness, where the reference's fp32 Cholesky raises too
        assert k > 64 and eps == 1e-6
        return
    torch.cuda.synchronize()
    want = op.power_iteration(cov.double().cpu().numpy(), V0.double().cpu().numpy(), 5, eps)
    g_np = got.double().cpu().numpy()
    # fp32 against fp64: 2e-3 up to k = 64; the full-width bases carry the
    # conditioning of the smallest eigenvalues (1e-2)
    tol = 2e-3 if k <= 64 else 1e-2
    assert np.abs(g_np - want).max() < tol * max(1.0, np.abs(want).max())
    # V^T V is the identity only up to the ridge (the reference's Cholesky
    # guard, rotation.py:36-50): it must deviate exactly as the oracle's does
    VtV = np.swapaxes(g_np, -1, -2) @ g_np
    VtV_want = np.swapaxes(want, -1, -2) @ want
    assert np.abs(VtV - VtV_want).max() < tol
    if eps == 1e-6 and k <= 64:
        # (a full-width basis reaches eigenvalues the ridge dominates, where
        # the oracle's V^T V departs from I just as much)
        assert np.abs(VtV - np.eye(k)).max() < 1e-2


def test_power_iteration_agrees_with_torch_loop_and_eigh():
    from rotatek_amd import rotation
    _say("power iteration vs torch loop / eigh")
    cov = _cov(4, 4, seed=99)
    g = torch.Generator(device="cuda").manual_seed(0)
    V0 = torch.randn(4, 4, 128, 16, generator=g, device="cuda")
    hip = rotation.power_iteration_hip(cov, V0, 5, 1e-4)
    ref = _power_iter_torch(cov, V0.clone(), 5, 1e-4)
    torch.cuda.synchronize()
    assert (hip - ref).abs().max().item() < 2e-3
    # the gapped top-16 block: projector equals eigh's
    w, U = torch.linalg.eigh(cov.double().cpu())
    Ut = U[..., -16:]
    P_e = Ut @ Ut.transpose(-1, -2)
    H = hip.double().cpu()
    P_h = H @ H.transpose(-1, -2)
    assert (P_e - P_h).abs().max().item() < 2e-2


def test_power_iteration_gpu_uses_hip_and_zero_iterations():
    from rotatek_amd import rotation
    _say("power_iteration_gpu dispatch / iters=0")
    cov = _cov(1, 2, seed=3)
    out = rotation.power_iteration_gpu(cov, k=32, num_iters=5, seed=0)
    g = torch.Generator(device="cuda").manual_seed(0)
    V0 = torch.randn(1, 2, 128, 32, device="cuda", generator=g)
    same = rotation.power_iteration_hip(cov, V0, 5)
    torch.cuda.synchronize()
    assert torch.equal(out, same)
    zero = rotation.power_iteration_hip(cov, V0, 0)
    torch.cuda.synchronize()
    assert torch.equal(zero, V0)


def test_power_iteration_many_matrices_strided_views():
    """300 matrices (more workgroups than CUs); covariance, start block and
    output as permuted / transposed views, so every stride is non-trivial."""
    from rotatek_amd.rotation import power_iteration_hip
    _say("power iteration 6 x 50 matrices, strided views, k=24")
    B, H, k = 6, 50, 24
    cov = _cov(H, B, seed=5).permute(1, 0, 2, 3)                  # [B,H,128,128], batch stride < head stride
    g = torch.Generator(device="cuda").manual_seed(1)
    V0 = torch.randn(B, H, k, 128, generator=g, device="cuda").transpose(-1, -2)   # column stride 128
    assert not cov.is_contiguous() and not V0.is_contiguous()
    got = power_iteration_hip(cov, V0, 5, 1e-4)
    torch.cuda.synchronize()
    want = op.power_iteration(cov.double().cpu().numpy(), V0.double().cpu().numpy(), 5, 1e-4)
    assert np.abs(got.double().cpu().numpy() - want).max() < 2e-3 * max(1.0, np.abs(want).max())


@pytest.mark.parametrize("iters", [1, 10])
def test_power_iteration_iteration_counts(iters):
    from rotatek_amd.rotation import power_iteration_hip
    _say(f"power iteration iters={iters} k=48")
    cov = _cov(2, 2, seed=iters)
    g = torch.Generator(device="cuda").manual_seed(2)
    V0 = torch.randn(2, 2, 128, 48, generator=g, device="cuda")
    got = power_iteration_hip(cov, V0, iters, 1e-4)
    torch.cuda.synchronize()
    want = op.power_iteration(cov.double().cpu().numpy(), V0.double().cpu().numpy(), iters, 1e-4)
    assert np.abs(got.double().cpu().numpy() - want).max() < 2e-3 * max(1.0, np.abs(want).max())


def test_power_iteration_rank_deficient_covariance():
    """Rank 8 covariance, k = 16: the Gram matrix is singular but for the
    ridge, which alone keeps the Cholesky defined (rotation.py:36-50)."""
    from rotatek_amd.rotation import power_iteration_hip
    _say("power iteration rank-8 covariance, k=16")
    g = torch.Generator(device="cuda").manual_seed(7)
    X = torch.randn(2, 3, 128, 8, generator=g, device="cuda", dtype=torch.float64)
    cov = (X @ X.transpose(-1, -2) / 8).float().contiguous()
    V0 = torch.randn(2, 3, 128, 16, generator=g, device="cuda")
    got = power_iteration_hip(cov, V0, 5, 1e-4)
    torch.cuda.synchronize()
    want = op.power_iteration(cov.double().cpu().numpy(), V0.double().cpu().numpy(), 5, 1e-4)
    g_np = got.double().cpu().numpy()
    assert np.isfinite(g_np).all()
    assert np.abs(g_np - want).max() < 2e-3 * max(1.0, np.abs(want).max())


@pytest.mark.parametrize("k", [16, 48])
def test_power_iteration_failed_pivot_raises(k):
    """A zero covariance with no ridge: every Gram pivot is 0.  The HIP
    Cholesky records it and the call raises torch.linalg.LinAlgError, as the
    reference's torch.linalg.cholesky does (rotation.py:49); the same call
    with the ridge on a sound covariance does not."""
    from rotatek_amd.rotation import power_iteration_hip
    _say(f"power iteration failed pivot, k={k}")
    cov = torch.zeros(1, 2, 128, 128, device="cuda")
    V0 = torch.randn(1, 2, 128, k, device="cuda")
    with pytest.raises(torch.linalg.LinAlgError):
        power_iteration_hip(cov, V0, 2, 0.0)
    g = torch.Generator(device="cuda").manual_seed(3)
    X = torch.randn(1, 2, 128, 128, generator=g, device="cuda")
    good = (X @ X.transpose(-1, -2)).contiguous()
    out = power_iteration_hip(good, V0, 5, 1e-4)
    torch.cuda.synchronize()
    assert torch.isfinite(out).all()


def test_power_iteration_rank_deficient_small_ridge():
    """Rank 8 covariance, k = 16 and the 1e-6 ridge (query weighting off):
    either the factorisation holds and the basis matches the oracle, or the
    call raises; it never returns a non-finite basis."""
    from rotatek_amd.rotation import power_iteration_hip
    _say("power iteration rank-8 covariance, k=16, eps 1e-6")
    g = torch.Generator(device="cuda").manual_seed(8)
    X = torch.randn(2, 3, 128, 8, generator=g, device="cuda", dtype=torch.float64)
    cov = (X @ X.transpose(-1, -2) / 8).float().contiguous()
    V0 = torch.randn(2, 3, 128, 16, generator=g, device="cuda")
    try:
        got = power_iteration_hip(cov, V0, 5, 1e-6)
    except torch.linalg.LinAlgError:
        return
    torch.cuda.synchronize()
    assert torch.isfinite(got).all()


@pytest.mark.parametrize("k", [96, 128])
def test_power_iteration_wide_basis_matches_torch_loop(k):
    """64 < k <= 128 (channel_ratio < 0.5): the HIP kernel against the torch
    loop from the same start, strided covariance view included."""
    from rotatek_amd.rotation import power_iteration_hip
    _say(f"power iteration wide k={k}")
    cov = _cov(3, 2, seed=k + 5)
    g = torch.Generator(device="cuda").manual_seed(k)
    V0 = torch.randn(3, 2, 128, k, generator=g, device="cuda")
    ref = _power_iter_torch(cov.double(), V0.double(), 5, 1e-4)
    got = power_iteration_hip(cov, V0, 5, 1e-4)
    big = torch.zeros(3, 2, 128, 160, device="cuda")
    big[..., :128] = cov
    got_s = power_iteration_hip(big[..., :128], V0, 5, 1e-4)
    torch.cuda.synchronize()
    scale = max(1.0, ref.abs().max().item())
    assert (got.double() - ref).abs().max().item() < 2e-3 * scale
    assert torch.equal(got, got_s)


@pytest.mark.parametrize("dtype", [torch.float64, torch.bfloat16])
def test_power_iteration_gpu_other_float_types(dtype):
    """Covariances in another float type are iterated in fp32 and the basis
    comes back in their dtype; its subspace is eigh's on the gapped block."""
    from rotatek_amd import rotation
    _say(f"power_iteration_gpu {dtype}")
    cov = _cov(1, 2, seed=17).to(dtype)
    out = rotation.power_iteration_gpu(cov, k=16, num_iters=5, seed=0)
    torch.cuda.synchronize()
    assert out.dtype == dtype and out.shape == (1, 2, 128, 16)
    U = torch.linalg.eigh(cov.double().cpu())[1][..., -16:]
    H = out.double().cpu()
    tol = 2e-2 if dtype == torch.bfloat16 else 2e-3
    assert ((U @ U.mT) - (H @ H.mT)).abs().max().item() < tol


def test_power_iteration_gpu_shapes():
    from rotatek_amd import rotation
    _say("power_iteration_gpu shapes")
    with pytest.raises(ValueError):       # head_dim past 128
        rotation.power_iteration_gpu(torch.zeros(2, 129, 129, device="cuda"), k=8)
    with pytest.raises(ValueError):       # not square
        rotation.power_iteration_gpu(torch.zeros(2, 64, 32, device="cuda"), k=8)
    with pytest.raises(ValueError):       # k past D
        rotation.power_iteration_gpu(torch.zeros(2, 64, 64, device="cuda"), k=65)
    with pytest.raises(ValueError):
        rotation.power_iteration_gpu(torch.zeros(2, 128, 128, device="cuda"), k=129)
    cov = _cov(1, 6, seed=4)[0]                       # [6, 128, 128]: any leading dims
    out = rotation.power_iteration_gpu(cov, k=24)
    torch.cuda.synchronize()
    assert out.shape == (6, 128, 24) and torch.isfinite(out).all()


def _lowrank_keys(B, H, S, seed, rank=32):
    g = torch.Generator(device="cuda").manual_seed(seed)
    U = torch.linalg.qr(torch.randn(B, H, 128, rank, generator=g, device="cuda"))[0]
    Z = torch.randn(B, H, S, rank, generator=g, device="cuda")
    E = torch.randn(B, H, S, 128, generator=g, device="cuda")
    return (4.0 * Z @ U.transpose(-1, -2) + 0.5 * E).to(torch.bfloat16)


def test_power_iteration_and_update_rotatek_in_a_hip_graph():
    """power_iteration_gpu and a whole ChannelPruner.update_rotatek with the
    reference's default solver (power_iter) captured in one HIP graph (the
    capture-friendly path of rotation.py:58-65, ROTATEK_COMPILE
    reduce-overhead).  After one eager call, which draws the seeded start
    block as the reference does on every call, each replay equals the eager
    results bit for bit: the subspace basis, the truncated Keys, R_partial,
    delta_mu and the keep mask.  Outputs are poisoned before each replay,
    and other eager iterations and prunings run between replays."""
    from rotatek_amd.pruning import ChannelPruner
    from rotatek_amd.rotation import power_iteration_gpu
    _say("power iteration + update_rotatek captured in a HIP graph")
    B, H, G, S = 2, 4, 7, 1100
    cov = _cov(B, H, seed=77)
    K = _lowrank_keys(B, H, S, seed=78)
    Q = torch.randn(B, H * G, S, 128, device="cuda").to(torch.bfloat16)
    V = torch.randn(B, H, S, 128, device="cuda").to(torch.bfloat16)
    pr = ChannelPruner(0.75, 30, 40, solver="power_iter", query_aware=True)
    want_R = power_iteration_gpu(cov, 32)
    kept0, _, _, mask0, _ = pr.update_rotatek(K, Q, V, None, G)
    want = [t.clone() for t in (want_R, kept0, pr.current_rotatek_R_partial, pr.current_rotatek_delta_mu, mask0)]
    torch.cuda.synchronize()

    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=s):
        R_g = power_iteration_gpu(cov, 32)
        kept_g, _, _, mask_g, _ = pr.update_rotatek(K, Q, V, None, G)
        got = [R_g, kept_g, pr.current_rotatek_R_partial, pr.current_rotatek_delta_mu, mask_g]
    other_cov = _cov(1, 2, seed=79)
    other = ChannelPruner(0.875, 10, 10, solver="power_iter", query_aware=True)
    for i in range(3):
        for t in got:
            t.fill_(0 if t.dtype == torch.bool else float("nan"))
        graph.replay()
        torch.cuda.synchronize()
        for name, a, b in zip(("basis", "k_sparse", "R_partial", "delta_mu", "mask"), got, want):
            assert torch.equal(a, b), (i, name)
        power_iteration_gpu(other_cov, 24)
        other.update_rotatek(K[:1, :2, :500], Q[:1, :14, :500], None, None, G)
        torch.cuda.synchronize()


def _pi_cases(n=20, seed=31):
    rng = np.random.default_rng(seed)
    out = []
    for i in range(n):
        D = int(rng.choice([8, 24, 40, 64, 80, 100, 128]))
        out.append(dict(i=i, D=D, k=int(rng.integers(1, D + 1)), iters=int(rng.choice([1, 3, 5, 8])),
                        B=int(rng.integers(1, 3)), H=int(rng.integers(1, 4))))
    return out


@pytest.mark.parametrize("case", _pi_cases(), ids=lambda c: f"{c['i']}")
def test_power_iteration_random_shapes(case):
    """Seeded random head dims (8-128), widths k (1..D) and iteration counts
    (1-8), from the same start block as the float64 oracle, ridge 1e-4:
    2e-3 of the largest entry while k <= D / 2, 1e-2 for wider bases (they
    reach eigenvalues down to 0.01 of the top block's 20)."""
    from rotatek_amd.rotation import power_iteration_hip
    c = case
    D, k, iters, B, H = c["D"], c["k"], c["iters"], c["B"], c["H"]
    _say(f"power iteration random {c}")
    g = torch.Generator(device="cuda").manual_seed(900 + c["i"])
    Q = torch.linalg.qr(torch.randn(B, H, D, D, generator=g, device="cuda", dtype=torch.float64))[0]
    lam = torch.linspace(1.0, 0.01, D, device="cuda", dtype=torch.float64)
    lam[:min(16, D)] *= 20.0
    lam = lam * (1 + 0.1 * torch.rand(B, H, D, generator=g, device="cuda", dtype=torch.float64))
    C = (Q * lam[..., None, :]) @ Q.transpose(-1, -2)
    cov = (0.5 * (C + C.transpose(-1, -2))).float().contiguous()
    V0 = torch.randn(B, H, D, k, generator=g, device="cuda")
    got = power_iteration_hip(cov, V0, iters, 1e-4)
    torch.cuda.synchronize()
    want = op.power_iteration(cov.double().cpu().numpy(), V0.double().cpu().numpy(), iters, 1e-4)
    g_np = got.double().cpu().numpy()
    assert g_np.shape == want.shape == (B, H, D, k)
    tol = 2e-3 if 2 * k <= D else 1e-2
    assert np.abs(g_np - want).max() < tol * max(1.0, np.abs(want).max())
