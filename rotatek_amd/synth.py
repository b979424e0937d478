"""Seeded synthetic decode inputs for the benchmark configurations.

There are no checkpoints or datasets offline, so every configuration is
synthesised as the benchmark definitions describe: q, K and V drawn from
N(0, 1); four Key channels per KV head scaled by 8 (outliers); a random
orthogonal R_k per (batch, KV head) from the QR of a seeded Gaussian
(float64 on the host, so the basis is identical on every machine); the
kept channels are the top ``keep`` rotated channels by mean |K R_k| (ties to
the lower index, indices ascending); ``k_sparse = K_vis R_partial`` and
``delta_mu = mu - (mu R) R^T`` with mu the fp32 mean of the visual Keys.

Layout follows the reference's unified value cache (cache_utils.py:14-43):
one V tensor ``[B, H_kv, S_v + S_f, D]`` whose first ``S_v`` tokens are the
visual span and the rest the full-width prompt/text span; ``v_sparse`` and
``v_full`` are views of it (as ``value_states[:, :, s_p:s_p+s_v]`` is at
llama_visionzip.py:212).  Generation runs on the target device with torch
(plumbing, never timed).
"""
from __future__ import annotations

import dataclasses

import torch


@dataclasses.dataclass(frozen=True)
class DecodeConfig:
    name: str
    B: int
    H_q: int
    H_kv: int
    S_v: int
    S_f: int
    keep: int
    dtype: torch.dtype
    D: int = 128
    outliers: int = 4

    @property
    def G(self) -> int:
        return self.H_q // self.H_kv


CONFIGS = {
    "cfg0": DecodeConfig("cfg0", 1, 32, 32, 2304, 128, 32, torch.float32),
    "cfg1": DecodeConfig("cfg1", 1, 32, 32, 15360, 640, 32, torch.float16),
    "cfg2": DecodeConfig("cfg2", 32, 32, 32, 14000, 2000, 32, torch.float16),
    "cfg3": DecodeConfig("cfg3", 16, 28, 4, 30720, 2048, 32, torch.bfloat16),
    # the reference's kernel microbenchmark shape (scripts/paper/kernel/
    # kernel_profile.py:37-45 and its usage line): H_q 32, H_kv 8, D_keep 32,
    # 50 prompt + 30 text tokens, bf16, 16000 visual tokens at batch 32
    "kp": DecodeConfig("kp", 32, 32, 8, 16000, 80, 32, torch.bfloat16),
}


def decode_bytes(c: DecodeConfig, esz: int | None = None, dense: bool = False) -> int:
    """Algorithmic HBM bytes of one decode step: every input read once and the
    output written once (K~, V, full-width K/V, R_partial, delta_mu, q, out,
    mask).  ``dense``: the full-channel baseline over all S_v + S_f tokens."""
    e = esz or torch.tensor([], dtype=c.dtype).element_size()
    if dense:
        return c.B * c.H_kv * (c.S_v + c.S_f) * 2 * c.D * e + 2 * c.B * c.H_q * c.D * e
    n = c.B * c.H_kv * c.S_v * (c.keep + c.D) * e
    n += c.B * c.H_kv * c.S_f * 2 * c.D * e
    n += c.B * c.H_kv * c.D * c.keep * e
    n += c.B * c.H_kv * c.D * e
    n += 2 * c.B * c.H_q * c.D * e
    n += c.B * c.S_f
    return n


def random_rotations(B: int, H: int, D: int, seed: int) -> torch.Tensor:
    """[B, H, D, D] float64 orthogonal matrices: Q of QR(seeded Gaussian)."""
    g = torch.Generator().manual_seed(seed)
    A = torch.randn(B, H, D, D, generator=g, dtype=torch.float64)
    Q, Rr = torch.linalg.qr(A)
    # fix the sign convention so Q is unique: diag(R) > 0
    return Q * torch.sign(torch.diagonal(Rr, dim1=-2, dim2=-1)).unsqueeze(-2)


def topk_ascending(scores: torch.Tensor, k: int) -> torch.Tensor:
    """Indices of the k largest scores per row (ties to the lower index),
    sorted ascending."""
    D = scores.shape[-1]
    # rank by (score desc, index asc) via a stable sort on -score
    order = torch.sort(-scores, dim=-1, stable=True).indices
    return torch.sort(order[..., :k], dim=-1).values


def make_decode_inputs(c: DecodeConfig, device="cuda", seed: int = 0, with_raw: bool = False,
                       with_dense: bool = False, chunk_b: int = 4, hip_select: bool | None = None) -> dict:
    """Synthesise one decode step of configuration ``c`` on ``device``.

    ``hip_select`` (default: for fp32 configurations, i.e. BASELINE config
    0, on a GPU) forms the kept channels, R_partial, delta_mu and k_sparse
    with the HIP prefill kernels (channel scores at the Keys' precision,
    head-wise top-k, gather, truncated write) instead of torch."""
    if hip_select is None:
        hip_select = c.dtype == torch.float32 and torch.device(device).type == "cuda"
    dev = torch.device(device)
    g = torch.Generator(device=dev).manual_seed(seed)
    B, Hq, Hkv, D, S_v, S_f = c.B, c.H_q, c.H_kv, c.D, c.S_v, c.S_f
    dt = c.dtype

    def randn(*shape):
        return torch.randn(*shape, generator=g, device=dev, dtype=torch.float32)

    q = randn(B, Hq, D).to(dt)
    V = randn(B, Hkv, S_v + S_f, D).to(dt)
    k_full = randn(B, Hkv, S_f, D).to(dt)
    # outlier channels per (b, kv): the same 4 channels for the visual Keys
    gen_cpu = torch.Generator().manual_seed(seed + 1)
    out_ch = torch.stack([torch.randperm(D, generator=gen_cpu)[: c.outliers] for _ in range(B * Hkv)])
    out_scale = torch.ones(B * Hkv, D)
    out_scale.scatter_(1, out_ch, 8.0)
    out_scale = out_scale.view(B, Hkv, 1, D).to(dev)
    Rk = random_rotations(B, Hkv, D, seed + 2).to(dev, torch.float32)

    k_sparse = torch.empty(B, Hkv, S_v, c.keep, device=dev, dtype=dt)
    R_partial = torch.empty(B, Hkv, D, c.keep, device=dev, dtype=dt)
    delta_mu = torch.empty(B, Hkv, D, device=dev, dtype=dt)
    keep_idx = torch.empty(B, Hkv, c.keep, device=dev, dtype=torch.int64)
    raw = torch.empty(B, Hkv, S_v, D, device=dev, dtype=dt) if with_raw else None
    dense_k = torch.empty(B, Hkv, S_v + S_f, D, device=dev, dtype=dt) if with_dense else None
    for b0 in range(0, B, chunk_b):
        b1 = min(B, b0 + chunk_b)
        Kv = (randn(b1 - b0, Hkv, S_v, D) * out_scale[b0:b1]).to(dt)
        Kf32 = Kv.float()
        Rb = Rk[b0:b1]
        if hip_select and S_v and c.keep:
            from rotatek_amd import prefill
            idx = prefill.topk_channels(prefill.channel_scores(Kv, Rb), c.keep)[0]
            mu = prefill.key_covariance(Kv)[0]
            Rp, dmu = prefill.gather_rotation(Rb, idx, mu, dt)
            k_sparse[b0:b1] = prefill.rotate_keys(Kv, Rp)
        else:
            scores = torch.matmul(Kf32, Rb).abs().mean(dim=-2) if S_v else torch.zeros(b1 - b0, Hkv, D, device=dev)
            idx = topk_ascending(scores, c.keep)
            Rp = torch.gather(Rb, -1, idx.unsqueeze(-2).expand(-1, -1, D, -1)).to(dt)
            mu = Kf32.mean(dim=-2) if S_v else torch.zeros(b1 - b0, Hkv, D, device=dev)
            Rpf = Rp.float()
            dmu = mu - torch.matmul(torch.matmul(mu.unsqueeze(-2), Rpf), Rpf.transpose(-1, -2)).squeeze(-2)
            k_sparse[b0:b1] = torch.matmul(Kf32, Rpf).to(dt)
        R_partial[b0:b1] = Rp
        delta_mu[b0:b1] = dmu.to(dt)
        keep_idx[b0:b1] = idx
        if raw is not None:
            raw[b0:b1] = Kv
        if dense_k is not None:
            dense_k[b0:b1, :, :S_v] = Kv
            dense_k[b0:b1, :, S_v:] = k_full[b0:b1]
        del Kv, Kf32
    out = {
        "q_full": q,
        "R_partial": R_partial,
        "delta_mu": delta_mu,
        "k_full": k_full,
        "v_full": V[:, :, S_v:],
        "mask_full": torch.ones(B, S_f, device=dev, dtype=torch.uint8),
        "k_sparse": k_sparse,
        "v_sparse": V[:, :, :S_v],
        "num_kv_groups": c.G,
        "keep_idx": keep_idx,
        "R_k": Rk,
        "V": V,
    }
    if raw is not None:
        out["k_vis_raw"] = raw
    if dense_k is not None:
        out["k_dense"] = dense_k
        out["v_dense"] = V
    return out


def clone_inputs(inp: dict) -> dict:
    """Same values at new addresses (V cloned once, its span views re-derived),
    so that a benchmark can cycle through copies and read from HBM rather than
    from the 256 MB MALL."""
    out = dict(inp)
    S_v = inp["v_sparse"].shape[2]
    V = inp["V"].clone()
    out["V"], out["v_sparse"], out["v_full"] = V, V[:, :, :S_v], V[:, :, S_v:]
    for k in ("q_full", "R_partial", "delta_mu", "k_full", "mask_full", "k_sparse", "k_dense"):
        if inp.get(k) is not None:
            out[k] = inp[k].clone()
    if "v_dense" in inp:
        out["v_dense"] = V
    return out


DECODE_KEYS = ("q_full", "R_partial", "delta_mu", "k_full", "v_full", "mask_full", "k_sparse",
               "v_sparse", "num_kv_groups")


def decode_args(inp: dict) -> dict:
    """The keyword arguments ``rotatek_decode`` takes, picked from ``inp``."""
    return {k: inp[k] for k in DECODE_KEYS}


# ------------------------------------------------------------ config 4 flow
@dataclasses.dataclass(frozen=True)
class FlowConfig:
    """Prefill rotation + decode sweep of a Qwen2.5-VL-7B-shaped stack:
    prompt and text spans of 30 tokens, the text span growing by one token
    per decode step (model_end_to_end_qwen.py:51-52)."""
    layers: int = 28
    B: int = 8
    H_q: int = 28
    H_kv: int = 4
    prompt: int = 30
    text: int = 30
    steps: int = 128
    visual: tuple = (4097, 12001)
    keep: tuple = (64, 32, 16)
    rank: int = 16
    dtype: torch.dtype = torch.bfloat16
    D: int = 128

    @property
    def G(self) -> int:
        return self.H_q // self.H_kv


FLOW = FlowConfig()
KEEP_TO_RATIO = {64: 0.5, 32: 0.75, 16: 0.875}   # keep = 128 - int(128 * ratio)


def make_flow_layer(c: FlowConfig, S_v: int, seed: int, device="cuda") -> dict:
    """One layer's prefill states ``K, V [B, H_kv, S, D]`` and ``Q [B, H_q, S, D]``
    with S = prompt + S_v + text.  Visual Keys are ``4 Z U^T + 0.5 E``: a
    rank-``c.rank`` signal (Z ~ N(0,1) [S_v, rank], U orthonormal [D, rank]
    per KV head) plus N(0,1) noise E; everything else is N(0,1)."""
    dev = torch.device(device)
    g = torch.Generator(device=dev).manual_seed(seed)
    B, Hq, Hkv, D = c.B, c.H_q, c.H_kv, c.D
    S = c.prompt + S_v + c.text

    def randn(*shape):
        return torch.randn(*shape, generator=g, device=dev, dtype=torch.float32)

    U = torch.linalg.qr(randn(B, Hkv, D, c.rank))[0]
    K = randn(B, Hkv, S, D)
    vis = K[:, :, c.prompt:c.prompt + S_v]
    vis.mul_(0.5).add_(4.0 * torch.matmul(randn(B, Hkv, S_v, c.rank), U.transpose(-1, -2)))
    K = K.to(c.dtype)
    V = randn(B, Hkv, S, D).to(c.dtype)
    Q = torch.empty(B, Hq, S, D, device=dev, dtype=c.dtype)
    for h in range(Hq):
        Q[:, h] = randn(B, S, D).to(c.dtype)
    return {"K": K, "V": V, "Q": Q}


def flow_step_bytes(c: FlowConfig, S_v: int, keep: int, S_f: int) -> int:
    """Algorithmic HBM bytes of one decode step over all layers with S_f
    prompt + text tokens attended: per layer, the RotateK decode bytes plus
    the append (new K and V rows read and written)."""
    layer = DecodeConfig("flow", c.B, c.H_q, c.H_kv, S_v, S_f, keep, c.dtype)
    append = 2 * 2 * c.B * c.H_kv * c.D * torch.tensor([], dtype=c.dtype).element_size()
    # the span-cache decode takes no mask
    return c.layers * (decode_bytes(layer) - c.B * S_f + append)
