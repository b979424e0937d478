"""BASELINE config 4 at its own workload: B=8, H_q=28 / H_kv=4 (G=7), bf16,
prompt 30 + text 30 tokens around S_v in {4097, 12001} visual tokens, keep in
{64, 32, 16} (channel_ratio 0.5 / 0.75 / 0.875), visual Keys 4 Z U^T + 0.5 E.

Per point, all 28 layers of the stack go through
``ChannelPruner.update_rotatek`` (HIP covariance, HIP query weighting, eigh,
HIP head-wise channel scores and top-k, truncated write;
kv_pruning_utils.py:92-160) into ``DynamicCache`` (cache_utils.py:48-55);
then ten decode steps are replayed from one captured HIP graph that appends
a token and decodes every layer (llama_visionzip.py:197-215).  The prompt +
text span grows from 60 to 70 tokens, across the 64-token boundary of the
decode's 32-token blocks.

Checks, on the first, a middle and the last layer:
* kept channels: the HIP top-k of the HIP channel scores equals the oracle's
  top-k of the very same scores (indices and masks bit-exact), and equals the
  mask the pruner stored;
* every replayed step: sampled (batch, KV head) groups against
  ``oracle.decode.rotatek_decode`` on the cached tensors plus the appended
  tokens (bf16 bar, max-abs 1e-2); the device lengths of every layer.
"""
import sys

import numpy as np
import pytest
import torch

from oracle import decode as od
from oracle import prefill as op

pytestmark = pytest.mark.gpu

TOL = 1e-2
STEPS = 10
CHECKED = (0, 13, 27)              # layers checked against the oracle
GROUPS = [(0, 0), (3, 2), (7, 3)]  # sampled (batch row, KV head)


def _np(t):
    return None if t is None else t.detach().float().cpu().numpy().astype(np.float64)


def _say(msg):
    print(f"[case] {msg}", flush=True)
    sys.stdout.flush()


@pytest.mark.parametrize("keep", [64, 32, 16])
@pytest.mark.parametrize("S_v", [4097, 12001])
def test_config4_flow_matches_oracle(S_v, keep):
    from rotatek_amd import prefill, synth
    from rotatek_amd.cache import DynamicCache
    from rotatek_amd.pruning import ChannelPruner
    c = synth.FLOW
    G = c.G
    LAYERS = c.layers
    _say(f"config 4 flow S_v={S_v} keep={keep} B={c.B} H_q={c.H_q} H_kv={c.H_kv} layers={LAYERS} steps={STEPS}")
    pruner = ChannelPruner(synth.KEEP_TO_RATIO[keep], c.prompt, c.text, solver="eigh", select="score",
                           query_aware=True)
    cache = DynamicCache(reserve_tokens=STEPS + 1)
    states = []
    for layer in range(LAYERS):
        st = synth.make_flow_layer(c, S_v, seed=1000 * S_v + layer, device="cuda")
        kept, kp, kt, mask, v = pruner.update_rotatek(st["K"], st["Q"], st["V"], None, G)
        assert kept.shape == (c.B, c.H_kv, S_v, keep)
        cache.store_pruned(kept, kp, kt, mask, v, layer)
        cache.rotatek_rotations.append(pruner.current_rotatek_R_partial)
        cache.rotatek_means.append(pruner.current_rotatek_delta_mu)
        if layer not in CHECKED:
            states.append(None)
            del st, kept, kp, kt, v
            continue
        # the selection on the same scores: HIP top-k == oracle top-k == the pruner's mask
        visual = st["K"][:, :, c.prompt:c.prompt + S_v]
        _, cov = prefill.key_covariance(visual)
        cov = prefill.query_weight(cov, st["Q"], G)
        scores = prefill.channel_scores(visual, prefill.eigen_rotation(cov))
        idx, m_hip = prefill.topk_channels(scores, keep)
        torch.cuda.synchronize()
        wi, wm = op.topk_channels(scores.cpu().numpy(), keep)
        np.testing.assert_array_equal(idx.cpu().numpy(), wi)
        np.testing.assert_array_equal(m_hip.cpu().numpy(), wm)
        np.testing.assert_array_equal(mask.cpu().numpy(), wm)
        # host copies of what the oracle needs, sampled groups only
        states.append({(b, kv): dict(k_prompt=_np(kp[b, kv]), k_text=_np(kt[b, kv]),
                                     v_prompt=_np(v[b, kv, :c.prompt]), v_text=_np(v[b, kv, c.prompt + S_v:]),
                                     v_vis=_np(v[b, kv, c.prompt:c.prompt + S_v]), k_sparse=_np(kept[b, kv]),
                                     R=_np(pruner.current_rotatek_R_partial[b, kv]),
                                     dm=_np(pruner.current_rotatek_delta_mu[b, kv]))
                       for b, kv in GROUPS})
        del st, kept, kp, kt, v, visual, cov, scores
    g = torch.Generator(device="cuda").manual_seed(S_v + keep)
    q = torch.zeros(LAYERS, c.B, c.H_q, c.D, device="cuda", dtype=c.dtype)
    kn = torch.zeros(LAYERS, c.B, c.H_kv, 1, c.D, device="cuda", dtype=c.dtype)
    vn = torch.zeros_like(kn)
    out = torch.empty(LAYERS, c.B, c.H_q, c.D, device="cuda", dtype=c.dtype)
    graph = cache.capture_decode(q, kn, vn, out, G)
    appended = [{grp: ([], []) for grp in GROUPS} for _ in range(LAYERS)]
    for step in range(STEPS):
        q.copy_(torch.randn(q.shape, generator=g, device="cuda").to(c.dtype))
        kn.copy_(torch.randn(kn.shape, generator=g, device="cuda").to(c.dtype))
        vn.copy_(torch.randn(vn.shape, generator=g, device="cuda").to(c.dtype))
        graph.replay()
        torch.cuda.synchronize()
        for layer in range(LAYERS):
            assert bool((cache.lengths(layer) == c.prompt + c.text + step + 1).all())
            if layer not in CHECKED:
                continue
            for b, kv in GROUPS:
                s = states[layer][(b, kv)]
                ka, va = appended[layer][(b, kv)]
                ka.append(_np(kn[layer, b, kv]))
                va.append(_np(vn[layer, b, kv]))
                k_full = np.concatenate([s["k_prompt"], s["k_text"]] + ka, axis=0)
                v_full = np.concatenate([s["v_prompt"], s["v_text"]] + va, axis=0)
                want = od.rotatek_decode(_np(q[layer, b, kv * G:(kv + 1) * G])[None], s["R"][None, None],
                                         s["dm"][None, None], k_full[None, None], v_full[None, None], None,
                                         s["k_sparse"][None, None], s["v_vis"][None, None], G)
                got = _np(out[layer, b, kv * G:(kv + 1) * G])
                err = np.abs(got - want[0, 0]).max()
                assert err <= TOL, (step, layer, b, kv, err)
