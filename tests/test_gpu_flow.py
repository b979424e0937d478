"""The config 4 flow end to end at a reduced size: prefill of a small stack
through ``ChannelPruner.update_rotatek`` (eigh + head-wise top-k) into the
span cache, then graph-replayed decode steps, each layer's output checked
against the oracle on the same cached tensors."""
import sys

import numpy as np
import pytest
import torch

from oracle import decode as od

pytestmark = pytest.mark.gpu


def _np(t):
    return None if t is None else t.detach().float().cpu().numpy().astype(np.float64)


def test_flow_prefill_then_graph_decode():
    import dataclasses

    from rotatek_amd import synth
    from rotatek_amd.cache import DynamicCache
    from rotatek_amd.pruning import ChannelPruner
    c = dataclasses.replace(synth.FLOW, layers=2, B=2, steps=3)
    S_v, keep = 1025, 16
    print(f"[case] flow layers={c.layers} B={c.B} S_v={S_v} keep={keep}", flush=True)
    sys.stdout.flush()
    pruner = ChannelPruner(synth.KEEP_TO_RATIO[keep], c.prompt, c.text, solver="eigh", select="score")
    cache = DynamicCache(reserve_tokens=c.steps)
    states = []
    for layer in range(c.layers):
        st = synth.make_flow_layer(c, S_v, seed=layer, device="cuda")
        kept, kp, kt, mask, v = pruner.update_rotatek(st["K"], st["Q"], st["V"], None, c.G)
        assert kept.shape == (c.B, c.H_kv, S_v, keep) and mask.sum(-1).eq(keep).all()
        cache.store_pruned(kept, kp, kt, mask, v, layer)
        cache.rotatek_rotations.append(pruner.current_rotatek_R_partial)
        cache.rotatek_means.append(pruner.current_rotatek_delta_mu)
        states.append(st)
    g = torch.Generator(device="cuda").manual_seed(9)
    q = torch.randn(c.layers, c.B, c.H_q, c.D, generator=g, device="cuda").to(c.dtype)
    kn = torch.randn(c.layers, c.B, c.H_kv, 1, c.D, generator=g, device="cuda").to(c.dtype)
    vn = torch.randn(c.layers, c.B, c.H_kv, 1, c.D, generator=g, device="cuda").to(c.dtype)
    out = torch.empty(c.layers, c.B, c.H_q, c.D, device="cuda", dtype=c.dtype)
    graph = cache.capture_decode(q, kn, vn, out, c.G)
    for step in range(c.steps):
        graph.replay()
        torch.cuda.synchronize()
        for layer in range(c.layers):
            st = states[layer]
            n_text = c.text + step + 1
            K, V = st["K"], st["V"]
            k_text = torch.cat([K[:, :, -c.text:]] + [kn[layer]] * (step + 1), dim=-2)
            v_text = torch.cat([V[:, :, -c.text:]] + [vn[layer]] * (step + 1), dim=-2)
            k_full = torch.cat([K[:, :, :c.prompt], k_text], dim=-2)
            v_full = torch.cat([V[:, :, :c.prompt], v_text], dim=-2)
            assert k_full.shape[-2] == c.prompt + n_text
            want = od.rotatek_decode(_np(q[layer]), _np(cache.rotatek_rotations[layer]),
                                     _np(cache.rotatek_means[layer]), _np(k_full), _np(v_full),
                                     np.ones((c.B, k_full.shape[-2])), _np(cache.key_cache_pruned[layer]),
                                     _np(V[:, :, c.prompt:c.prompt + S_v]), c.G)
            assert np.abs(_np(out[layer])[:, None] - want).max() <= 1e-2, (step, layer)
    cache.sync_lengths()
    assert cache.get_seq_length(0) == c.prompt + S_v + c.text + c.steps
