#!/usr/bin/env python3
"""RotateK decode benchmark on one MI355X (BASELINE.json metric).

Workload: one decode step at batch 32, 32 heads (MHA),
head_dim 128, fp16; visual span 14,000 tokens stored rotated and truncated to
32 of 128 channels, plus 2,000 full-width text tokens; synthetic seeded
inputs (no checkpoints offline).  A "step" is one call of
``rotatek_decode`` (two HIP launches on the current stream: the split-K
decode kernel, then the merge kernel) with every input resident in HBM.

Printed JSON line (rank 0): ``value`` = microseconds per decode step (eager,
wall clock over exactly ``--steps`` steps between device synchronisations);
``roofline`` = algorithmic bytes per launch / average launch duration (HIP
events around each launch on the launching stream) against the 8 TB/s HBM
peak; ``cpu_baseline`` = the reference's decode restated on the CPU (the
reference has no CPU path) over whole steps of the same inputs, on every
core of the process's affinity mask: the batched torch-eager fp32
restatement (``value``) and the numpy fp32 oracle beside it.  Also reported:
hipGraph-replayed step time and the full-channel HIP baseline on the same
seeded data.
Working sets under 1 GB (configs 1 and 3) are cycled through up to eight
copies of the inputs so that repeated steps read HBM, not the 256 MB MALL.

``--copy-calibration BYTES`` adds a plain device-to-device copy of BYTES
bytes per step (after the timed region), so that a ``rocprofv3 --pmc
FETCH_SIZE`` / ``WRITE_SIZE`` pass over this script sees a kernel of known
traffic next to the decode kernel; ``roofline.traffic`` is read from the
committed summary of those passes (profiles/traffic_<config>.json).
"""
from __future__ import annotations

import argparse
import dataclasses
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

METRIC = "µs per decode step + achieved HBM GB/s (% of peak), B=32, 16k ctx, keep 25%"
HBM_PEAK_GBPS = 8000.0


def _log(msg):
    print(msg, file=sys.stderr, flush=True)


def _time_wall(fn, steps):
    import torch
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        fn()
    torch.cuda.synchronize()
    return (time.perf_counter() - t0) / steps * 1e6


def _time_launches(fn, steps):
    """Average per-launch duration (us) from event pairs on the current stream."""
    import torch
    evs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(steps)]
    torch.cuda.synchronize()
    for s, e in evs:
        s.record()
        fn()
        e.record()
    torch.cuda.synchronize()
    return sum(s.elapsed_time(e) for s, e in evs) / steps * 1e3


def _time_graph(fn, steps, warmup, per_graph=1):
    """hipGraph replay time per call of ``fn``; the graph holds ``per_graph``
    consecutive calls (one per input copy when inputs are rotated)."""
    import torch
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for _ in range(max(1, warmup)):
            fn()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        for _ in range(per_graph):
            fn()
    torch.cuda.synchronize()
    for _ in range(5):
        g.replay()
    torch.cuda.synchronize()
    reps = max(1, -(-steps // per_graph))
    s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    s.record()
    for _ in range(reps):
        g.replay()
    e.record()
    torch.cuda.synchronize()
    return s.elapsed_time(e) / (reps * per_graph) * 1e3


def _timed(fn, reps, graph=True):
    """(result, device us per call, wall us per call) over ``reps`` calls.
    Device-only stages are replayed from a HIP graph, so small kernels are not
    timed at the speed of the Python call that launches them."""
    import torch
    out = fn()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    if graph:
        g = torch.cuda.CUDAGraph()
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            with torch.cuda.graph(g, stream=side):
                for _ in range(reps):
                    fn()
        torch.cuda.current_stream().wait_stream(side)
        g.replay()
        torch.cuda.synchronize()
        run = g.replay
    else:
        def run():
            for _ in range(reps):
                fn()
    t0 = time.perf_counter()
    e0.record()
    run()
    e1.record()
    torch.cuda.synchronize()
    wall = (time.perf_counter() - t0) / reps * 1e6
    return out, e0.elapsed_time(e1) * 1e3 / reps, wall


def _host_cores():
    """CPU cores this process may run on (its affinity mask)."""
    return len(os.sched_getaffinity(0))


def _host_decode_inputs(inp, b0=0, b1=None):
    """fp32 numpy copies of the decode inputs of batch rows b0..b1."""
    import numpy as np

    names = ("q_full", "R_partial", "delta_mu", "k_full", "v_full", "mask_full", "k_sparse", "v_sparse")
    out = {}
    for k in names:
        t = inp[k]
        out[k] = None if t is None else np.ascontiguousarray(t[b0:b1].float().cpu().numpy(), dtype=np.float32)
    return out


def _time_oracle_steps(a, G, budget_s):
    """Median wall time (s) of whole oracle decode steps over ``a``, repeated
    for about ``budget_s`` seconds (at least three)."""
    import numpy as np

    from oracle import decode as od
    times, total = [], 0.0
    while total < budget_s or len(times) < 3:
        t0 = time.perf_counter()
        od.rotatek_decode(a["q_full"], a["R_partial"], a["delta_mu"], a["k_full"], a["v_full"], a["mask_full"],
                          a["k_sparse"], a["v_sparse"], G, compute_dtype=np.float32)
        dt = time.perf_counter() - t0
        times.append(dt)
        total += dt
    return sorted(times)[len(times) // 2], len(times), total


def _time_torch_steps(a, G, budget_s):
    """Median wall time (s) of whole decode steps of the batched torch
    restatement (oracle.decode.rotatek_decode_torch) over the fp32 host
    arrays ``a`` (shared, not copied), repeated for about ``budget_s``
    seconds (at least three)."""
    import torch

    from oracle import decode as od
    t = {k: None if v is None else torch.from_numpy(v) for k, v in a.items()}
    times, total = [], 0.0
    with torch.inference_mode():
        while total < budget_s or len(times) < 3:
            t0 = time.perf_counter()
            od.rotatek_decode_torch(t["q_full"], t["R_partial"], t["delta_mu"], t["k_full"], t["v_full"],
                                    t["mask_full"], t["k_sparse"], t["v_sparse"], G)
            dt = time.perf_counter() - t0
            times.append(dt)
            total += dt
    return sorted(times)[len(times) // 2], len(times), total


def _cpu_baseline(inp, cfg, budget_s=8.0):
    """The reference's decode restated on the CPU (the reference has no CPU
    path) on every core of this process's affinity mask: whole decode steps
    of the same inputs (all B batch rows, every head, full context), each
    repeated for about ``budget_s`` seconds, the median step.  ``value`` is
    the batched torch-eager fp32 restatement (oracle.decode.
    rotatek_decode_torch, torch.set_num_threads(cores)); the numpy fp32 oracle
    (a loop over batch rows and KV heads, BLAS pool limited to the same
    cores) is reported beside it."""
    from threadpoolctl import threadpool_limits
    import torch

    cores = _host_cores()
    torch.set_num_threads(cores)
    a = _host_decode_inputs(inp)
    with threadpool_limits(limits=cores):
        med_t, n_t, tot_t = _time_torch_steps(a, inp["num_kv_groups"], budget_s)
        med, n, total = _time_oracle_steps(a, inp["num_kv_groups"], budget_s)
    return {
        "value": round(med_t * 1e6, 1),
        "unit": "us/step",
        "cores": cores,
        "kind": "port",
        "sample": f"batched torch-eager fp32 restatement (oracle/decode.py rotatek_decode_torch: whole-span "
                  f"products over [B, H_kv, G, S]) over whole steps of the same inputs ({cfg.name}: all "
                  f"{cfg.B} batch rows, {cfg.H_q} heads, {cfg.S_v}+{cfg.S_f} context), {n_t} steps, median; "
                  f"{tot_t:.1f} s of CPU work, torch.set_num_threads({cores})",
        "numpy_oracle_us_per_step": round(med * 1e6, 1),
        "numpy_oracle_sample": f"numpy fp32 oracle (oracle/decode.py rotatek_decode, a loop over (b, kv)), "
                               f"{n} whole steps, median; {total:.1f} s on {cores} threads",
    }


def _cfg0_leg(budget_s=3.0):
    """BASELINE config 0 (B=1, 32 heads, 2304 + 128 tokens, fp32): the CPU
    oracle over whole steps on every core of the affinity mask, and the HIP
    fp32 decode of the same inputs (eager, inputs resident in HBM)."""
    from threadpoolctl import threadpool_limits
    import torch

    from rotatek_amd import synth
    from rotatek_amd.kernels.fused_decode import rotatek_decode_fused
    cfg = synth.CONFIGS["cfg0"]
    inp = synth.make_decode_inputs(cfg, "cuda", seed=0)
    args = synth.decode_args(inp)
    for _ in range(5):
        rotatek_decode_fused(**args)
    gpu_us = _time_wall(lambda: rotatek_decode_fused(**args), 100)
    cores = _host_cores()
    torch.set_num_threads(cores)
    a = _host_decode_inputs(inp)
    with threadpool_limits(limits=cores):
        med_t, n_t, _ = _time_torch_steps(a, inp["num_kv_groups"], budget_s)
        med, n, total = _time_oracle_steps(a, inp["num_kv_groups"], budget_s)
    return {"cpu_us_per_step": round(med_t * 1e6, 1), "cpu_kind": "batched torch-eager fp32 restatement",
            "cpu_cores": cores, "cpu_steps": n_t, "cpu_numpy_oracle_us_per_step": round(med * 1e6, 1),
            "hip_fp32_us_per_step": round(gpu_us, 2),
            "workload": "cfg0: B=1, H=32 MHA, D=128, S_v=2304 (keep 32), S_f=128, fp32; kept channels selected "
                        "by the HIP prefill kernels at fp32"}


# the decode path's sources: host code, kernels, their per-dtype units and
# the shared device helpers
DECODE_SOURCES = [os.path.join(ROOT, "rotatek_amd", "csrc", f)
                  for f in ("rk_decode.hip", "rk_decode.h", "rk_decode_dev.h", "rk_decode_f16.hip",
                            "rk_decode_bf16.hip", "rk_decode_f32.hip", "rk_common.h")]
PREFILL_SOURCES = [os.path.join(ROOT, "rotatek_amd", "csrc", f) for f in ("rk_prefill.hip", "rk_rotation.hip",
                                                                          "rk_common.h")]
# the ThinK / SparK baseline kernels (their dense decode is the decode path's)
BASELINE_SOURCES = [os.path.join(ROOT, "rotatek_amd", "csrc", f) for f in ("rk_baselines.hip", "rk_common.h")]


def _code_text(src: str) -> str:
    """The source with // and /* */ comments removed and whitespace runs
    collapsed: what the compiler sees, so that edits of comments alone keep
    a measurement valid (the decode source has no string literal holding a
    comment marker)."""
    import re
    src = re.sub(r"/\*.*?\*/", " ", src, flags=re.S)
    src = re.sub(r"//[^\n]*", " ", src)
    return " ".join(src.split())


def _source_sha(text: str | None = None, files=None):
    """sha256 prefix of the code (comments stripped) of ``text``, or of the
    files (default: the decode sources), each preceded by its name."""
    import hashlib
    if text is None:
        parts = []
        for path in files or DECODE_SOURCES:
            with open(path) as f:
                parts.append(os.path.basename(path) + " " + _code_text(f.read()))
        text = "\n".join(parts)
        return hashlib.sha256(text.encode()).hexdigest()[:16]
    return hashlib.sha256(_code_text(text).encode()).hexdigest()[:16]


def _traffic(cfg_name):
    """HBM bytes per decode launch from the committed counter summary, or
    None when that summary was taken on other decode code than this tree's
    (it records the sha256 of the decode sources' code, comments stripped)."""
    path = os.path.join(ROOT, "profiles", f"traffic_{cfg_name}.json")
    if not os.path.exists(path):
        return None
    with open(path) as f:
        d = json.load(f)
    if d.get("decode_source_sha256") != _source_sha():
        return None
    return d.get("hbm_bytes_per_launch")


def _pmc_rows(path):
    import csv
    with open(path) as f:
        rows = list(csv.DictReader(f))
    rows.sort(key=lambda r: int(r["Dispatch_Id"]))
    return rows


def pmc_summary(fetch_csv, write_csv, calib_bytes, calib_copies, cfg_name):
    """Turn two ``rocprofv3 --pmc`` passes over ``bench.py --copy-calibration``
    (FETCH_SIZE, then WRITE_SIZE; KiB per dispatch) into HBM bytes per
    launch of the decode and merge kernels.  Each counter is scaled by what
    it reads for the calibration copies (the last ``calib_copies``
    dispatches of the run, ``calib_bytes`` read and written each)."""
    from rotatek_amd import synth
    out = {"config": cfg_name, "calibration_bytes": calib_bytes}
    for counter, path in (("FETCH_SIZE", fetch_csv), ("WRITE_SIZE", write_csv)):
        rows = [r for r in _pmc_rows(path) if r["Counter_Name"] == counter]
        calib = rows[-calib_copies:]
        kib = sum(float(r["Counter_Value"]) for r in calib) / len(calib)
        factor = kib * 1024.0 / calib_bytes
        out[counter] = {"calibration_kernel": calib[0]["Kernel_Name"][:60],
                        "calibration_kib": round(kib, 1), "factor": round(factor, 4), "kernels": {}}
        for tag in ("rk::decode_kernel", "rk::merge_kernel"):
            sel = [float(r["Counter_Value"]) for r in rows if tag in r["Kernel_Name"]]
            if sel:
                avg = sum(sel) / len(sel)
                out[counter]["kernels"][tag] = {"dispatches": len(sel), "kib": round(avg, 1),
                                                "bytes": round(avg * 1024.0 / factor)}
    dk = "rk::decode_kernel"
    rd = out["FETCH_SIZE"]["kernels"][dk]["bytes"]
    wr = out["WRITE_SIZE"]["kernels"][dk]["bytes"]
    cfg = synth.CONFIGS[cfg_name]
    alg = synth.decode_bytes(cfg)
    out["hbm_bytes_per_launch"] = rd + wr
    out["decode_kernel_read_bytes"] = rd
    out["decode_kernel_write_bytes"] = wr
    out["algorithmic_bytes_per_step"] = alg
    out["traffic_over_algorithmic"] = round((rd + wr) / alg, 4)
    # what was measured: the decode source the counters ran (bench.py reports
    # the traffic only while the tree's source matches) and the commit
    out["decode_source_sha256"] = _source_sha()
    try:
        import subprocess
        out["commit"] = subprocess.run(["git", "-C", ROOT, "rev-parse", "--short=12", "HEAD"], capture_output=True,
                                       text=True, check=True).stdout.strip()
    except Exception:
        out["commit"] = None
    path = os.path.join(ROOT, "profiles", f"traffic_{cfg_name}.json")
    with open(path, "w") as f:
        json.dump(out, f, indent=1)
        f.write("\n")
    print(json.dumps(out, indent=1))


def run_flow(args):
    """Config 4: per (visual length, keep) point, prefill a 28-layer stack
    (HIP covariance -> device eigh -> head-wise channel top-k -> truncated Key
    write into the span cache), then time ``--steps`` decode steps, each one
    replay of a HIP graph that appends a token and runs the RotateK decode
    for every layer."""
    import torch

    from rotatek_amd import synth
    from rotatek_amd.cache import DynamicCache
    from rotatek_amd.pruning import ChannelPruner

    from rotatek_amd._lib import RK_POLICY_GQA, RK_POLICY_PAPER

    c = synth.FLOW
    steps = args.steps if args.steps_given else c.steps
    # a GQA stack (G = 7): the gqa family shares each K/V tile across the
    # query heads of its group; ``--family paper`` re-reads it per query head
    family = args.family if args.family_given else "gqa"
    policy = RK_POLICY_GQA if family == "gqa" else RK_POLICY_PAPER
    torch.cuda.set_device(0)
    dev = torch.device("cuda", 0)
    sweep = []
    for S_v in c.visual:
        for keep in c.keep:
            pruner = ChannelPruner(synth.KEEP_TO_RATIO[keep], c.prompt, c.text, solver="eigh", select="score",
                                   query_aware=True)
            cache = DynamicCache(reserve_tokens=steps + 1)
            pre_ms = []
            for layer in range(c.layers):
                st = synth.make_flow_layer(c, S_v, seed=1000 * S_v + layer, device=dev)
                torch.cuda.synchronize()
                t0 = time.perf_counter()
                kept, kp, kt, mask, v = pruner.update_rotatek(st["K"], st["Q"], st["V"], None, c.G)
                cache.store_pruned(kept, kp, kt, mask, v, layer)
                cache.rotatek_rotations.append(pruner.current_rotatek_R_partial)
                cache.rotatek_means.append(pruner.current_rotatek_delta_mu)
                torch.cuda.synchronize()
                pre_ms.append((time.perf_counter() - t0) * 1e3)
                del st, kept, kp, kt, v
            g = torch.Generator(device=dev).manual_seed(S_v + keep)
            q = torch.randn(c.layers, c.B, c.H_q, c.D, generator=g, device=dev).to(c.dtype)
            kn = torch.randn(c.layers, c.B, c.H_kv, 1, c.D, generator=g, device=dev).to(c.dtype)
            vn = torch.randn(c.layers, c.B, c.H_kv, 1, c.D, generator=g, device=dev).to(c.dtype)
            out = torch.empty(c.layers, c.B, c.H_q, c.D, device=dev, dtype=c.dtype)
            lens0 = [cache.lengths(i).clone() for i in range(c.layers)]
            graph = cache.capture_decode(q, kn, vn, out, c.G, policy=policy)
            graph.replay()                      # warm-up replay, then rewind the lengths
            torch.cuda.synchronize()
            for i in range(c.layers):
                cache.lengths(i).copy_(lens0[i])
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            torch.cuda.synchronize()
            e0.record()
            for _ in range(steps):
                graph.replay()
            e1.record()
            torch.cuda.synchronize()
            us = e0.elapsed_time(e1) * 1e3 / steps
            cache.sync_lengths()
            want = c.prompt + S_v + c.text + steps
            if cache.get_seq_length(0) != want or cache.get_seq_length(c.layers - 1) != want:
                raise RuntimeError(f"cache length {cache.get_seq_length(0)} after {steps} steps, expected {want}")
            nbytes = sum(synth.flow_step_bytes(c, S_v, keep, c.prompt + c.text + i + 1) for i in range(steps))
            gbps = nbytes / steps / (us * 1e-6) / 1e9
            pre = sorted(pre_ms)[len(pre_ms) // 2]
            _log(f"[flow] S_v={S_v} keep={keep}: prefill {pre:.2f} ms/layer (median), decode {us:.1f} us/step "
                 f"({c.layers} layers, graph), {gbps:.0f} GB/s")
            sweep.append({"visual_tokens": S_v, "keep": keep, "prefill_ms_per_layer": round(pre, 3),
                          "decode_us_per_step": round(us, 2), "decode_gbps": round(gbps, 1),
                          "decode_pct_of_peak_hbm": round(gbps / HBM_PEAK_GBPS * 100, 2)})
            del cache, graph, q, kn, vn, out
            torch.cuda.empty_cache()
    head = next(r for r in sweep if r["visual_tokens"] == max(c.visual) and r["keep"] == 32)
    line = {
        "metric": "config 4 flow: decode us per step over 28 layers (hipGraph replay) + prefill ms per layer",
        "value": head["decode_us_per_step"], "unit": "us/step", "n_gpus": 1, "steps": steps, "warmup": 1,
        "ms_per_step": round(head["decode_us_per_step"] / 1e3, 4), "higher_is_better": False,
        "scaling": "weak", "vs_baseline": None, "dtype": "bf16",
        "data": "synthetic: visual Keys 4 Z U^T + 0.5 E (rank 16), N(0,1) elsewhere",
        "config": {"workload": f"cfg4: {c.layers} layers, B={c.B}, H_q={c.H_q}, H_kv={c.H_kv}, prompt {c.prompt} + "
                               f"text {c.text} growing, eigh + head-wise top-k, family={family}; value at "
                               f"S_v={head['visual_tokens']}, keep 32", "family": family, "sweep": sweep},
    }
    print(json.dumps(line), flush=True)


def run_prefill(args):
    """Config 4 prefill, one layer per visual length, each stage timed on
    the device (HIP events over ``--steps`` repetitions, replayed from a HIP
    graph where the stage is device-only): key covariance
    (mean pass + MFMA covariance pass + finalize), query weighting (HIP),
    eigh (torch, on the host as the reference and on the device, the
    default here), the HIP subspace iteration
    (the reference's default solver), channel scores, top-k, R_partial /
    delta_mu gather and the truncated Key write."""
    import torch

    from rotatek_amd import prefill, synth
    from rotatek_amd.rotation import power_iteration_gpu

    c = synth.FLOW
    torch.cuda.set_device(0)
    dev = torch.device("cuda", 0)
    reps = args.steps if args.steps_given else 20
    keep = 32
    rows = []

    def timed(fn, graph=True):
        return _timed(fn, reps, graph)

    for S_v in c.visual:
        st = synth.make_flow_layer(c, S_v, seed=S_v, device=dev)
        kv = st["K"][:, :, c.prompt:c.prompt + S_v]
        (mean, cov), t_cov, _ = timed(lambda: prefill.key_covariance(kv))
        covw, t_qw, _ = timed(lambda: prefill.query_weight(cov, st["Q"], c.G))
        # the weighting folded into the covariance's last launch (what update_rotatek runs)
        _, t_covw, _ = timed(lambda: prefill.key_covariance(kv, st["Q"], c.G))
        _, _, w_eigh = timed(lambda: prefill.eigen_rotation(covw, on_host=True), graph=False)
        R_full, _, w_eigh_dev = timed(lambda: prefill.eigen_rotation(covw, on_host=False), graph=False)
        _, t_pi, _ = timed(lambda: power_iteration_gpu(covw, keep, num_iters=5, seed=0), graph=False)
        scores, t_sc, _ = timed(lambda: prefill.channel_scores(kv, R_full))
        (idx, mask), t_tk, _ = timed(lambda: prefill.topk_channels(scores, keep))
        (Rp, dmu), t_ga, _ = timed(lambda: prefill.gather_rotation(R_full, idx, mean, kv.dtype))
        _, t_rot, _ = timed(lambda: prefill.rotate_keys(kv, Rp))
        heads = c.B * c.H_kv
        kbytes = heads * S_v * c.D * 2
        cov_flops = heads * 36 * 256 * 2 * S_v   # the 36 upper 16x16 tiles computed on the MFMA
        row = {"visual_tokens": S_v, "keep": keep,
               "covariance_us": round(t_cov, 2),
               "covariance_gbps_two_passes": round(2 * kbytes / t_cov / 1e3, 1),
               "covariance_mfma_tflops": round(cov_flops / t_cov / 1e6, 2),
               "query_weight_us": round(t_qw, 2),
               "covariance_weighted_us": round(t_covw, 2),
               "eigh_host_us": round(w_eigh, 1),
               "eigh_device_us": round(w_eigh_dev, 1),
               "power_iteration_us": round(t_pi, 2),
               "channel_scores_us": round(t_sc, 2), "topk_us": round(t_tk, 2),
               "gather_us": round(t_ga, 2), "rotate_write_us": round(t_rot, 2),
               "rotate_write_gbps": round((kbytes + heads * S_v * keep * 2) / t_rot / 1e3, 1)}
        _log(f"[prefill] S_v={S_v}: " + ", ".join(f"{k}={v}" for k, v in row.items() if k != "visual_tokens"))
        rows.append(row)
        del st, kv
    line = {"metric": "config 4 prefill stages per layer (us, HIP events)", "value": rows[-1]["covariance_us"],
            "unit": "us", "n_gpus": 1, "steps": reps, "warmup": 1, "higher_is_better": False, "dtype": "bf16",
            "data": "synthetic: visual Keys 4 Z U^T + 0.5 E (rank 16)",
            "config": {"workload": f"cfg4 prefill, B={c.B}, H_kv={c.H_kv}, keep {keep}, eigh + head-wise top-k; "
                                   f"value = key covariance at S_v={c.visual[-1]}", "stages": rows}}
    print(json.dumps(line), flush=True)


def run_baselines(args):
    """ThinK and SparK (kv_pruning_utils.py:44-90, llama_visionzip.py:216-241)
    at a decode configuration (default config 2) on one GPU: the prefill
    selection of each over the visual Keys, the decode-time recovery (the
    recovered visual rows and the full-width span written by one launch) and
    the decode step (recovery + dense decode), next to ThinK's attention on
    the RotateK kernel (one-hot R, no recovery) and the RotateK step on the
    same data.  Every stage is >= 100 us at config 2, so it is timed eagerly
    with HIP events over ``--steps`` calls; bytes are algorithmic."""
    import torch

    from rotatek_amd import synth
    from rotatek_amd.baselines import (recover_spark, recover_think, selection_rotation, spark_prune,
                                       think_score_and_compact)
    from rotatek_amd.kernels.full_channel_flash_decoding import full_channel_decode
    from rotatek_amd.kernels.fused_decode import rotatek_decode_fused
    from rotatek_amd.kernels.gqa_decode import full_channel_decode_gqa, rotatek_decode_gqa

    cfg = synth.CONFIGS[args.config]
    # GQA shapes default to the gqa family (each K/V tile shared by the group)
    family = args.family if args.family_given else ("gqa" if cfg.G > 1 else "paper")
    rot = rotatek_decode_gqa if family == "gqa" else rotatek_decode_fused
    dense = full_channel_decode_gqa if family == "gqa" else full_channel_decode
    torch.cuda.set_device(0)
    reps = args.steps if args.steps_given else 20
    inp = synth.make_decode_inputs(cfg, "cuda", seed=0, with_raw=True)
    B, Hq, H, S_v, S_f, keep, G = cfg.B, cfg.H_q, cfg.H_kv, cfg.S_v, cfg.S_f, cfg.keep, cfg.G
    prune, e, heads, rows = 128 - keep, 2, cfg.B * cfg.H_kv, cfg.S_v + cfg.S_f
    g = torch.Generator(device="cuda").manual_seed(1)
    Kv, q, kf, V = inp["k_vis_raw"], inp["q_full"], inp["k_full"], inp["V"]   # V rows: [visual | full]
    Qw = torch.randn(B, Hq, 32, 128, generator=g, device="cuda").to(cfg.dtype)
    stage = torch.empty(B, H, rows, 128, device="cuda", dtype=cfg.dtype)
    _log(f"[baselines] {torch.cuda.get_device_name(0)}; {cfg}")

    def timed(fn):
        return _timed(fn, reps, graph=False)

    r = {}
    kbytes = heads * S_v * 128 * e
    (Kc_t, tm), t, _ = timed(lambda: think_score_and_compact(Kv, Qw, H, prune))
    r["think_prefill_us"] = t
    r["think_prefill_gbps"] = (2 * kbytes + heads * S_v * keep * e) / t / 1e3   # two passes over K
    (Kc_s, sm, pm), t, _ = timed(lambda: spark_prune(Kv, Qw, G, prune))
    r["spark_prefill_us"] = t
    r["spark_prefill_gbps"] = (kbytes + heads * S_v * (keep * e + 128 + e)) / t / 1e3
    full_bytes = heads * S_f * 128 * e + heads * rows * 128 * e               # read the full span, write all rows
    _, t, _ = timed(lambda: recover_think(Kc_t, tm, out=stage, k_text=kf))
    r["think_recover_us"] = t
    r["think_recover_gbps"] = (heads * S_v * keep * e + full_bytes) / t / 1e3
    _, t, _ = timed(lambda: recover_spark(Kc_s, sm, pm, out=stage, k_text=kf))
    r["spark_recover_us"] = t
    r["spark_recover_gbps"] = (heads * S_v * (keep * e + 128 + e) + full_bytes) / t / 1e3

    def think_step():
        recover_think(Kc_t, tm, out=stage, k_text=kf)
        return dense(q, stage, V, G)

    def spark_step():
        recover_spark(Kc_s, sm, pm, out=stage, k_text=kf)
        return dense(q, stage, V, G)

    da = synth.decode_args(inp)
    R_sel = selection_rotation(tm, keep, cfg.dtype)
    think_fused_args = dict(da, R_partial=R_sel, delta_mu=None, k_sparse=Kc_t)
    for name, fn in (("think_decode_step", think_step), ("spark_decode_step", spark_step),
                     ("think_fused_decode", lambda: rot(**think_fused_args)),
                     ("rotatek_decode", lambda: rot(**da))):
        _, t, _ = timed(fn)
        r[name + "_us"] = t
    r = {k: round(v, 2) for k, v in r.items()}
    _log("[baselines] " + ", ".join(f"{k}={v}" for k, v in r.items()))
    line = {"metric": "ThinK / SparK baselines on HIP: prefill per layer and decode step (us, HIP events)",
            "value": r["think_decode_step_us"], "unit": "us", "n_gpus": 1, "steps": reps, "warmup": 1,
            "higher_is_better": False, "dtype": "fp16" if cfg.dtype == torch.float16 else "bf16",
            "data": "synthetic: the decode inputs of the configuration, full-width visual Keys, N(0,1) "
                    "query window of 32",
            "config": {"workload": f"{cfg.name} baselines: B={B}, H_q={Hq}, H_kv={H}, S_v={S_v}, S_f={S_f}, "
                                   f"keep {keep}, family={family}; value = ThinK decode step (recover + dense "
                                   f"decode)",
                       "stages": r}}
    print(json.dumps(line), flush=True)


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--config", default="cfg2")
    ap.add_argument("--family", default="paper", choices=["paper", "gqa"],
                    help="decode family (default: gqa when G > 1, else paper)")
    ap.add_argument("--seqlen", type=int, default=0,
                    help="override the visual span length (kernel_profile.py's --seqlen)")
    ap.add_argument("--batch-size", type=int, default=0,
                    help="override the batch (kernel_profile.py's --batch_size)")
    ap.add_argument("--merge", default="auto", choices=["auto", "two", "one"],
                    help="decode merge: the library default (auto: one launch for a single round of "
                         "one-query-head units, else two), two launches, or one launch")
    ap.add_argument("--graph-steps", type=int, default=32,
                    help="decode steps captured per hipGraph replay (rounded up to the input copies); "
                         "a one-step graph is timed as well")
    ap.add_argument("--chunk-align", type=int, default=0, choices=[0, 32, 64, 128],
                    help="visual chunk granularity of the decode planner (0: the library default)")
    ap.add_argument("--skew", type=int, default=-1, metavar="PERMILLE",
                    help="share of the first-dispatched visual chunks of a one-round grid, in thousandths "
                         "of the others' (-1: the library default, 0: equal chunks)")
    ap.add_argument("--wgs-per-cu", type=int, default=0, metavar="N",
                    help="decode workgroups planned per CU (0: the library default, two or one for a "
                         "single round of small workgroups)")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-dense", action="store_true")
    ap.add_argument("--no-graph", action="store_true")
    ap.add_argument("--prefill-only", action="store_true", help="config 4: time the prefill stages")
    ap.add_argument("--baselines", action="store_true",
                    help="time the ThinK / SparK prefill, recovery and decode at --config")
    ap.add_argument("--copy-calibration", type=int, default=0, metavar="BYTES")
    ap.add_argument("--pmc-summary", nargs=2, metavar=("FETCH_CSV", "WRITE_CSV"),
                    help="summarise two rocprofv3 --pmc passes (no GPU needed)")
    ap.add_argument("--source-sha", action="store_true",
                    help="print the code hashes (comments stripped) that profiles are stamped with")
    args = ap.parse_args()
    if args.source_sha:
        print(json.dumps({"decode_source_sha256": _source_sha(),
                          "prefill_source_sha256": _source_sha(files=PREFILL_SOURCES),
                          "baseline_source_sha256": _source_sha(files=BASELINE_SOURCES)}))
        return
    args.steps_given = any(a == "--steps" or a.startswith("--steps=") for a in sys.argv[1:])
    args.family_given = any(a == "--family" or a.startswith("--family=") for a in sys.argv[1:])
    if args.chunk_align and not args.pmc_summary:
        from rotatek_amd import _lib
        _lib.set_decode_chunk_align(args.chunk_align)
    if args.skew >= 0 and not args.pmc_summary:
        from rotatek_amd import _lib
        _lib.set_decode_skew(args.skew)
    if args.wgs_per_cu > 0 and not args.pmc_summary:
        from rotatek_amd import _lib
        _lib.set_decode_tuning(0, 0, args.wgs_per_cu)
    if args.merge != "auto" and not args.pmc_summary:
        from rotatek_amd import _lib
        _lib.set_decode_merge({"two": _lib.MERGE_TWO_LAUNCHES, "one": _lib.MERGE_SINGLE_LAUNCH}[args.merge])
    if args.config == "cfg4":
        if args.gpus != 1:
            print("bench.py measures one GPU only", file=sys.stderr)
            sys.exit(2)
        run_prefill(args) if args.prefill_only else run_flow(args)
        return
    if args.pmc_summary:
        pmc_summary(args.pmc_summary[0], args.pmc_summary[1], args.copy_calibration, args.steps, args.config)
        return
    if args.baselines:
        if args.gpus != 1:
            print("bench.py measures one GPU only", file=sys.stderr)
            sys.exit(2)
        run_baselines(args)
        return
    if args.gpus != 1:
        print(f"bench.py measures one GPU only (asked for --gpus {args.gpus}); the RotateK decode "
              "shards by (batch, KV head) with no exchange, so N GPUs run N independent copies.",
              file=sys.stderr)
        sys.exit(2)

    import torch

    from rotatek_amd import synth
    from rotatek_amd.kernels.fused_decode import rotatek_decode_fused
    from rotatek_amd.kernels.full_channel_flash_decoding import full_channel_decode
    from rotatek_amd.kernels.gqa_decode import full_channel_decode_gqa, rotatek_decode_gqa

    cfg = synth.CONFIGS[args.config]
    if args.seqlen > 0 or args.batch_size > 0:
        cfg = dataclasses.replace(cfg, S_v=args.seqlen or cfg.S_v, B=args.batch_size or cfg.B)
    torch.cuda.set_device(0)
    _log(f"[bench] {torch.cuda.get_device_name(0)}; generating {cfg}")
    inp = synth.make_decode_inputs(cfg, "cuda", seed=0, with_dense=not args.no_dense)
    nbytes = synth.decode_bytes(cfg)
    # working sets under 1 GB would be served partly from the 256 MB MALL when
    # the same inputs are read back to back: cycle through copies instead
    copies = 1 if nbytes >= (1 << 30) else min(8, -(-(1 << 30) // nbytes))
    sets = [inp] + [synth.clone_inputs(inp) for _ in range(copies - 1)]
    dsets = [synth.decode_args(x) for x in sets]
    # default family: gqa when query heads share a KV head (the per-query-head
    # paper decomposition re-reads K/V G times), paper otherwise (identical)
    if not args.family_given:
        args.family = "gqa" if cfg.G > 1 else "paper"
    rot = rotatek_decode_gqa if args.family == "gqa" else rotatek_decode_fused
    dense = full_channel_decode_gqa if args.family == "gqa" else full_channel_decode
    turn = [0, 0]

    def step():
        turn[0] += 1
        return rot(**dsets[turn[0] % copies])

    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    _log("[bench] warmup done")
    us = _time_wall(step, args.steps)
    us_launch = _time_launches(step, args.steps)
    # Each hipGraph launch costs a gap of several microseconds before its
    # first kernel (the kernel trace shows ~8 us between one replay's merge
    # and the next replay's split kernel, none between eager launches), so a
    # one-step graph pays it every step; several steps per replay amortise it
    per_graph = copies * max(1, -(-args.graph_steps // copies))
    us_graph = _time_graph(step, args.steps, args.warmup, per_graph) if not args.no_graph else None
    us_graph1 = (_time_graph(step, args.steps, args.warmup, copies) if not args.no_graph and per_graph != copies
                 else us_graph)
    gbps = nbytes / (us_launch * 1e-6) / 1e9
    _log(f"[bench] rotatek eager {us:.1f} us/step, per-launch {us_launch:.1f} us, graph {us_graph} us "
         f"({per_graph} steps per replay; one-step replays {us_graph1} us), "
         f"{gbps:.0f} GB/s ({gbps / HBM_PEAK_GBPS * 100:.1f}% of peak)")

    extra = {}
    if not args.no_dense:
        def dstep():
            turn[1] += 1
            x = sets[turn[1] % copies]
            return dense(x["q_full"], x["k_dense"], x["v_dense"], num_kv_groups=cfg.G)

        for _ in range(args.warmup):
            dstep()
        d_us = _time_wall(dstep, args.steps)
        d_launch = _time_launches(dstep, args.steps)
        d_graph = _time_graph(dstep, args.steps, args.warmup, per_graph) if not args.no_graph else None
        dbytes = synth.decode_bytes(cfg, dense=True)
        extra = {
            "dense_us_per_step": round(d_us, 2),
            "dense_graph_us_per_step": round(d_graph, 2) if d_graph else None,
            "dense_achieved_gbps": round(dbytes / (d_launch * 1e-6) / 1e9, 1),
            "speedup_vs_dense": round(d_us / us, 3),
            "speedup_vs_dense_graph": round(d_graph / us_graph, 3) if d_graph else None,
        }
        _log(f"[bench] dense eager {d_us:.1f} us/step, graph {d_graph} us -> speedup {d_us / us:.2f}x eager")

    if args.copy_calibration > 0:
        n = args.copy_calibration
        src = torch.ones(n, dtype=torch.uint8, device="cuda")
        dst = torch.empty_like(src)
        for _ in range(max(args.steps, 1)):
            dst.copy_(src)
        torch.cuda.synchronize()
        _log(f"[bench] copy calibration: {args.steps} copies of {n} bytes")
        del src, dst

    cpu, cfg0 = None, None
    if not args.no_cpu:
        del sets, dsets
        torch.cuda.empty_cache()
        _log("[bench] timing the CPU oracle over whole steps")
        cpu = _cpu_baseline(inp, cfg)
        _log(f"[bench] cpu baseline {cpu['value']:.0f} us/step (torch eager), numpy oracle "
             f"{cpu['numpy_oracle_us_per_step']:.0f} us/step, on {cpu['cores']} threads")
        if args.config == "cfg2":
            cfg0 = _cfg0_leg()
            _log(f"[bench] config 0: cpu {cfg0['cpu_us_per_step']} us/step on {cfg0['cpu_cores']} threads, "
                 f"HIP fp32 {cfg0['hip_fp32_us_per_step']} us/step")

    line = {
        "metric": METRIC,
        "value": round(us, 2),
        "unit": "us/step",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(us / 1e3, 4),
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": {torch.float16: "fp16", torch.bfloat16: "bf16", torch.float32: "fp32"}[cfg.dtype],
        "data": "synthetic: seeded N(0,1) q/K/V, x8 outlier Key channels, orthogonal R_k per head, "
                "top-32 channels by mean |K R_k|",
        "config": {
            "workload": f"{cfg.name}: RotateK decode step, B={cfg.B}, H_q={cfg.H_q}, H_kv={cfg.H_kv}, D=128, "
                        f"S_v={cfg.S_v} (keep {cfg.keep}), S_f={cfg.S_f}, family={args.family}",
            "batch": cfg.B, "heads_q": cfg.H_q, "heads_kv": cfg.H_kv, "visual_tokens": cfg.S_v,
            "full_tokens": cfg.S_f, "kept_channels": cfg.keep, "family": args.family,
        },
        "achieved_gbps": round(gbps, 1),
        "pct_of_peak_hbm": round(gbps / HBM_PEAK_GBPS * 100, 2),
        "graph_us_per_step": round(us_graph, 2) if us_graph else None,
        "graph_steps_per_replay": per_graph,
        "graph_one_step_replay_us": round(us_graph1, 2) if us_graph1 else None,
        "input_copies": copies,
        "launch_us": round(us_launch, 2),
        "roofline": {
            "bound": "hbm",
            "achieved": round(gbps, 1),
            "peak": HBM_PEAK_GBPS,
            "unit": "GB/s",
            "frac": round(gbps / HBM_PEAK_GBPS, 4),
            "traffic": _traffic(cfg.name),
        },
        "cpu_baseline": cpu,
        "config0": cfg0,
    }
    line.update(extra)
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
