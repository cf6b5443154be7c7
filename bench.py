"""Benchmark of the FP8 block-scale MoE operator on one MI355X.

``python bench.py [--gpus 1] [--steps K] [--warmup W] [--config ds_t64] [--sweep]``

A step is one call of the operator (routing -> permute -> GEMM1+SwiGLU -> GEMM2 -> combine) on a
seeded synthetic batch already resident in HBM. The headline workload is the decode-sized DS-V3
case (T=64); the prefill-sized T=4096 case is measured in the same run and reported under
``secondary``. ``--sweep`` adds the skewed T=16384 and the Qwen3 T=1024 cases.

Prints ONE JSON line. ``value`` is TFLOP/s of the headline workload over algorithmic FLOPs
(6*H*I per local (token, expert) pair, pairs counted from the routing of the run); ``roofline``
describes the dominant kernel (GEMM1 + SwiGLU) from stage events recorded on the operator's stream;
``cpu_baseline`` times the CPU oracle (the dequantise-then-fp32 PyTorch-CPU restatement of the
operator) on the host cores.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

import torch

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, HERE)

from justgoal_amd import _lib  # noqa: E402
from justgoal_amd import inputs as jin  # noqa: E402
from justgoal_amd.geometry import BLOCK, bytes_per_token, flops_per_pair, weight_bytes_per_expert  # noqa: E402
from justgoal_amd.moe import bind, workspace_views  # noqa: E402

METRIC = "ms/call + TFLOPS, DS-V3 FP8 MoE at T=64 and T=4096; % of FP8 MFMA/HBM peak"
PEAK_HBM_GBS = 8000.0
PEAK_FP8_TFLOPS = 5000.0
PEAK_BF16_TFLOPS = 2500.0
STAGES = ("route", "permute", "gemm1_swiglu", "gemm2", "combine")
# GEMM1 kernel-family thresholds of justgoal_amd/csrc/moe_gemm.hip (JG_STREAM_MAX_ROWS,
# JG_BIG_ROWS defaults; tests/test_bench.py checks they match the source)
GEMM1_STREAM_MAX_ROWS = 4
GEMM1_BIG_ROWS = 64


def log(msg):
    print(msg, file=sys.stderr, flush=True)


def routing_stats(geom, T, ws):
    """Routed pairs, active local experts and tokens with a local pair, read from the workspace
    of the call that just ran."""
    v = workspace_views(geom, T, ws)
    counts = v["counts"].cpu()
    pairs = int(counts.sum())
    active = int((counts > 0).sum())
    tok_local = int(((v["pair_of"].cpu() >= 0).any(dim=1)).sum())
    return pairs, active, tok_local


def algorithmic(geom, T, pairs, active, tok_local):
    """FLOPs and HBM bytes the operator must move (intermediates excluded)."""
    H, I = geom.hidden, geom.intermediate
    flops = flops_per_pair(geom) * pairs
    bytes_ = active * weight_bytes_per_expert(geom) + T * bytes_per_token(geom) + 2 * geom.num_experts
    # GEMM1 + SwiGLU alone: W13 + S13 of active experts, routed fp8 rows + scales, bf16 C rows
    w13 = 2 * I * H + 4 * (2 * I // BLOCK) * (H // BLOCK)
    g1_bytes = active * w13 + tok_local * (H + 4 * H // BLOCK) + pairs * I * 2
    g1_flops = 2 * H * 2 * I * pairs
    return flops, bytes_, g1_flops, g1_bytes


def time_calls(call, steps, warmup, dev):
    for _ in range(warmup):
        call()
    torch.cuda.synchronize(dev)
    start = torch.cuda.Event(enable_timing=True)
    end = torch.cuda.Event(enable_timing=True)
    start.record()
    for _ in range(steps):
        call()
    end.record()
    torch.cuda.synchronize(dev)
    return start.elapsed_time(end) / steps


def stage_times(call, reps, dev):
    """Average per-stage milliseconds from hipEvents the library records on its own stream."""
    import ctypes
    n = len(STAGES) + 1
    sets = [[torch.cuda.Event(enable_timing=True) for _ in range(n)] for _ in range(reps)]
    for evs in sets:  # torch creates the underlying hipEvent on first record
        for e in evs:
            e.record()
    torch.cuda.synchronize(dev)
    L = _lib.lib()
    tot = [0.0] * len(STAGES)
    try:
        # calls go back to back (no host sync in between), as in the timed loop
        for evs in sets:
            arr = (ctypes.c_void_p * n)(*[e.cuda_event for e in evs])
            _lib.check(L.moe_set_stage_events(arr, n), "moe_set_stage_events")
            call()
        torch.cuda.synchronize(dev)
    finally:
        L.moe_set_stage_events(None, 0)
    for evs in sets:
        for i in range(len(STAGES)):
            tot[i] += evs[i].elapsed_time(evs[i + 1])
    return {s: tot[i] / reps for i, s in enumerate(STAGES)}


def measure(cfg, weights_dev, steps, warmup, dev, seed=None):
    geom = cfg.geom
    seed = cfg.seed if seed is None else seed
    act = jin.make_activations(geom, cfg.tokens, seed=seed, device=dev,
                               skew_experts=cfg.skew_experts, skew_offset=cfg.skew_offset)
    w13, s13, w2, s2 = weights_dev
    kw = dict(act, gemm1_weights=w13, gemm1_weights_scale=s13, gemm2_weights=w2,
              gemm2_weights_scale=s2, local_expert_offset=0,
              routed_scaling_factor=2.5 if geom.routing_method == 0 else 1.0)
    call = bind(**kw, geometry=geom)
    ms = time_calls(call, steps, warmup, dev)
    st = stage_times(call, max(5, min(steps, 20)), dev)
    pairs, active, tok_local = routing_stats(geom, cfg.tokens, call.workspace)
    if pairs == 0:
        raise RuntimeError(f"{cfg.name}: no routed pairs read back from the call's workspace")
    flops, bytes_, g1_flops, g1_bytes = algorithmic(geom, cfg.tokens, pairs, active, tok_local)
    tflops = flops / (ms * 1e-3) / 1e12
    gbs = bytes_ / (ms * 1e-3) / 1e9
    t_floor_ms = max(flops / (PEAK_FP8_TFLOPS * 1e12), bytes_ / (PEAK_HBM_GBS * 1e9)) * 1e3
    g1_ms = st["gemm1_swiglu"]
    res = dict(workload=cfg.name, tokens=cfg.tokens, ms_per_call=ms, tflops=tflops, gb_s=gbs,
               pairs=pairs, active_experts=active, algorithmic_flops=flops,
               algorithmic_bytes=bytes_, roofline_floor_ms=t_floor_ms,
               roofline_frac=t_floor_ms / ms, hbm_frac=gbs / PEAK_HBM_GBS,
               fp8_mfma_frac=tflops / PEAK_FP8_TFLOPS, stage_ms=st,
               gemm1=dict(ms=g1_ms, bytes=g1_bytes, flops=g1_flops,
                          gb_s=g1_bytes / (g1_ms * 1e-3) / 1e9,
                          tflops=g1_flops / (g1_ms * 1e-3) / 1e12))
    return res, kw


def measure_quant(T, H, steps, warmup, dev):
    """The activation-quantisation kernel on a bf16 [T, H] batch already in HBM: algorithmic bytes
    = bf16 read + e4m3 write + fp32 scales (2 + 1 + 4/128 bytes per element)."""
    from justgoal_amd.moe import quantize_activations
    x = torch.randn(T, H, generator=torch.Generator().manual_seed(2)).bfloat16().to(dev)
    q = torch.empty((T, H), dtype=torch.float8_e4m3fn, device=dev)
    sc = torch.empty((H // BLOCK, T), dtype=torch.float32, device=dev)
    ms = time_calls(lambda: quantize_activations(x, q, sc), steps, warmup, dev)
    nbytes = T * H * 3 + T * (H // BLOCK) * 4
    gbs = nbytes / (ms * 1e-3) / 1e9
    return dict(tokens=T, hidden=H, ms_per_call=ms, bytes=nbytes, gb_s=gbs,
                hbm_frac=gbs / PEAK_HBM_GBS)


def gemm1_kernel_name(cfg):
    """The GEMM1+SwiGLU kernel family the library picks for this shape: the shape-only rule of
    justgoal_amd/csrc/moe_gemm.hip (expected pairs per expert T*top_k/E: <= GEMM1_STREAM_MAX_ROWS
    streaming, >= GEMM1_BIG_ROWS large tiles, else LDS tiles)."""
    g = cfg.geom
    rows = cfg.tokens * g.top_k // g.num_experts
    return ("gemm1_stream_kernel" if rows <= GEMM1_STREAM_MAX_ROWS else
            "gemm1_tile_kernel" if rows < GEMM1_BIG_ROWS else "gemm1_big_kernel")


def load_traffic(name):
    """HBM bytes per launch measured by rocprofv3 --pmc (committed under profiles/), if present."""
    p = os.path.join(HERE, "profiles", f"traffic_gemm1_swiglu_{name}.json")
    if not os.path.exists(p):
        return None
    with open(p) as f:
        return json.load(f).get("bytes_per_launch")


def cpu_baseline(cfg, kw_dev, reps=3):
    """The CPU oracle on this host's cores, on the full headline workload (median of ``reps``)."""
    import oracle
    cores = max(1, min(16, os.cpu_count() or 1))
    torch.set_num_threads(cores)
    kw = {k: (v.cpu() if isinstance(v, torch.Tensor) else v) for k, v in kw_dev.items()}
    geom = cfg.geom
    oracle.moe_reference(kw, geom)  # warm-up
    ts = []
    for _ in range(reps):
        t0 = time.perf_counter()
        oracle.moe_reference(kw, geom)
        ts.append(time.perf_counter() - t0)
    ts.sort()
    sec = ts[len(ts) // 2]
    return sec, cores


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=100)
    ap.add_argument("--config", default="ds_t64", choices=sorted(jin.CONFIGS))
    ap.add_argument("--secondary", default="ds_t4096")
    ap.add_argument("--sweep", action="store_true", help="also measure ds_t16384_skew and qwen3_t1024")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="only run 5 device-to-device copies of 1 GiB (reference kernel for "
                         "scaling rocprofv3 FETCH_SIZE / WRITE_SIZE readings) and exit")
    args = ap.parse_args()
    if args.copy_calibration:
        src = torch.ones(1 << 30, dtype=torch.uint8, device="cuda:0")
        dst = torch.empty_like(src)
        for _ in range(5):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({"copy_bytes": 1 << 30, "copies": 5}))
        return
    if args.gpus != 1:
        print("bench.py measures one GPU only: this build runs the operator on a single MI355X "
              "(expert-parallel sharding across GPUs is a design note, not built); use --gpus 1.",
              file=sys.stderr)
        sys.exit(2)
    if not torch.cuda.is_available():
        print("bench.py needs a GPU", file=sys.stderr)
        sys.exit(2)
    dev = torch.device("cuda:0")
    _lib.lib()
    cfg = jin.CONFIGS[args.config]
    t0 = time.time()
    log(f"[bench] generating {cfg.geom.name} weights")
    wts = tuple(t.to(dev) for t in jin.make_weights(cfg.geom, seed=0))
    log(f"[bench] weights ready in {time.time() - t0:.1f}s; timing {cfg.name}")
    head, head_kw = measure(cfg, wts, args.steps, args.warmup, dev)
    log(f"[bench] {cfg.name}: {head['ms_per_call']:.4f} ms, {head['tflops']:.2f} TFLOPS, "
        f"{head['gb_s']:.0f} GB/s, stages {head['stage_ms']}")
    secondary = []
    names = [args.secondary] if args.secondary else []
    if args.sweep:
        names += ["ds_t16384_skew", "qwen3_t1024"]
    for n in names:
        c = jin.CONFIGS[n]
        if c.geom != cfg.geom:
            log(f"[bench] generating {c.geom.name} weights")
            w = tuple(t.to(dev) for t in jin.make_weights(c.geom, seed=0))
        else:
            w = wts
        # The full warm-up count: clocks settle over tens of ms of load, whatever the call length.
        r, _ = measure(c, w, max(5, args.steps // 4), args.warmup, dev)
        log(f"[bench] {c.name}: {r['ms_per_call']:.4f} ms, {r['tflops']:.2f} TFLOPS, "
            f"{r['gb_s']:.0f} GB/s, stages {r['stage_ms']}")
        secondary.append(r)
        del w
    quant = [measure_quant(T, cfg.geom.hidden, args.steps, args.warmup, dev) for T in (4096, 64)]
    for r in quant:
        log(f"[bench] activation quant T={r['tokens']}: {r['ms_per_call'] * 1e3:.1f} us, "
            f"{r['gb_s']:.0f} GB/s")
    cpu = None
    if not args.no_cpu_baseline:
        log("[bench] timing the CPU oracle")
        sec, cores = cpu_baseline(cfg, head_kw)
        cpu = {"value": head["algorithmic_flops"] / sec / 1e12, "unit": "TFLOPS", "cores": cores,
               "kind": "port", "ms_per_call": sec * 1e3,
               "sample": f"full {cfg.name} call (T={cfg.tokens}, {head['pairs']} local pairs), "
                         "median of 3 after 1 warm-up, torch-CPU fp32 dequantise-then-matmul"}
    g1 = head["gemm1"]
    out = {
        "metric": METRIC, "value": head["tflops"], "unit": "TFLOPS", "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup, "ms_per_step": head["ms_per_call"],
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "fp8-e4m3 (GEMM1) / bf16 (GEMM2), fp32 accumulate",
        "data": f"synthetic (seed {cfg.seed}: N(0,1) activations/logits, N(0,0.1) bias, "
                "N(0,0.02) weights, 128x128 block scales)",
        "config": {"workload": cfg.name, "geometry": cfg.geom.name, "tokens": cfg.tokens,
                   "seed": cfg.seed, "local_pairs": head["pairs"],
                   "active_local_experts": head["active_experts"],
                   "hidden": cfg.geom.hidden, "intermediate": cfg.geom.intermediate,
                   "local_experts": cfg.geom.local_experts, "top_k": cfg.geom.top_k,
                   "parallelism": "single GPU (EP rank 0 of 8: local experts 0..31)"},
        "roofline": {"bound": "hbm", "kernel": gemm1_kernel_name(cfg), "achieved": g1["gb_s"],
                     "peak": PEAK_HBM_GBS, "unit": "GB/s", "frac": g1["gb_s"] / PEAK_HBM_GBS,
                     "traffic": load_traffic(cfg.name), "algorithmic_bytes": g1["bytes"],
                     "avg_launch_ms": g1["ms"]},
        "cpu_baseline": cpu,
        "headline": head,
        "secondary": secondary,
        "activation_quant": quant,
    }
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
