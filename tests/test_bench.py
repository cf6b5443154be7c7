"""bench.py on the host: the one-GPU guard, the unit figures its roofline arithmetic rests on, and
the routing statistics it reads back from a call's workspace (no GPU needed)."""
import os
import subprocess
import sys

import torch

from justgoal_amd import _lib
from justgoal_amd.geometry import DS_V3, QWEN3, bytes_per_token, flops_per_pair, weight_bytes_per_expert
from justgoal_amd.moe import workspace_views

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, ROOT)
import bench  # noqa: E402


def test_more_than_one_gpu_exits_with_a_message():
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2"],
                       capture_output=True, text=True, timeout=300)
    assert r.returncode == 2
    assert "one GPU" in r.stderr and r.stdout == ""


def test_unit_figures():
    # DS-V3: 6*H*I FLOPs per local pair; W13 + W2 fp8 with their fp32 128x128 block scales per
    # active expert; fp8 row + scales + fp32 logits + bf16 output row per token
    assert flops_per_pair(DS_V3) == 88_080_384
    assert weight_bytes_per_expert(DS_V3) == 3 * 2048 * 7168 + 4 * (32 * 56 + 56 * 16)
    assert weight_bytes_per_expert(DS_V3) == 44_050_944
    assert bytes_per_token(DS_V3) == 22_752
    assert flops_per_pair(QWEN3) == 37_748_736
    flops, nbytes, g1_flops, g1_bytes = bench.algorithmic(DS_V3, 64, 55, 16, 40)
    assert flops == 55 * 88_080_384 and g1_flops == 55 * 2 * 7168 * 4096
    assert nbytes == 16 * 44_050_944 + 64 * 22_752 + 2 * 256
    # GEMM1 + SwiGLU: W13 + S13 of 16 experts, 40 routed token rows with scales, 55 bf16 C rows
    assert g1_bytes == 16 * (4096 * 7168 + 4 * 32 * 56) + 40 * (7168 + 4 * 56) + 55 * 2048 * 2


def test_routing_stats_read_the_given_workspace():
    T = 8
    ws = torch.zeros(_lib.workspace_layout(DS_V3, T)["total"], dtype=torch.uint8)
    v = workspace_views(DS_V3, T, ws)
    v["counts"][:] = 0
    v["counts"][3] = 2
    v["counts"][30] = 1
    v["pair_of"][:] = -1
    v["pair_of"][0, 1] = 0
    v["pair_of"][5, 0] = 1
    v["pair_of"][5, 7] = 2
    assert bench.routing_stats(DS_V3, T, ws) == (3, 2, 2)


def test_kernel_family_thresholds_match_the_library_source():
    import re
    src = open(os.path.join(ROOT, "justgoal_amd", "csrc", "moe_gemm.hip")).read()
    stream = int(re.search(r"constexpr int kStreamMaxRows = (\d+);", src).group(1))
    big = int(re.search(r"constexpr int kBigRows = (\d+);", src).group(1))
    g2 = int(re.search(r"constexpr int kG2TileMaxRows = (\d+);", src).group(1))
    assert (bench.GEMM1_STREAM_MAX_ROWS, bench.GEMM1_BIG_ROWS) == (stream, big)
    assert bench.GEMM2_TILE_MAX_ROWS == g2
    from justgoal_amd import inputs as jin
    names = {n: bench.gemm1_kernel_name(c) for n, c in jin.CONFIGS.items()}
    assert names["ds_t16"] == "gemm1_stream_kernel"
    assert names["ds_t64"] == "gemm1_stream_kernel"
    assert names["ds_t256"] == "gemm1_tile_kernel"
    assert names["ds_t512"] == "gemm1_big_kernel"
    assert names["ds_t4096"] == "gemm1_big_kernel"
    g2names = {n: bench.gemm2_kernel_name(c) for n, c in jin.CONFIGS.items()}
    assert g2names["ds_t16"] == g2names["ds_t192"] == "gemm2_tile_kernel"
    assert g2names["ds_t512"] == "gemm2_big_kernel"
    assert g2names["ds_t1024"] == "gemm2_big_kernel"


def test_gemm2_unit_figures_and_roofline_bound():
    # GEMM2: 2*I*H FLOPs per pair; W2 + S2 per active expert, bf16 C read and one bf16 row
    # written per pair
    f, b = bench.gemm2_algorithmic(DS_V3, 55, 16)
    assert f == 55 * 2 * 2048 * 7168
    assert b == 16 * (7168 * 2048 + 4 * 56 * 16) + 55 * 2048 * 2 + 55 * 7168 * 2
    # 55 pairs: bytes dominate (HBM); 68197 pairs: FLOPs dominate (MFMA)
    r = bench.roofline_block("gemm2", "k", 0.05, f, b, bench.PEAK_BF16_TFLOPS, "none")
    assert r["bound"] == "hbm" and abs(r["achieved"] - b / 0.05e-3 / 1e9) < 1e-6
    f, b = bench.gemm2_algorithmic(DS_V3, 68197, 23)
    r = bench.roofline_block("gemm2", "k", 2.0, f, b, bench.PEAK_BF16_TFLOPS, "none")
    assert r["bound"] == "mfma" and r["unit"] == "TFLOP/s"
    assert abs(r["frac"] - f / 2e-3 / 1e12 / 2500.0) < 1e-9


def test_committed_profiles_name_the_kernels_bench_reports():
    """profiles/kernel_avg_us.json (the rocprofv3 trace of this bench) has an entry for the kernel
    family bench.py names for each GEMM of each default workload, so every roofline block carries
    its rocprof figure; a changed kernel-family threshold without retaken profiles fails here."""
    import json
    from justgoal_amd import inputs as jin
    with open(os.path.join(ROOT, "profiles", "kernel_avg_us.json")) as f:
        prof = json.load(f)["workloads"]
    for name in bench.DEFAULT_WORKLOADS:
        cfg = jin.CONFIGS[name]
        for kernel in (bench.gemm1_kernel_name(cfg), bench.gemm2_kernel_name(cfg)):
            assert kernel in prof[name], (name, kernel, sorted(prof[name]))
            assert bench.load_rocprof_avg_us(kernel, name) == prof[name][kernel]["average_us"] > 0
    r = bench.roofline_block("gemm1_swiglu", bench.gemm1_kernel_name(jin.CONFIGS["ds_t64"]), 0.075,
                             1.0, 470e6, bench.PEAK_FP8_TFLOPS, "ds_t64")
    us = prof["ds_t64"][r["kernel"]]["average_us"]
    assert abs(r["frac_rocprof"] - 470e6 / (us * 1e-6) / 1e9 / bench.PEAK_HBM_GBS) < 1e-9
