"""Seeded synthetic inputs for the benchmark configurations.

Distributions (the same in every configuration):
* hidden states: bf16 N(0,1), quantised to e4m3 with per-token 1x128 scales (amax/448), scales
  stored transposed as [H/128, T] -- the layout of the operator's ``hidden_states_scale``;
* W13 [E_l, 2I, H] and W2 [E_l, H, I]: N(0, 0.02) quantised in 128x128 blocks with scale
  amax/448, scales [E_l, 2I/128, H/128] and [E_l, H/128, I/128];
* router logits fp32 N(0,1) [T, E_g]; routing bias bf16 N(0, 0.1) [E_g];
* routed_scaling_factor 2.5 for DS-V3 (1.0 for softmax routing), local_expert_offset 0.

Generation is on the CPU from a ``torch.Generator`` seed, so the same tensors are reproducible on
any machine; they are then moved to ``device``.
"""
from __future__ import annotations

from dataclasses import dataclass

import torch

from .geometry import BLOCK, DS_V3, QWEN3, ROUTING_DS, Geometry

F8 = torch.float8_e4m3fn
F8_MAX = 448.0


@dataclass(frozen=True)
class Config:
    name: str
    geom: Geometry
    tokens: int
    skew_experts: int = 0      # number of local experts whose logits get +skew_offset
    skew_offset: float = 0.0
    seed: int = 0              # activation seed of the measured workload


# The measured workloads use seed 2. The routing bias is one draw per seed, and it sets how many
# of a token's picks land in the local group (experts 0..31): over seeds 0..31 the T=64 batch
# gets a median of 55 local pairs on 16 experts and the T=4096 batch 3537 pairs on 27 experts.
# Seed 2 sits at that median (55 / 16 and 4066 / 26); seed 0 is the lightest draw of the 32
# (18 / 8 and 1299 / 21) and stays the seed of the T=16 plumbing case and its fixtures.
BENCH_SEED = 2

CONFIGS = {
    "ds_t16": Config("ds_t16", DS_V3, 16),
    "ds_t64": Config("ds_t64", DS_V3, 64, seed=BENCH_SEED),
    "ds_t4096": Config("ds_t4096", DS_V3, 4096, seed=BENCH_SEED),
    "ds_t16384_skew": Config("ds_t16384_skew", DS_V3, 16384, skew_experts=8, skew_offset=3.0,
                             seed=BENCH_SEED),
    "qwen3_t1024": Config("qwen3_t1024", QWEN3, 1024, seed=BENCH_SEED),
    "qwen3_t128": Config("qwen3_t128", QWEN3, 128, seed=BENCH_SEED),
    "qwen3_t512": Config("qwen3_t512", QWEN3, 512, seed=BENCH_SEED),
    # prefill chunks between the decode and the large-batch cases (LDS-tile kernels)
    "ds_t32": Config("ds_t32", DS_V3, 32, seed=BENCH_SEED),
    "ds_t128": Config("ds_t128", DS_V3, 128, seed=BENCH_SEED),
    "ds_t192": Config("ds_t192", DS_V3, 192, seed=BENCH_SEED),
    "ds_t256": Config("ds_t256", DS_V3, 256, seed=BENCH_SEED),
    "ds_t512": Config("ds_t512", DS_V3, 512, seed=BENCH_SEED),
    "ds_t768": Config("ds_t768", DS_V3, 768, seed=BENCH_SEED),
    "ds_t1024": Config("ds_t1024", DS_V3, 1024, seed=BENCH_SEED),
    "ds_t2048": Config("ds_t2048", DS_V3, 2048, seed=BENCH_SEED),
}


def quantize_rows_1x128(x: torch.Tensor):
    """bf16/fp32 [T, H] -> (fp8 [T, H], fp32 scales [H/128, T]) with scale = amax/448 per 1x128 block."""
    T, H = x.shape
    xb = x.float().reshape(T, H // BLOCK, BLOCK)
    amax = xb.abs().amax(dim=2)
    scale = torch.where(amax > 0, amax / F8_MAX, torch.ones_like(amax))
    q = (xb / scale[:, :, None]).clamp(-F8_MAX, F8_MAX).to(F8).reshape(T, H)
    return q, scale.t().contiguous()


def quantize_blocks_128x128(w: torch.Tensor):
    """fp32 [..., R, C] -> (fp8 [..., R, C], fp32 scales [..., R/128, C/128])."""
    *lead, R, C = w.shape
    wb = w.reshape(*lead, R // BLOCK, BLOCK, C // BLOCK, BLOCK)
    amax = wb.abs().amax(dim=(-3, -1))
    scale = torch.where(amax > 0, amax / F8_MAX, torch.ones_like(amax))
    q = (wb / scale[..., :, None, :, None]).clamp(-F8_MAX, F8_MAX).to(F8).reshape(*lead, R, C)
    return q, scale


def make_weights(geom: Geometry, seed: int = 0, device="cpu", experts: int | None = None):
    """Quantised expert weights, generated one expert at a time to bound host memory."""
    E = geom.local_experts if experts is None else experts
    H, I = geom.hidden, geom.intermediate
    g = torch.Generator().manual_seed(seed * 1000003 + 17)
    w13 = torch.empty(E, 2 * I, H, dtype=F8, device=device)
    s13 = torch.empty(E, 2 * I // BLOCK, H // BLOCK, dtype=torch.float32, device=device)
    w2 = torch.empty(E, H, I, dtype=F8, device=device)
    s2 = torch.empty(E, H // BLOCK, I // BLOCK, dtype=torch.float32, device=device)
    for e in range(E):
        q, s = quantize_blocks_128x128(torch.randn(2 * I, H, generator=g) * 0.02)
        w13[e].copy_(q)
        s13[e].copy_(s)
        q, s = quantize_blocks_128x128(torch.randn(H, I, generator=g) * 0.02)
        w2[e].copy_(q)
        s2[e].copy_(s)
    return w13, s13, w2, s2


def make_routing_inputs(geom: Geometry, T: int, seed: int = 0, skew_experts: int = 0,
                        skew_offset: float = 0.0, local_offset: int = 0):
    """(logits fp32 [T, E], bias bf16 [E]) exactly as ``make_activations`` draws them."""
    # one generator per tensor, so the bias does not depend on T
    g_bias = torch.Generator().manual_seed(seed * 7919 + 1)
    g_logits = torch.Generator().manual_seed(seed * 7919 + 2)
    bias = (torch.randn(geom.num_experts, generator=g_bias) * 0.1).to(torch.bfloat16)
    logits = torch.randn(T, geom.num_experts, generator=g_logits)
    if skew_experts:
        logits[:, local_offset:local_offset + skew_experts] += skew_offset
    return logits, bias


def make_activations(geom: Geometry, T: int, seed: int = 0, device="cpu", skew_experts: int = 0,
                     skew_offset: float = 0.0, local_offset: int = 0):
    logits, bias = make_routing_inputs(geom, T, seed, skew_experts, skew_offset, local_offset)
    g_hs = torch.Generator().manual_seed(seed * 7919 + 3)
    hs_bf16 = torch.randn(T, geom.hidden, generator=g_hs).to(torch.bfloat16)
    hs, hs_scale = quantize_rows_1x128(hs_bf16)
    return dict(routing_logits=logits.to(device), routing_bias=bias.to(device),
                hidden_states=hs.to(device), hidden_states_scale=hs_scale.to(device))


def make_inputs(cfg: Config | str, seed: int | None = None, device="cpu",
                tokens: int | None = None, weights=None):
    """All ten operator arguments (reference names) for a configuration (seed: the config's)."""
    if isinstance(cfg, str):
        cfg = CONFIGS[cfg]
    if seed is None:
        seed = cfg.seed
    geom = cfg.geom
    T = cfg.tokens if tokens is None else tokens
    d = make_activations(geom, T, seed, device, cfg.skew_experts, cfg.skew_offset)
    if weights is None:
        weights = make_weights(geom, seed, device)
    w13, s13, w2, s2 = weights
    d.update(gemm1_weights=w13, gemm1_weights_scale=s13, gemm2_weights=w2, gemm2_weights_scale=s2,
             local_expert_offset=0,
             routed_scaling_factor=2.5 if geom.routing_method == ROUTING_DS else 1.0)
    return d
