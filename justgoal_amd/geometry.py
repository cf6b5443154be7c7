"""MoE geometries and the operator's fixed constants.

The DeepSeek-V3 geometry is the one the reference operator is specialised to
(goal_full_shape/opus-4.8/moe_fp8_fwd/MOEDIR/main.py:5-18; moe_common.cuh:11-20):
H=7168, I=2048, 256 global experts of which 32 are local, top-8, 8 groups keep 4, 128-wide
scale blocks. The Qwen3-235B-A22B-style geometry (H=4096, I=1536, 128 experts all local,
softmax top-8) has no code in the reference and is the second benchmark geometry.
"""
from __future__ import annotations

import ctypes
from dataclasses import dataclass

BLOCK = 128
ROUTING_DS = 0        # sigmoid + bias, group-limited top-k, renormalise x scaling factor
ROUTING_SOFTMAX = 1   # softmax top-k, renormalise


@dataclass(frozen=True)
class Geometry:
    hidden: int
    intermediate: int
    num_experts: int
    local_experts: int
    top_k: int
    n_group: int
    topk_group: int
    routing_method: int
    name: str = ""

    def c_struct(self) -> "MoeGeometryC":
        return MoeGeometryC(self.hidden, self.intermediate, self.num_experts, self.local_experts,
                            self.top_k, self.n_group, self.topk_group, self.routing_method)


class MoeGeometryC(ctypes.Structure):
    """Mirror of ``moe_geometry`` in include/justgoal_moe.h."""
    _fields_ = [(n, ctypes.c_int) for n in (
        "hidden", "intermediate", "num_experts", "local_experts", "top_k", "n_group",
        "topk_group", "routing_method")]


DS_V3 = Geometry(7168, 2048, 256, 32, 8, 8, 4, ROUTING_DS, "DS-V3")
QWEN3 = Geometry(4096, 1536, 128, 128, 8, 1, 1, ROUTING_SOFTMAX, "Qwen3-235B-A22B")


def flops_per_pair(g: Geometry) -> int:
    """Algorithmic FLOPs of one (token, local expert) pair: 2*H*2I (GEMM1) + 2*I*H (GEMM2)."""
    return 6 * g.hidden * g.intermediate


def weight_bytes_per_expert(g: Geometry) -> int:
    """fp8 W13 + W2 plus their fp32 128x128 block scales."""
    H, I = g.hidden, g.intermediate
    return 2 * I * H + H * I + 4 * ((2 * I // BLOCK) * (H // BLOCK) + (H // BLOCK) * (I // BLOCK))


def bytes_per_token(g: Geometry) -> int:
    """fp8 activations + fp32 scales + fp32 logits + bf16 output."""
    H = g.hidden
    return H + 4 * (H // BLOCK) + 4 * g.num_experts + 2 * H
