"""CPU oracle for the FP8 block-scale MoE hot path.

TEST INFRASTRUCTURE ONLY: the checker the HIP product is compared against. Only ``tests/``,
``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline`` leg may import it, and only as
the checker or the reported CPU baseline; the product package never imports it.
"""
from .moe_oracle import (  # noqa: F401
    ROUTING_DS, ROUTING_SOFTMAX, oracle_lib, route, route_numpy, permute, dequant_blocks,
    dequant_activations, moe_reference, quantize_activations, sigmoid_f32, sigmoid_numpy, exp_f32,
    exp_numpy, fma32,
)
