"""Writes the committed golden fixtures of this directory from the CPU oracle.

The reference has no golden vectors, known-answer tests or fixtures for this operator (its
PyTorch definition lives in the external flashinfer-bench dataset, which is not vendored), so
these fixtures are the oracle's own outputs on seeded inputs. They pin the oracle against
regressions; the oracle itself is pinned by tests/test_oracle.py.

    python tests/golden/make_golden.py
"""
import hashlib
import json
import os
import sys

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)

import oracle  # noqa: E402
from justgoal_amd import inputs as jin  # noqa: E402
from justgoal_amd.geometry import DS_V3, ROUTING_DS, Geometry  # noqa: E402

# tiny geometry for a full-pipeline fixture small enough to commit
TINY = Geometry(128, 128, 64, 4, 4, 4, 2, ROUTING_DS, "tiny")


def routing_fixture(logits, bias, geom, rsf, off):
    idx, w = oracle.route(logits, bias, geom, rsf)
    p = oracle.permute(idx, w, off, geom.local_experts)
    return dict(logits=logits.numpy(), bias_bf16=bias.view(torch.int16).numpy(), topk_idx=idx,
                topk_w=w, counts=p["counts"], offsets=p["offsets"], sorted_tok=p["sorted_tok"],
                sorted_w=p["sorted_w"], pair_of=p["pair_of"])


def main():
    # 1. DS-V3 config 0 (T=16, seed 0) routing + permute
    act = jin.make_activations(DS_V3, 16, seed=0)
    np.savez_compressed(os.path.join(HERE, "routing_ds_t16.npz"),
                        **routing_fixture(act["routing_logits"], act["routing_bias"], DS_V3, 2.5, 0))

    # 2. many exact ties (logits on a 0.25 grid, zero bias), DS-V3 routing, EP rank 3
    g = torch.Generator().manual_seed(7)
    lg = torch.round(torch.randn(64, 256, generator=g) * 4) / 4
    np.savez_compressed(os.path.join(HERE, "routing_ds_ties.npz"),
                        **routing_fixture(lg, torch.zeros(256, dtype=torch.bfloat16), DS_V3, 2.5, 96))

    # 3. tiny-geometry full pipeline
    T = 24
    act = jin.make_activations(TINY, T, seed=3)
    w13, s13, w2, s2 = jin.make_weights(TINY, seed=3)
    inp = dict(act, gemm1_weights=w13, gemm1_weights_scale=s13, gemm2_weights=w2,
               gemm2_weights_scale=s2, local_expert_offset=0, routed_scaling_factor=2.5)
    out = oracle.moe_reference(inp, TINY)
    np.savez_compressed(
        os.path.join(HERE, "pipeline_tiny.npz"),
        geometry=np.array([TINY.hidden, TINY.intermediate, TINY.num_experts, TINY.local_experts,
                           TINY.top_k, TINY.n_group, TINY.topk_group, TINY.routing_method]),
        routing_logits=act["routing_logits"].numpy(),
        routing_bias=act["routing_bias"].view(torch.int16).numpy(),
        hidden_states=act["hidden_states"].view(torch.uint8).numpy(),
        hidden_states_scale=act["hidden_states_scale"].numpy(),
        gemm1_weights=w13.view(torch.uint8).numpy(), gemm1_weights_scale=s13.numpy(),
        gemm2_weights=w2.view(torch.uint8).numpy(), gemm2_weights_scale=s2.numpy(),
        local_expert_offset=np.array(0), routed_scaling_factor=np.array(2.5, np.float32),
        out_bf16=out.view(torch.int16).numpy())

    # 4. DS-V3 config 0 full output: a digest plus four sampled rows
    w = jin.make_weights(DS_V3, seed=0)
    act = jin.make_activations(DS_V3, 16, seed=0)
    inp = dict(act, gemm1_weights=w[0], gemm1_weights_scale=w[1], gemm2_weights=w[2],
               gemm2_weights_scale=w[3], local_expert_offset=0, routed_scaling_factor=2.5)
    out = oracle.moe_reference(inp, DS_V3)
    rows = [0, 5, 10, 15]
    np.savez_compressed(os.path.join(HERE, "output_ds_t16_rows.npz"), rows=np.array(rows),
                        out_bf16=out[rows].view(torch.int16).numpy())
    with open(os.path.join(HERE, "output_ds_t16.json"), "w") as f:
        json.dump({"config": "ds_t16", "seed": 0,
                   "sha256_bf16": hashlib.sha256(out.view(torch.int16).numpy().tobytes()).hexdigest(),
                   "note": "informational; the test compares sampled rows within tolerance because "
                           "CPU matmul summation order may differ between machines"}, f, indent=1)
    print("fixtures written to", HERE)


if __name__ == "__main__":
    main()
