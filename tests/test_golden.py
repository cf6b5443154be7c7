"""The oracle against the committed fixtures of tests/golden (written by make_golden.py), and --
on a GPU -- the HIP operator against the same fixtures."""
import json
import os

import numpy as np
import pytest
import torch

import oracle
from justgoal_amd import inputs as jin
from justgoal_amd.geometry import DS_V3, Geometry

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def load(name):
    return dict(np.load(os.path.join(GOLDEN, name), allow_pickle=False))


def tiny_inputs():
    f = load("pipeline_tiny.npz")
    geom = Geometry(*[int(x) for x in f["geometry"]], name="tiny")
    inp = dict(
        routing_logits=torch.from_numpy(f["routing_logits"]),
        routing_bias=torch.from_numpy(f["routing_bias"]).view(torch.bfloat16),
        hidden_states=torch.from_numpy(f["hidden_states"]).view(torch.float8_e4m3fn),
        hidden_states_scale=torch.from_numpy(f["hidden_states_scale"]),
        gemm1_weights=torch.from_numpy(f["gemm1_weights"]).view(torch.float8_e4m3fn),
        gemm1_weights_scale=torch.from_numpy(f["gemm1_weights_scale"]),
        gemm2_weights=torch.from_numpy(f["gemm2_weights"]).view(torch.float8_e4m3fn),
        gemm2_weights_scale=torch.from_numpy(f["gemm2_weights_scale"]),
        local_expert_offset=int(f["local_expert_offset"]),
        routed_scaling_factor=float(f["routed_scaling_factor"]))
    return geom, inp, torch.from_numpy(f["out_bf16"]).view(torch.bfloat16)


@pytest.mark.parametrize("name,off", [("routing_ds_t16.npz", 0), ("routing_ds_ties.npz", 96)])
def test_routing_fixtures(name, off):
    f = load(name)
    lg = torch.from_numpy(f["logits"])
    b = torch.from_numpy(f["bias_bf16"]).view(torch.bfloat16)
    idx, w = oracle.route(lg, b, DS_V3, 2.5)
    np.testing.assert_array_equal(idx, f["topk_idx"])
    np.testing.assert_array_equal(w.view(np.uint32), f["topk_w"].view(np.uint32))
    p = oracle.permute(idx, w, off, DS_V3.local_experts)
    for k in ("counts", "offsets", "sorted_tok", "pair_of"):
        np.testing.assert_array_equal(p[k], f[k])


def test_config0_inputs_regenerate():
    """The seeded generator reproduces the fixture's logits and bias bit for bit."""
    f = load("routing_ds_t16.npz")
    act = jin.make_activations(DS_V3, 16, seed=0)
    np.testing.assert_array_equal(act["routing_logits"].numpy(), f["logits"])
    np.testing.assert_array_equal(act["routing_bias"].view(torch.int16).numpy(), f["bias_bf16"])


def test_tiny_pipeline_fixture():
    geom, inp, ref = tiny_inputs()
    out = oracle.moe_reference(inp, geom)
    torch.testing.assert_close(out.float(), ref.float(), rtol=1e-2, atol=1e-2)


def test_config0_output_rows():
    f = load("output_ds_t16_rows.npz")
    meta = json.load(open(os.path.join(GOLDEN, "output_ds_t16.json")))
    assert meta["config"] == "ds_t16"
    w = jin.make_weights(DS_V3, seed=0)
    act = jin.make_activations(DS_V3, 16, seed=0)
    inp = dict(act, gemm1_weights=w[0], gemm1_weights_scale=w[1], gemm2_weights=w[2],
               gemm2_weights_scale=w[3], local_expert_offset=0, routed_scaling_factor=2.5)
    out = oracle.moe_reference(inp, DS_V3)
    ref = torch.from_numpy(f["out_bf16"]).view(torch.bfloat16)
    torch.testing.assert_close(out[f["rows"]].float(), ref.float(), rtol=1e-2, atol=1e-2)


@pytest.mark.gpu
def test_gpu_tiny_pipeline_fixture(gpu):
    from justgoal_amd.moe import run, workspace, workspace_views
    geom, inp, ref = tiny_inputs()
    d = {k: (v.to(gpu) if isinstance(v, torch.Tensor) else v) for k, v in inp.items()}
    out = run(**d, geometry=geom)
    torch.testing.assert_close(out.cpu().float(), ref.float(), rtol=2e-2, atol=2e-2)


@pytest.mark.gpu
@pytest.mark.parametrize("name,off", [("routing_ds_t16.npz", 0), ("routing_ds_ties.npz", 96)])
def test_gpu_routing_fixtures(gpu, name, off):
    from justgoal_amd.moe import route
    f = load(name)
    lg = torch.from_numpy(f["logits"]).to(gpu)
    b = torch.from_numpy(f["bias_bf16"]).view(torch.bfloat16).to(gpu)
    v = route(lg, b, off, 2.5, geometry=DS_V3)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(v["topk_idx"].cpu().numpy(), f["topk_idx"])
    np.testing.assert_array_equal(v["topk_w"].cpu().numpy().view(np.uint32),
                                  f["topk_w"].view(np.uint32))
    for k in ("counts", "offsets", "pair_of"):
        np.testing.assert_array_equal(v[k].cpu().numpy(), f[k])
    n = int(f["offsets"][-1])
    np.testing.assert_array_equal(v["sorted_tok"][:n].cpu().numpy(), f["sorted_tok"])
