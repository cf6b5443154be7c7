"""moe_run_noalloc (the entry point that allocates nothing) against moe_run_ex with a caller
workspace, through the C ABI: bit-identical outputs on two calls in a row, the second with a
smaller batch (the scratch array keeps the first call's contents), at both model geometries
and both GEMM kernel families; a call too large for the scratch array is refused with
MOE_ERR_SCRATCH_SIZE before anything is enqueued."""
import ctypes
import sys

import pytest
import torch

from justgoal_amd import _lib
from justgoal_amd import inputs as jin
from justgoal_amd.geometry import DS_V3, QWEN3

pytestmark = pytest.mark.gpu

MOE_ERR_SCRATCH_SIZE = -4


def _args(geom, w, act, out):
    return [ctypes.byref(geom.c_struct()), act["routing_logits"].data_ptr(),
            act["routing_bias"].data_ptr(), act["hidden_states"].data_ptr(),
            act["hidden_states_scale"].data_ptr(), w[0].data_ptr(), w[1].data_ptr(),
            w[2].data_ptr(), w[3].data_ptr(), 0,
            2.5 if geom.routing_method == 0 else 1.0, out.data_ptr()]


def _both(geom, w, T, seed, dev):
    L = _lib.lib()
    act = {k: v.to(dev) for k, v in jin.make_activations(geom, T, seed=seed).items()}
    stream = torch.cuda.current_stream(dev).cuda_stream
    ref = torch.full((T, geom.hidden), float("nan"), dtype=torch.bfloat16, device=dev)
    ws = torch.empty(_lib.workspace_layout(geom, T)["total"], dtype=torch.uint8, device=dev)
    rc = L.moe_run_ex(*_args(geom, w, act, ref), ws.data_ptr(), T, stream)
    assert rc == 0, rc
    got = torch.full((T, geom.hidden), float("nan"), dtype=torch.bfloat16, device=dev)
    rc = L.moe_run_noalloc(*_args(geom, w, act, got), T, stream)
    assert rc == 0, rc
    torch.cuda.synchronize()
    return got, ref


@pytest.mark.parametrize("geom,sizes", [(DS_V3, (480, 64)), (DS_V3, (256, 16)),
                                        (QWEN3, (800, 96))])
def test_noalloc_matches_workspace_entry(gpu, geom, sizes):
    w = tuple(t.to(gpu) for t in jin.make_weights(geom, seed=3))
    for i, T in enumerate(sizes):
        print(f"noalloc: {geom.name} call {i} T={T}", flush=True)
        got, ref = _both(geom, w, T, seed=40 + i, dev=gpu)
        assert torch.equal(got, ref), f"call {i} (T={T}) differs from moe_run_ex"
    # the entry point's contract: a call allocates no device memory (free bytes unchanged around
    # a call whose inputs and output already exist)
    L = _lib.lib()
    T = sizes[-1]
    act = {k: v.to(gpu) for k, v in jin.make_activations(geom, T, seed=7).items()}
    out = torch.empty((T, geom.hidden), dtype=torch.bfloat16, device=gpu)
    stream = torch.cuda.current_stream(gpu).cuda_stream
    torch.cuda.synchronize()
    free0 = torch.cuda.mem_get_info(gpu)[0]
    assert L.moe_run_noalloc(*_args(geom, w, act, out), T, stream) == 0
    torch.cuda.synchronize()
    assert torch.cuda.mem_get_info(gpu)[0] == free0, "moe_run_noalloc changed free device memory"
    del w


def test_noalloc_refuses_a_batch_larger_than_its_scratch(gpu):
    L = _lib.lib()
    g = DS_V3
    T = 504  # 64 MiB of scratch holds the DS-V3 workspace of up to 503 tokens
    assert _lib.workspace_layout(g, T)["total"] > 64 << 20 >= _lib.workspace_layout(g, 503)["total"]
    out = torch.empty((T, g.hidden), dtype=torch.bfloat16, device=gpu)
    # the size check comes before any pointer is used: null inputs are fine here
    rc = L.moe_run_noalloc(ctypes.byref(g.c_struct()), None, None, None, None, None, None, None,
                           None, 0, 2.5, out.data_ptr(), T, None)
    assert rc == MOE_ERR_SCRATCH_SIZE
    assert b"scratch" in L.moe_error_string(rc)
