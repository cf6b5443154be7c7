"""The flashinfer-bench solution packaging: schema of solution.json (the reference's fields,
goal_full_shape/opus-4.8/moe_fp8_fwd/MOEDIR/solution.json:1-20), every listed source shipped,
the entry point importable without a GPU, and the shipped sources compiling on their own.
On a GPU, the packaged entry point gives exactly the library's output."""
import importlib.util
import json
import os
import subprocess
import sys

import pytest
import torch

from justgoal_amd import solution


def load_main(d):
    spec = importlib.util.spec_from_file_location(f"sol_main_{abs(hash(d))}", os.path.join(d, "main.py"))
    m = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(m)
    return m


def test_schema_and_sources(tmp_path):
    p = solution.write_solution(str(tmp_path), embed=True)
    d = json.load(open(p))
    assert set(d) == {"name", "definition", "author", "spec", "sources", "description"}
    assert d["definition"] == "moe_fp8_block_scale_ds_routing_topk8_ng8_kg4_e32_h7168_i2048"
    assert set(d["spec"]) == {"language", "target_hardware", "entry_point", "dependencies",
                              "destination_passing_style", "binding"}
    assert d["spec"]["entry_point"] == "main.py::run"
    assert d["spec"]["destination_passing_style"] is False
    names = [s["path"] for s in d["sources"]]
    assert "main.py" in names and "justgoal_moe.h" in names
    for s in d["sources"]:
        with open(tmp_path / s["path"]) as f:
            assert f.read() == s["content"]
    m = load_main(str(tmp_path))
    assert callable(m.run)
    for src in m.SOURCES:  # every source the build compiles is shipped
        assert src in names


def test_dps_flag(tmp_path):
    d = json.load(open(solution.write_solution(str(tmp_path), dps=True)))
    assert d["spec"]["destination_passing_style"] is True
    import inspect
    params = list(inspect.signature(load_main(str(tmp_path)).run).parameters)
    assert len(params) == 11 and params[-1] == "output"


def test_shipped_sources_compile(tmp_path):
    """The entry point's own build recipe, on the shipped files only (hipcc cross-compiles)."""
    solution.write_solution(str(tmp_path))
    m = load_main(str(tmp_path))
    so = m.build(out_dir=str(tmp_path / "build"))
    assert os.path.getsize(so) > 0
    out = subprocess.run(["nm", "-D", "--defined-only", so], capture_output=True, text=True).stdout
    for sym in ("moe_run", "moe_workspace_bytes", "moe_error_string"):
        assert f" {sym}" in out


@pytest.mark.gpu
def test_entry_point_matches_library(gpu, tmp_path):
    from justgoal_amd import inputs as jin
    from justgoal_amd.geometry import DS_V3
    from justgoal_amd.moe import run
    solution.write_solution(str(tmp_path), with_lib=True)
    m = load_main(str(tmp_path))
    act = jin.make_activations(DS_V3, 16, seed=0)
    w = jin.make_weights(DS_V3, seed=0)
    args = [act["routing_logits"], act["routing_bias"], act["hidden_states"],
            act["hidden_states_scale"], *w]
    args = [a.to(gpu) for a in args]
    got = m.run(*args, torch.tensor(0), torch.tensor(2.5))
    ref = run(*args, 0, 2.5)
    dst = torch.full_like(ref, float("nan"))
    assert m.run(*args, 0, 2.5, dst) is dst  # destination-passing form
    torch.cuda.synchronize()
    assert torch.equal(got, ref)
    assert torch.equal(dst, ref)
    with pytest.raises(ValueError):
        m.run(*args, 0, 2.5, torch.empty(ref.shape, dtype=torch.float32, device=gpu))
