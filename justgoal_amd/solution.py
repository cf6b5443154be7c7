"""Writes this operator as a flashinfer-bench solution directory.

Layout and schema follow the reference's MoE solutions
(goal_full_shape/opus-4.8/moe_fp8_fwd/MOEDIR/solution.json:1-20 and
kda05_reproduction_single_shape/fable-5.1/moe_fp8_fwd/t1/solution.json): ``solution.json`` with
name / definition / author / spec (language, target_hardware, entry_point ``main.py::run``,
dependencies, destination_passing_style, binding) / sources / description, next to the source
files it lists. ``main.py`` is ``solution_main.py`` of this package; the HIP sources and the C
header ship beside it.

``python -m justgoal_amd.solution DEST [--embed] [--with-lib] [--dps]``: ``--embed`` also stores
each source's text in solution.json (the opus-4.8 form); ``--with-lib`` ships the built
libjustgoal_moe.so so the entry point loads it instead of compiling; ``--dps`` declares the
destination-passing form (the harness passes ``output`` as an eleventh argument, t901/main.py).
"""
from __future__ import annotations

import argparse
import json
import os
import shutil

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
ROOT = os.path.dirname(HERE)
DEFINITION = "moe_fp8_block_scale_ds_routing_topk8_ng8_kg4_e32_h7168_i2048"


def source_files():
    """(name in the solution, path in this repository) of every shipped source."""
    files = [("main.py", os.path.join(HERE, "solution_main.py")),
             ("justgoal_moe.h", os.path.join(ROOT, "include", "justgoal_moe.h"))]
    for name in sorted(os.listdir(CSRC)):
        if name.endswith((".hip", ".h")):
            files.append((name, os.path.join(CSRC, name)))
    return files


def write_solution(dest: str, embed: bool = False, with_lib: bool = False,
                   dps: bool = False) -> str:
    """Writes the solution directory; returns the path of solution.json."""
    os.makedirs(dest, exist_ok=True)
    sources = []
    for name, path in source_files():
        shutil.copyfile(path, os.path.join(dest, name))
        entry = {"path": name}
        if embed:
            with open(path) as f:
                entry["content"] = f.read()
        sources.append(entry)
    if with_lib:
        lib = os.path.join(HERE, "libjustgoal_moe.so")
        if not os.path.isfile(lib):
            raise FileNotFoundError(f"{lib} is not built")
        shutil.copyfile(lib, os.path.join(dest, "libjustgoal_moe.so"))
    sol = {
        "name": "justgoal-amd-moe-fp8-mi355x",
        "definition": DEFINITION,
        "author": "justgoal_amd",
        "spec": {
            "language": "python",
            "target_hardware": ["AMD MI355X"],
            "entry_point": "main.py::run",
            "dependencies": [],
            "destination_passing_style": dps,
            "binding": None,
        },
        "sources": sources,
        "description": "HIP/CDNA4 FP8 block-scale MoE: DPP routing, bitmask permute, LDS-DMA "
                       "weight-streaming and large-tile fp8/bf16 MFMA grouped GEMMs, weighted "
                       "combine; C ABI bound through ctypes.",
    }
    out = os.path.join(dest, "solution.json")
    with open(out, "w") as f:
        json.dump(sol, f, indent=1)
    return out


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("dest")
    ap.add_argument("--embed", action="store_true")
    ap.add_argument("--with-lib", action="store_true")
    ap.add_argument("--dps", action="store_true")
    a = ap.parse_args()
    print(write_solution(a.dest, embed=a.embed, with_lib=a.with_lib, dps=a.dps))


if __name__ == "__main__":
    main()
