"""ctypes binding of ``libjustgoal_moe.so`` (the C ABI declared in include/justgoal_moe.h).

The library must have been built (``justgoal_amd.build.build()``); there is no fallback: a missing
library raises instead of silently computing elsewhere.
"""
from __future__ import annotations

import ctypes
import os

from .geometry import MoeGeometryC

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.environ.get("JUSTGOAL_MOE_LIB") or os.path.join(_HERE, "libjustgoal_moe.so")

# Every symbol include/justgoal_moe.h declares.
EXPORTED = ("moe_run", "moe_workspace_bytes", "moe_run_ex", "moe_workspace_bytes_ex",
            "moe_route_ex", "moe_workspace_layout", "moe_set_stage_events", "moe_error_string",
            "moe_quantize_activations", "moe_run_noalloc")

MOE_WS_NUM_REGIONS = 11
WS_REGIONS = ("topk_idx", "topk_w", "pair_of", "counts", "offsets", "sorted_tok", "sorted_w", "C",
              "partial", "chunk_counts", "pair_dst")

_LIB = None


class MoeError(RuntimeError):
    pass


def lib() -> ctypes.CDLL:
    global _LIB
    if _LIB is None:
        if not os.path.exists(LIB_PATH):
            raise MoeError(f"{LIB_PATH} is not built; run justgoal_amd.build.build() first")
        L = ctypes.CDLL(LIB_PATH)
        P, I, F = ctypes.c_void_p, ctypes.c_int, ctypes.c_float
        G = ctypes.POINTER(MoeGeometryC)
        L.moe_run.argtypes = [P] * 8 + [I, F, P, P, I, P]
        L.moe_run.restype = I
        L.moe_workspace_bytes.argtypes = [I]
        L.moe_workspace_bytes.restype = I
        L.moe_run_ex.argtypes = [G] + [P] * 8 + [I, F, P, P, I, P]
        L.moe_run_ex.restype = I
        L.moe_workspace_bytes_ex.argtypes = [G, I]
        L.moe_workspace_bytes_ex.restype = ctypes.c_int64
        L.moe_route_ex.argtypes = [G, P, P, I, F, P, I, P]
        L.moe_route_ex.restype = I
        L.moe_workspace_layout.argtypes = [G, I, ctypes.POINTER(ctypes.c_int64)]
        L.moe_workspace_layout.restype = I
        L.moe_set_stage_events.argtypes = [ctypes.POINTER(ctypes.c_void_p), I]
        L.moe_set_stage_events.restype = I
        L.moe_run_noalloc.argtypes = [G] + [P] * 8 + [I, F, P, I, P]
        L.moe_run_noalloc.restype = I
        L.moe_quantize_activations.argtypes = [P, I, I, P, P, P]
        L.moe_quantize_activations.restype = I
        L.moe_error_string.argtypes = [I]
        L.moe_error_string.restype = ctypes.c_char_p
        _LIB = L
    return _LIB


def check(rc: int, what: str) -> None:
    if rc != 0:
        msg = lib().moe_error_string(rc).decode()
        raise MoeError(f"{what} failed with code {rc}: {msg}")


def workspace_layout(geom, T: int) -> dict:
    """Byte offsets of the workspace regions plus ``total``."""
    offs = (ctypes.c_int64 * (MOE_WS_NUM_REGIONS + 1))()
    g = geom.c_struct()
    check(lib().moe_workspace_layout(ctypes.byref(g), int(T), offs), "moe_workspace_layout")
    d = {name: int(offs[i]) for i, name in enumerate(WS_REGIONS)}
    d["total"] = int(offs[MOE_WS_NUM_REGIONS])
    return d
