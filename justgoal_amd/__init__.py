"""MI355X-native (gfx950) FP8 block-scale Mixture-of-Experts with DeepSeek-style routing.

The operator runs in hand-written HIP kernels behind the C ABI in include/justgoal_moe.h
(``libjustgoal_moe.so``); ``run`` is the reference-compatible Python entry point.
"""
from .geometry import DS_V3, QWEN3, Geometry  # noqa: F401
from .moe import bind, route, run, workspace, workspace_views  # noqa: F401
