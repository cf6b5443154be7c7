"""Python entry points mirroring the reference solutions' ``run``.

* ``run(routing_logits, routing_bias, hidden_states, hidden_states_scale, gemm1_weights,
  gemm1_weights_scale, gemm2_weights, gemm2_weights_scale, local_expert_offset,
  routed_scaling_factor)`` -> bf16 [T, H]: value-returning form,
  goal_full_shape/opus-4.8/moe_fp8_fwd/MOEDIR/main.py:286-288.
* ``run(..., output)``: destination-passing form,
  kda05_reproduction_single_shape/fable-5.1/moe_fp8_fwd/t901/main.py:45-57.

Argument handling follows kda05_reproduction_single_shape/fable-5.1/moe_fp8_fwd/t1/main.py:99-133:
scalars may be 0-d tensors, logits/bias/scales are coerced to fp32/bf16 contiguous, fp8 tensors
must already be e4m3fn and contiguous. A ``None`` bias means zeros
(kda05_reproduction_single_shape/fable-5.1/moe_fp8_fwd/t14107/main.py:97-98). The work runs in
HIP kernels through the C ABI on the current torch stream; this module only checks arguments and
owns the cached workspaces (one per stream).
"""
from __future__ import annotations

import ctypes

import torch

from . import _lib
from .geometry import DS_V3, Geometry

F8 = torch.float8_e4m3fn
_WS: dict = {}


def workspace(geom: Geometry, T: int, device, stream=None) -> torch.Tensor:
    """The workspace ``run`` and ``route`` use on (device, stream): one buffer per stream that
    grows to the largest ``moe_workspace_bytes`` seen (any buffer at least that large serves a
    call with T tokens; its contents need no initialisation). Calls on one stream are ordered,
    so they can share it; calls on different streams get different buffers, as calls that
    overlap in time must. ``stream`` defaults to the device's current torch stream."""
    dev = torch.device(device)
    if stream is None:
        stream = torch.cuda.current_stream(dev)
    key = (dev, int(stream.cuda_stream))
    n = max(_lib.workspace_layout(geom, T)["total"], 1)
    ws = _WS.get(key)
    if ws is None or ws.numel() < n:
        ws = torch.empty(n, dtype=torch.uint8, device=dev)
        _WS[key] = ws
    return ws


def release_workspaces() -> None:
    """Drops the cached per-stream workspaces (their memory returns to torch's allocator)."""
    _WS.clear()


def _scalar(x, cast):
    if isinstance(x, torch.Tensor):
        return cast(x.item())
    return cast(x)


def _check_shapes(geom: Geometry, T, logits, hs, hs_scale, w13, s13, w2, s2):
    H, I, E, El, B = geom.hidden, geom.intermediate, geom.num_experts, geom.local_experts, 128
    want = {
        "routing_logits": (logits, (T, E)),
        "hidden_states": (hs, (T, H)),
        "hidden_states_scale": (hs_scale, (H // B, T)),
        "gemm1_weights": (w13, (El, 2 * I, H)),
        "gemm1_weights_scale": (s13, (El, 2 * I // B, H // B)),
        "gemm2_weights": (w2, (El, H, I)),
        "gemm2_weights_scale": (s2, (El, H // B, I // B)),
    }
    for name, (t, shape) in want.items():
        if tuple(t.shape) != shape:
            raise ValueError(f"{name}: expected shape {shape}, got {tuple(t.shape)}")


def _routing_args(geom: Geometry, routing_logits, routing_bias, on_gpu=True):
    """Coerced logits fp32 [T, E] and bias bf16 [E] (or None), shape-checked."""
    if routing_logits.dim() != 2 or int(routing_logits.shape[1]) != geom.num_experts:
        raise ValueError(f"routing_logits: expected shape (T, {geom.num_experts}), got "
                         f"{tuple(routing_logits.shape)}")
    if routing_logits.dtype != torch.float32 or not routing_logits.is_contiguous():
        routing_logits = routing_logits.contiguous().to(torch.float32)
    if routing_bias is not None:
        if tuple(routing_bias.shape) != (geom.num_experts,):
            raise ValueError(f"routing_bias: expected shape ({geom.num_experts},), got "
                             f"{tuple(routing_bias.shape)}")
        if routing_bias.dtype != torch.bfloat16 or not routing_bias.is_contiguous():
            routing_bias = routing_bias.contiguous().to(torch.bfloat16)
        if routing_bias.device != routing_logits.device:
            raise ValueError("routing_bias must be on the logits' device")
    if on_gpu and routing_logits.device.type != "cuda":
        raise ValueError("routing_logits must be on a GPU")
    return routing_logits, routing_bias


def _prepare(geom: Geometry, routing_logits, routing_bias, hidden_states, hidden_states_scale,
             gemm1_weights, gemm1_weights_scale, gemm2_weights, gemm2_weights_scale, output):
    """The argument rules of ``run`` (t1/main.py:99-133 coercions plus shape, dtype, contiguity
    and device checks), shared by ``run`` and ``bind``. Returns (T, device, tensors, bias,
    output) with ``tensors`` = (logits, hs, hs_scale, w13, s13, w2, s2)."""
    T = int(routing_logits.shape[0])
    dev = hidden_states.device
    routing_logits, routing_bias = _routing_args(geom, routing_logits, routing_bias, on_gpu=False)
    for name, t in (("hidden_states", hidden_states), ("gemm1_weights", gemm1_weights),
                    ("gemm2_weights", gemm2_weights)):
        if t.dtype != F8 or not t.is_contiguous():
            raise TypeError(f"{name} must be a contiguous float8_e4m3fn tensor")
    hss = hidden_states_scale.contiguous().to(torch.float32)
    s13 = gemm1_weights_scale.contiguous().to(torch.float32)
    s2 = gemm2_weights_scale.contiguous().to(torch.float32)
    _check_shapes(geom, T, routing_logits, hidden_states, hss, gemm1_weights, s13, gemm2_weights,
                  s2)
    if output is None:
        output = torch.empty((T, geom.hidden), dtype=torch.bfloat16, device=dev)
    elif (output.dtype != torch.bfloat16 or tuple(output.shape) != (T, geom.hidden)
          or not output.is_contiguous()):
        raise ValueError("output must be a contiguous bf16 [T, H] tensor")
    tensors = (routing_logits, hidden_states, hss, gemm1_weights, s13, gemm2_weights, s2)
    devs = [t.device for t in tensors] + [output.device]
    if routing_bias is not None:
        devs.append(routing_bias.device)
    if any(d != dev for d in devs) or dev.type != "cuda":
        raise ValueError("all tensors must be on the same GPU")
    return T, dev, tensors, routing_bias, output


@torch.no_grad()
def run(routing_logits, routing_bias, hidden_states, hidden_states_scale, gemm1_weights,
        gemm1_weights_scale, gemm2_weights, gemm2_weights_scale, local_expert_offset,
        routed_scaling_factor, output=None, *, geometry: Geometry = DS_V3):
    """FP8 block-scale MoE forward. Returns ``output`` (allocated when not given)."""
    geom = geometry
    off = _scalar(local_expert_offset, int)
    rsf = _scalar(routed_scaling_factor, float)
    T, dev, tensors, bias, output = _prepare(
        geom, routing_logits, routing_bias, hidden_states, hidden_states_scale, gemm1_weights,
        gemm1_weights_scale, gemm2_weights, gemm2_weights_scale, output)
    if T == 0:
        return output
    ws = workspace(geom, T, dev)
    stream = torch.cuda.current_stream(dev).cuda_stream
    g = geom.c_struct()
    bias_ptr = None if bias is None else bias.data_ptr()
    rc = _lib.lib().moe_run_ex(
        ctypes.byref(g), tensors[0].data_ptr(), bias_ptr, *[t.data_ptr() for t in tensors[1:]],
        off, rsf, output.data_ptr(), ws.data_ptr(), T, stream)
    _lib.check(rc, "moe_run_ex")
    return output


class BoundCall:
    """A validated argument set bound to the C ABI: calling it enqueues one operator call on the
    current stream with no per-call Python argument handling (the role of the reference
    solutions' per-T workspace/graph caches, goal_full_shape/opus-4.8/moe_fp8_fwd/MOEDIR/
    main.py:274-338). The bound tensors must stay alive and unchanged in shape."""

    def __init__(self, geom, tensors, bias, off, rsf, output, ws, T):
        self.geom, self.T, self.output = geom, T, output
        self.workspace = ws  # this call's own workspace (routing results stay readable here)
        self._keep = (tensors, bias, output, ws)
        self._g = geom.c_struct()
        self._fn = _lib.lib().moe_run_ex
        self._args = [ctypes.byref(self._g), tensors[0].data_ptr(),
                      None if bias is None else bias.data_ptr(),
                      *[t.data_ptr() for t in tensors[1:]], off, rsf, output.data_ptr(),
                      ws.data_ptr(), T]

    def __call__(self, stream=None):
        s = torch.cuda.current_stream().cuda_stream if stream is None else stream
        _lib.check(self._fn(*self._args, s), "moe_run_ex")
        return self.output


@torch.no_grad()
def bind(routing_logits, routing_bias, hidden_states, hidden_states_scale, gemm1_weights,
         gemm1_weights_scale, gemm2_weights, gemm2_weights_scale, local_expert_offset,
         routed_scaling_factor, output=None, *, geometry: Geometry = DS_V3) -> BoundCall:
    """Validate once (the same rules as ``run``) and return a ``BoundCall``."""
    geom = geometry
    T, dev, tensors, bias, output = _prepare(
        geom, routing_logits, routing_bias, hidden_states, hidden_states_scale, gemm1_weights,
        gemm1_weights_scale, gemm2_weights, gemm2_weights_scale, output)
    # a bound call owns its workspace, so bound calls on different streams never share one
    ws = torch.empty(max(_lib.workspace_layout(geom, T)["total"], 1), dtype=torch.uint8,
                     device=dev)
    return BoundCall(geom, tensors, bias, _scalar(local_expert_offset, int),
                     _scalar(routed_scaling_factor, float), output, ws, T)


@torch.no_grad()
def route(routing_logits, routing_bias, local_expert_offset, routed_scaling_factor, *,
          geometry: Geometry = DS_V3) -> dict:
    """Routing + permute only; returns views of the workspace regions they write."""
    geom = geometry
    T = int(routing_logits.shape[0])
    routing_logits, routing_bias = _routing_args(geom, routing_logits, routing_bias)
    dev = routing_logits.device
    ws = workspace(geom, T, dev)
    g = geom.c_struct()
    rc = _lib.lib().moe_route_ex(
        ctypes.byref(g), routing_logits.data_ptr(),
        None if routing_bias is None else routing_bias.data_ptr(),
        _scalar(local_expert_offset, int), _scalar(routed_scaling_factor, float), ws.data_ptr(), T,
        torch.cuda.current_stream(dev).cuda_stream)
    _lib.check(rc, "moe_route_ex")
    return workspace_views(geom, T, ws)


@torch.no_grad()
def quantize_activations(hidden_states, out=None, scale_out=None):
    """bf16 [T, H] -> (float8_e4m3fn [T, H], fp32 scales [H/128, T]): the per-token 1x128 block
    quantisation that produces ``hidden_states`` / ``hidden_states_scale`` for ``run``
    (rule of goal_full_shape/opus-4.8/moe_fp8_fwd/MOEDIR/main.py:151-156: scale = amax / 448).
    Runs the HIP kernel behind ``moe_quantize_activations`` on the current stream."""
    x = hidden_states
    if x.dim() != 2 or x.dtype != torch.bfloat16:
        raise TypeError("hidden_states must be a bf16 [T, H] tensor")
    x = x.contiguous()
    T, H = x.shape
    if H % 128 != 0:
        raise ValueError("H must be a multiple of 128")
    dev = x.device
    if dev.type != "cuda":
        raise ValueError("hidden_states must be on a GPU")
    if out is None:
        out = torch.empty((T, H), dtype=F8, device=dev)
    if scale_out is None:
        scale_out = torch.empty((H // 128, T), dtype=torch.float32, device=dev)
    if (out.dtype != F8 or tuple(out.shape) != (T, H) or not out.is_contiguous()
            or scale_out.dtype != torch.float32 or tuple(scale_out.shape) != (H // 128, T)
            or not scale_out.is_contiguous()):
        raise ValueError("out must be e4m3fn [T, H] and scale_out fp32 [H/128, T], contiguous")
    rc = _lib.lib().moe_quantize_activations(x.data_ptr(), T, H, out.data_ptr(),
                                             scale_out.data_ptr(),
                                             torch.cuda.current_stream(dev).cuda_stream)
    _lib.check(rc, "moe_quantize_activations")
    return out, scale_out


def workspace_views(geom: Geometry, T: int, ws: torch.Tensor) -> dict:
    """Typed views of the workspace regions (the layout moe_workspace_layout reports)."""
    L = _lib.workspace_layout(geom, T)
    K, El = geom.top_k, geom.local_experts
    Np = T * min(K, El)

    def view(name, dtype, shape):
        n = 1
        for s in shape:
            n *= s
        nbytes = n * torch.empty((), dtype=dtype).element_size()
        return ws[L[name]:L[name] + nbytes].view(dtype).view(shape)

    return dict(
        topk_idx=view("topk_idx", torch.int32, (T, K)),
        topk_w=view("topk_w", torch.float32, (T, K)),
        pair_of=view("pair_of", torch.int32, (T, K)),
        counts=view("counts", torch.int32, (El,)),
        offsets=view("offsets", torch.int32, (El + 1,)),
        sorted_tok=view("sorted_tok", torch.int32, (Np,)),
        sorted_w=view("sorted_w", torch.float32, (Np,)),
        C=view("C", torch.bfloat16, (Np, geom.intermediate)),
        partial=view("partial", torch.bfloat16, (T * (min(K, El) - 1), geom.hidden)),
        pair_dst=view("pair_dst", torch.int32, (Np,)),
    )
