"""CPU restatement of the FP8 block-scale MoE operator (dequantise-then-fp32).

TEST INFRASTRUCTURE ONLY (see the package docstring). Nothing in ``justgoal_amd`` imports this.

The reference definition (flashinfer-bench ``moe_fp8_block_scale_ds_routing_topk8_ng8_kg4_e32_h7168_i2048``)
is not vendored in the reference tree; every solution there says it mirrors it. The semantics
restated here follow:

* dequantisation D1: ``A[t,k] = hs[t,k] * hs_scale[k//128, t]``, ``W13[e,n,k] = w13 * s13[e,n//128,k//128]``,
  ``W2[e,h,i] = w2 * s2[e,h//128,i//128]`` --
  goal_full_shape/opus-4.8/moe_fp8_fwd/MOEDIR/main.py:127-132,183-187, moe_v3.cuh:79-83;
* routing R1-R6 and the local filter L1 -- ``moe_routing_oracle.c`` (C, exact fp32 order);
  ``route_numpy`` below is an independent vectorised restatement used to pin the C one;
* GEMM1 + SwiGLU G1: ``G = A[tok_e] @ W13[e].T``; ``C = X1 * silu(X2)`` with X1 the first I
  columns and silu applied to the second half -- opus-4.8 main.py:148-150,
  kda05_reproduction_single_shape/fable-5.1/moe_fp8_fwd/t14107/moe_kernel.cu:876;
* GEMM2 G2: ``O = C @ W2[e].T``, ``out[tok_e] += w * O`` -- opus-4.8 main.py:181-189;
* F: one rounding of the fp32 sum to bf16 (round to nearest even). The fp32 accumulation runs
  in ascending local-expert order.
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np
import torch

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB = None

ROUTING_DS = 0
ROUTING_SOFTMAX = 1


def oracle_lib():
    """Load (building if needed, on a machine with gcc) the C routing/permute oracle."""
    global _LIB
    if _LIB is None:
        so = os.path.join(_HERE, "liboracle_moe.so")
        src = os.path.join(_HERE, "moe_routing_oracle.c")
        if not os.path.exists(so) or os.path.getmtime(so) < os.path.getmtime(src):
            subprocess.run(["make", "-s", "-C", _HERE], check=True)
        lib = ctypes.CDLL(so)
        P = ctypes.c_void_p
        lib.oracle_route_ds.argtypes = [P, P, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int,
                                        ctypes.c_int, ctypes.c_float, P, P]
        lib.oracle_route_softmax.argtypes = [P, ctypes.c_int, ctypes.c_int, ctypes.c_int, P, P]
        lib.oracle_permute.argtypes = [P, P, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int,
                                       P, P, P, P, P]
        for f in (lib.oracle_route_ds, lib.oracle_route_softmax, lib.oracle_permute):
            f.restype = ctypes.c_int
        for f in (lib.oracle_sigmoid_batch, lib.oracle_exp_batch):
            f.argtypes = [P, P, ctypes.c_int64]
            f.restype = None
        _LIB = lib
    return _LIB


def _ptr(a: np.ndarray):
    return a.ctypes.data_as(ctypes.c_void_p)


def sigmoid_f32(x) -> np.ndarray:
    """R1 as the C oracle computes it (oracle_sigmoid_f32), element-wise over fp32 ``x``."""
    x = np.ascontiguousarray(x, np.float32)
    y = np.empty_like(x)
    oracle_lib().oracle_sigmoid_batch(_ptr(x), _ptr(y), x.size)
    return y


def exp_f32(x) -> np.ndarray:
    """The C oracle's fp32 exp (oracle_exp_f32), element-wise."""
    x = np.ascontiguousarray(x, np.float32)
    y = np.empty_like(x)
    oracle_lib().oracle_exp_batch(_ptr(x), _ptr(y), x.size)
    return y


def fma32(a, b, c) -> np.ndarray:
    """Correctly rounded fp32 fused multiply-add on arrays, in numpy: the fp64 product of two
    fp32 values is exact, TwoSum gives the exact sum as s + err, and rounding s to fp32 is
    corrected where s sits exactly on a rounding midpoint and err breaks the tie."""
    a, b, c = (np.asarray(v, np.float32).astype(np.float64) for v in (a, b, c))
    p = a * b
    s = p + c
    bb = s - p
    err = (p - (s - bb)) + (c - bb)
    r = s.astype(np.float32)
    rd = r.astype(np.float64)
    # the other fp32 neighbour of s, on the far side of r
    other = np.where(s > rd, np.nextafter(r, np.float32(np.inf)),
                     np.nextafter(r, np.float32(-np.inf))).astype(np.float64)
    mid = (s != rd) & ((s - rd) == (other - s)) & (err != 0)
    fix = mid & (np.sign(err) == np.sign(other - rd))
    return np.where(fix, other.astype(np.float32), r).astype(np.float32)


def _exp_parts_numpy(y):
    f = np.float32
    y = np.minimum(np.maximum(np.asarray(y, f), f(-104.0)), f(88.0))
    n = np.rint((y * f(1.44269504088896341)).astype(f))
    r = fma32(-n, f(0.693145751953125), y)
    r = fma32(-n, f(1.428606765330187045e-06), r)
    q = np.full_like(r, f(1.0) / f(5040.0))
    for c in (f(1.0) / f(720.0), f(1.0) / f(120.0), f(1.0) / f(24.0), f(1.0) / f(6.0), f(0.5),
              f(1.0)):
        q = fma32(q, r, c)
    h = fma32(r, q, f(1.0))
    lo = fma32(r, q, (f(1.0) - h).astype(f))
    return h, lo, n.astype(np.int32)


def sigmoid_numpy(x) -> np.ndarray:
    """Independent numpy statement of oracle_sigmoid_f32 (same steps, fma emulated exactly)."""
    f = np.float32
    x = np.asarray(x, f)
    small = x < f(-87.0)
    ph, pl, n = _exp_parts_numpy(np.where(small, x, -x))
    eh = np.ldexp(ph, n).astype(f)
    el = np.ldexp(pl, n).astype(f)
    dh = (f(1.0) + eh).astype(f)
    dl = (np.where(eh >= f(1.0), ((eh - dh).astype(f) + f(1.0)).astype(f),
                   ((f(1.0) - dh).astype(f) + eh).astype(f)) + el).astype(f)
    with np.errstate(divide="ignore"):
        s0 = (f(1.0) / dh).astype(f)
    res = fma32(-s0, dl, fma32(-s0, dh, f(1.0)))
    out = fma32(s0, res, s0)
    return np.where(small, eh, out).astype(f)


def exp_numpy(y) -> np.ndarray:
    ph, _, n = _exp_parts_numpy(y)
    return np.ldexp(ph, n).astype(np.float32)


def route(logits, bias, geom, rsf: float):
    """Routing R1-R6 (or softmax top-k) via the C oracle. Returns (topk_idx int32 [T,K], topk_w f32 [T,K])."""
    lg = np.ascontiguousarray(torch.as_tensor(logits).float().cpu().numpy())
    T = lg.shape[0]
    K = geom.top_k
    idx = np.zeros((T, K), np.int32)
    w = np.zeros((T, K), np.float32)
    lib = oracle_lib()
    if geom.routing_method == ROUTING_DS:
        if bias is None:
            b = None
        else:
            b = np.ascontiguousarray(torch.as_tensor(bias).to(torch.bfloat16).cpu().view(torch.int16).numpy())
        rc = lib.oracle_route_ds(_ptr(lg), None if b is None else _ptr(b), T, geom.num_experts,
                                 geom.n_group, geom.topk_group, K, float(rsf), _ptr(idx), _ptr(w))
    else:
        rc = lib.oracle_route_softmax(_ptr(lg), T, geom.num_experts, K, _ptr(idx), _ptr(w))
    if rc != 0:
        raise ValueError(f"oracle routing rejected the geometry (rc={rc})")
    return idx, w


def route_numpy(logits, bias, geom, rsf: float):
    """Independent vectorised restatement of routing, used to pin the C oracle.

    Selection uses a stable lexicographic sort on (-v, index) instead of the C code's
    iterative arg-max, so an index or tie-order slip in either one shows up as a mismatch.
    """
    x = np.asarray(torch.as_tensor(logits).float().cpu().numpy(), np.float32)
    T, E = x.shape
    K = geom.top_k
    order_idx = np.arange(E)
    if geom.routing_method == ROUTING_DS:
        s = sigmoid_numpy(x)
        b = (np.zeros(E, np.float32) if bias is None
             else torch.as_tensor(bias).to(torch.bfloat16).float().cpu().numpy())
        v = (s + b[None, :]).astype(np.float32)
        G = geom.n_group
        gsz = E // G
        vg = v.reshape(T, G, gsz)
        srt = -np.sort(-vg, axis=2, kind="stable")
        gscore = (srt[:, :, 0] + srt[:, :, 1]).astype(np.float32) if gsz > 1 else srt[:, :, 0]
        # groups ranked by (-score, group index); keep the first topk_group
        gorder = np.lexsort((np.broadcast_to(np.arange(G), (T, G)), -gscore), axis=1)
        kept = np.zeros((T, G), bool)
        np.put_along_axis(kept, gorder[:, : geom.topk_group], True, axis=1)
        cand = np.where(np.repeat(kept, gsz, axis=1), v, -np.inf).astype(np.float32)
        eorder = np.lexsort((np.broadcast_to(order_idx, (T, E)), -cand), axis=1)
        idx = eorder[:, :K].astype(np.int32)
        sel = np.take_along_axis(s, idx, axis=1)
        tot = np.zeros(T, np.float32)
        for k in range(K):  # selection-order fp32 accumulation
            tot = (tot + sel[:, k]).astype(np.float32)
        tot = (tot + np.float32(1e-20)).astype(np.float32)
        w = ((sel / tot[:, None]).astype(np.float32) * np.float32(rsf)).astype(np.float32)
    else:
        eorder = np.lexsort((np.broadcast_to(order_idx, (T, E)), -x), axis=1)
        idx = eorder[:, :K].astype(np.int32)
        xs = np.take_along_axis(x, idx, axis=1)
        d = (xs - xs[:, :1]).astype(np.float32)
        ex = exp_numpy(d)
        tot = np.zeros(T, np.float32)
        for k in range(K):
            tot = (tot + ex[:, k]).astype(np.float32)
        w = (ex / tot[:, None]).astype(np.float32)
    return idx, w


def permute(topk_idx, topk_w, local_offset: int, E_local: int):
    """Stable counting sort P1 via the C oracle.

    Returns dict(counts [E_l], offsets [E_l+1], sorted_tok [N], sorted_w [N], pair_of [T,K]).
    """
    idx = np.ascontiguousarray(topk_idx, np.int32)
    w = np.ascontiguousarray(topk_w, np.float32)
    T, K = idx.shape
    counts = np.zeros(E_local, np.int32)
    offsets = np.zeros(E_local + 1, np.int32)
    cap = max(1, T * K)
    st = np.zeros(cap, np.int32)
    sw = np.zeros(cap, np.float32)
    pair_of = np.zeros((T, K), np.int32)
    n = oracle_lib().oracle_permute(_ptr(idx), _ptr(w), T, K, int(local_offset), E_local,
                                    _ptr(counts), _ptr(offsets), _ptr(st), _ptr(sw), _ptr(pair_of))
    if n < 0:
        raise ValueError("oracle permute rejected the geometry")
    return dict(counts=counts, offsets=offsets, sorted_tok=st[:n].copy(), sorted_w=sw[:n].copy(),
                pair_of=pair_of, pair_dst=pair_destinations(idx, pair_of, local_offset, E_local))


def pair_destinations(topk_idx, pair_of, local_offset: int, E_local: int):
    """GEMM2 destination of each pair (this build's layout; the reference accumulates into its
    output with atomics, opus-4.8 main.py:188-189, and has no such table).

    A token's local pairs, taken in ascending local-expert order, get ranks j = 0, 1, ...: rank 0
    is written straight into output row t (code t), rank j >= 1 into partial row
    t * (k - 1) + j - 1 (code -1 - that row), k = min(top_k, E_local). Returns int32 [N] indexed by
    pair row."""
    idx = np.asarray(topk_idx, np.int64)
    T, K = idx.shape
    k = min(K, E_local)
    le = idx - int(local_offset)
    local = (le >= 0) & (le < E_local)
    # rank of slot (t, a) = local slots b of t with a smaller local expert
    rank = (local[:, None, :] & (le[:, None, :] < le[:, :, None])).sum(axis=2)
    t = np.broadcast_to(np.arange(T)[:, None], (T, K))
    code = np.where(rank == 0, t, -1 - (t * (k - 1) + rank - 1))
    n = int(local.sum())
    dst = np.zeros(n, np.int32)
    dst[np.asarray(pair_of)[local]] = code[local]
    return dst


def quantize_activations(x: torch.Tensor):
    """bf16/fp32 [T, H] -> (e4m3fn [T, H], fp32 scales [H/128, T]), per 1x128 row block.

    The reference's block-quantisation rule (goal_full_shape/opus-4.8/moe_fp8_fwd/MOEDIR/
    main.py:151-156): amax over the block, scale = amax / 448 (stored as is, so 0 for an all-zero
    block), divisor = scale or 1 when scale is 0, codes = clamp(x / divisor, -448, 448) rounded to
    e4m3 (nearest even). fp32 throughout; torch's CPU division is IEEE and its float8_e4m3fn cast
    rounds to nearest even (pinned against a table-driven encoder in tests/test_oracle.py).
    """
    T, H = x.shape
    xb = x.float().reshape(T, H // 128, 128)
    amax = xb.abs().amax(dim=2)
    scale = amax / 448.0
    div = torch.where(scale > 0, scale, torch.ones_like(scale))
    q = (xb / div[:, :, None]).clamp(-448.0, 448.0).to(torch.float8_e4m3fn).reshape(T, H)
    return q, scale.t().contiguous()


def dequant_blocks(q: torch.Tensor, scale: torch.Tensor, block: int = 128) -> torch.Tensor:
    """fp8 [..., R, C] with fp32 block scales [..., R/block, C/block] -> fp32 (D1)."""
    s = scale.float().repeat_interleave(block, dim=-2).repeat_interleave(block, dim=-1)
    return q.float() * s


def dequant_activations(hs: torch.Tensor, hs_scale: torch.Tensor, block: int = 128) -> torch.Tensor:
    """fp8 [T, H] with per-token 1x128 scales stored transposed [H/128, T] -> fp32 (D1)."""
    return hs.float() * hs_scale.float().t().repeat_interleave(block, dim=1)


@torch.no_grad()
def moe_reference(inputs: dict, geom, return_intermediates: bool = False, experts=None):
    """Full operator on the CPU in fp32: returns bf16 [T, H] (and intermediates if asked).

    ``inputs`` holds the operator's tensors under the reference's argument names.
    ``experts`` optionally limits the GEMMs to a subset of local experts (bounded CPU samples).
    """
    logits = inputs["routing_logits"].cpu()
    T = logits.shape[0]
    H, I = geom.hidden, geom.intermediate
    off = int(inputs["local_expert_offset"])
    rsf = float(inputs["routed_scaling_factor"])
    idx, w = route(logits, inputs.get("routing_bias"), geom, rsf)
    perm = permute(idx, w, off, geom.local_experts)
    A = dequant_activations(inputs["hidden_states"].cpu(), inputs["hidden_states_scale"].cpu())
    acc = torch.zeros(T, H, dtype=torch.float32)
    w13, s13 = inputs["gemm1_weights"], inputs["gemm1_weights_scale"]
    w2, s2 = inputs["gemm2_weights"], inputs["gemm2_weights_scale"]
    C_rows = {}
    for e in range(geom.local_experts):
        lo, hi = int(perm["offsets"][e]), int(perm["offsets"][e + 1])
        if hi == lo or (experts is not None and e not in experts):
            continue
        tok = torch.from_numpy(perm["sorted_tok"][lo:hi].astype(np.int64))
        wt = torch.from_numpy(perm["sorted_w"][lo:hi])
        W13 = dequant_blocks(w13[e].cpu(), s13[e].cpu())
        G = A[tok] @ W13.t()
        del W13
        X1, X2 = G[:, :I], G[:, I:]
        C = X1 * (X2 * torch.sigmoid(X2))
        W2 = dequant_blocks(w2[e].cpu(), s2[e].cpu())
        O = C @ W2.t()
        del W2
        acc.index_add_(0, tok, O * wt[:, None])
        if return_intermediates:
            C_rows[e] = C
    out = acc.to(torch.bfloat16)
    if not return_intermediates:
        return out
    return out, dict(topk_idx=idx, topk_w=w, C=C_rows, acc=acc, **perm)
