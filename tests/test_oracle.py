"""Pins the CPU oracle (no GPU).

The reference ships no tests, golden vectors or fixtures for this operator (its definition and
tolerances live in the external flashinfer-bench dataset), so the oracle is pinned by:

* two independent restatements of routing (scalar C with iterative arg-max; vectorised numpy with
  stable lexicographic sorts) that must agree bit for bit;
* brute-force formulations on small inputs (rank counting instead of sorting, max pair sum for
  the group top-2 score) and constructed ties;
* ``torch.topk`` / ``torch.sigmoid`` / ``torch.softmax`` cross-checks where ties are absent;
* closed-form known answers for the GEMM path (identity weights, distinct per-block scales, the
  SwiGLU half order);
* invariants of the permute (histogram, stable ascending segments, inverse pair map).
"""
import numpy as np
import pytest
import torch

import oracle
from justgoal_amd import inputs as jin
from justgoal_amd.geometry import DS_V3, QWEN3, ROUTING_DS, ROUTING_SOFTMAX, Geometry

SMALL_DS = Geometry(256, 128, 64, 16, 4, 4, 2, ROUTING_DS, "small-DS")
SMALL_SOFTMAX = Geometry(256, 128, 128, 128, 8, 1, 1, ROUTING_SOFTMAX, "small-softmax")


def _logits(T, E, seed, ties=False):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(T, E, generator=g)
    if ties:
        # quantise so that many values coincide exactly
        x = torch.round(x * 4) / 4
    return x


def _bias(E, seed, zero=False):
    if zero:
        return torch.zeros(E, dtype=torch.bfloat16)
    g = torch.Generator().manual_seed(seed + 99)
    return (torch.randn(E, generator=g) * 0.1).to(torch.bfloat16)


@pytest.mark.parametrize("geom", [DS_V3, SMALL_DS, QWEN3, SMALL_SOFTMAX])
@pytest.mark.parametrize("ties", [False, True])
def test_c_oracle_matches_numpy_restatement(geom, ties):
    x = _logits(257, geom.num_experts, seed=11, ties=ties)
    b = _bias(geom.num_experts, 11, zero=ties)
    i1, w1 = oracle.route(x, b, geom, 2.5)
    i2, w2 = oracle.route_numpy(x, b, geom, 2.5)
    np.testing.assert_array_equal(i1, i2)
    np.testing.assert_array_equal(w1.view(np.uint32), w2.view(np.uint32))


def _brute_route_ds(x, b, geom, rsf):
    """Rank-counting formulation (no sorting): an expert / group is selected iff fewer than k
    candidates beat it, where a beats b if its value is larger or equal with a lower index."""
    T, E = x.shape
    gs = E // geom.n_group
    s = oracle.sigmoid_numpy(x)
    v = (s + b[None, :]).astype(np.float32)
    out_idx = np.zeros((T, geom.top_k), np.int64)
    for t in range(T):
        # group score = max pair sum inside the group (== sum of the top two as a multiset)
        gsc = []
        for g in range(geom.n_group):
            vg = v[t, g * gs:(g + 1) * gs]
            best = -np.inf
            for i in range(gs):
                for j in range(gs):
                    if i != j:
                        best = max(best, np.float32(vg[i] + vg[j]))
            gsc.append(np.float32(best))
        kept = []
        for g in range(geom.n_group):
            beaten = sum(1 for h in range(geom.n_group)
                         if gsc[h] > gsc[g] or (gsc[h] == gsc[g] and h < g))
            kept.append(beaten < geom.topk_group)
        cand = [e for e in range(E) if kept[e // gs]]
        ranked = []
        for e in cand:
            beaten = sum(1 for f in cand if v[t, f] > v[t, e] or (v[t, f] == v[t, e] and f < e))
            if beaten < geom.top_k:
                ranked.append((beaten, e))
        ranked.sort()
        out_idx[t] = [e for _, e in ranked]
    return out_idx


@pytest.mark.parametrize("ties", [False, True])
def test_routing_brute_force_small(ties):
    geom = SMALL_DS
    x = _logits(24, geom.num_experts, seed=5, ties=ties)
    b = _bias(geom.num_experts, 5, zero=ties)
    idx, w = oracle.route(x, b, geom, 2.5)
    ref = _brute_route_ds(x.numpy(), b.float().numpy(), geom, 2.5)
    np.testing.assert_array_equal(idx, ref)


def test_constructed_ties_lower_index_wins():
    geom = Geometry(256, 128, 64, 16, 4, 4, 2, ROUTING_DS)
    E = 64
    # logits equal everywhere: every group score ties -> groups 0 and 1 kept, experts 0..3 win
    x = torch.zeros(1, E)
    idx, w = oracle.route(x, torch.zeros(E, dtype=torch.bfloat16), geom, 1.0)
    assert idx.tolist() == [[0, 1, 2, 3]]
    np.testing.assert_allclose(w, 0.25, rtol=1e-6)
    # a duplicated maximum counts twice in the group score: group 3 has two 5.0 values,
    # group 2 has one 6.0 and the rest low -> group 3 (score 2*s(5)) beats group 2 (s(6)+s(-4))
    x = torch.full((1, E), -4.0)
    x[0, 48] = 5.0
    x[0, 49] = 5.0
    x[0, 32] = 6.0
    x[0, 0] = 0.5
    idx, _ = oracle.route(x, torch.zeros(E, dtype=torch.bfloat16), geom, 1.0)
    kept_groups = sorted({int(e) // 16 for e in idx[0]})
    assert 3 in kept_groups and 48 in idx[0] and 49 in idx[0]
    # equal expert values across two kept groups: lower index first
    x = torch.full((1, E), -3.0)
    x[0, [5, 21]] = 2.0
    idx, _ = oracle.route(x, torch.zeros(E, dtype=torch.bfloat16), geom, 1.0)
    assert idx[0][0] == 5 and idx[0][1] == 21


def test_routing_against_torch_topk_and_sigmoid():
    geom = DS_V3
    x = _logits(300, 256, seed=3)
    b = _bias(256, 3)
    idx, w = oracle.route(x, b, geom, 2.5)
    s_ref = torch.sigmoid(x)  # fp32 library sigmoid, within 2 ulp of the correctly rounded one
    s_or = torch.from_numpy(oracle.sigmoid_f32(x.numpy()))
    ulp = torch.abs(s_ref.view(torch.int32) - s_or.view(torch.int32))
    assert int(ulp.max()) <= 2
    v = s_or + b.float()
    gs = v.view(300, 8, 32).topk(2, dim=2).values.sum(2)
    keep = torch.zeros(300, 8, dtype=torch.bool)
    keep.scatter_(1, gs.topk(4, dim=1).indices, True)
    cand = torch.where(keep.repeat_interleave(32, dim=1), v, torch.tensor(float("-inf")))
    top = cand.topk(8, dim=1)
    assert torch.equal(torch.from_numpy(idx).long(), top.indices)
    sel = torch.gather(s_or, 1, top.indices)
    w_ref = sel / (sel.sum(1, keepdim=True) + 1e-20) * 2.5
    torch.testing.assert_close(torch.from_numpy(w), w_ref, rtol=1e-6, atol=1e-7)
    # invariant: sum of the weights is the scaling factor
    np.testing.assert_allclose(w.sum(1), 2.5, rtol=1e-5)


def _ulps(a, b):
    return np.abs(a.view(np.int32).astype(np.int64) - b.view(np.int32).astype(np.int64))


def _float_sample(lo_abs, hi_abs, n):
    """About n fp32 values of each sign with |x| in [lo_abs, hi_abs], evenly spaced in bit
    pattern (so every binade is covered), plus the boundary values."""
    a = np.float32(lo_abs).view(np.int32)
    b = np.float32(hi_abs).view(np.int32)
    step = max(1, int(b - a) // n)
    m = np.arange(a, b, step, dtype=np.int32).view(np.float32)
    return np.concatenate([m, -m, np.float32([lo_abs, hi_abs, -lo_abs, -hi_abs])])


def test_sigmoid_f32_pinned():
    """R1 (oracle_sigmoid_f32, which the routing kernel restates step for step): within 1 ulp of
    the correctly rounded sigmoid (fp64 evaluation rounded once) on every binade of |x| in
    [2^-30, 90], exactly rounded in at least 99% of cases; within 2 ulp of torch.sigmoid
    (itself up to 2 ulp from the correctly rounded value); identical to the independent numpy
    statement; and fixed points of the closed form."""
    x = _float_sample(2.0 ** -30, 90.0, 1_500_000)
    s = oracle.sigmoid_f32(x)
    exact = (1.0 / (1.0 + np.exp(-x.astype(np.float64)))).astype(np.float32)
    d = _ulps(s, exact)
    assert d.max() <= 1
    assert (d == 0).mean() > 0.99  # 99.1% on this sample
    inner = np.abs(x) <= 80  # torch flushes part of the subnormal range beyond
    assert _ulps(s[inner], torch.sigmoid(torch.from_numpy(x[inner])).numpy()).max() <= 2
    np.testing.assert_array_equal(s.view(np.uint32), oracle.sigmoid_numpy(x).view(np.uint32))
    special = np.float32([0.0, -0.0, 88.0, 104.0, 1e30, -87.0, -87.5, -103.0, -104.0, -200.0,
                          -1e30])
    got = oracle.sigmoid_f32(special)
    assert got[0] == 0.5 and got[1] == 0.5
    assert (got[2:5] == 1.0).all()
    assert got[-3] == 0.0 and got[-2] == 0.0 and got[-1] == 0.0
    ref = (1.0 / (1.0 + np.exp(-special[5:8].astype(np.float64)))).astype(np.float32)
    assert _ulps(got[5:8], ref).max() <= 1
    # symmetry of the closed form: s(x) + s(-x) = 1 to within an ulp of 1
    y = x[(np.abs(x) < 16)]
    np.testing.assert_allclose(oracle.sigmoid_f32(y).astype(np.float64)
                               + oracle.sigmoid_f32(-y).astype(np.float64), 1.0, atol=2.0 ** -23)


def test_exp_f32_pinned():
    """The softmax weights' exp (oracle_exp_f32): within 1 ulp of the correctly rounded exp on
    [-87, 0] (softmax arguments x_k - x_max are <= 0), e^0 = 1 exactly, and equal to the numpy
    statement."""
    x = -_float_sample(2.0 ** -30, 87.0, 1_000_000)
    x = x[x <= 0]
    e = oracle.exp_f32(x)
    exact = np.exp(x.astype(np.float64)).astype(np.float32)
    assert _ulps(e, exact).max() <= 1
    np.testing.assert_array_equal(e.view(np.uint32), oracle.exp_numpy(x).view(np.uint32))
    assert oracle.exp_f32(np.float32([0.0]))[0] == 1.0


def test_fma32_emulation():
    """The numpy fma used by the numpy statements: exact against fp64 where the fp64 sum is
    exact, and the midpoint tie-break on constructed cases."""
    rng = np.random.default_rng(1)
    a = rng.standard_normal(100000).astype(np.float32)
    b = rng.standard_normal(100000).astype(np.float32)
    c = np.ldexp(rng.standard_normal(100000), rng.integers(-30, 30, 100000)).astype(np.float32)
    got = oracle.fma32(a, b, c)
    # fp64 products of fp32 are exact; with |c| not far from |ab| the fp64 sum is exact too,
    # and then one rounding to fp32 is the fused result
    p = a.astype(np.float64) * b.astype(np.float64)
    ok = np.abs(np.log2(np.abs(c) + 1e-300) - np.log2(np.abs(p) + 1e-300)) < 4
    np.testing.assert_array_equal(got[ok], (p + c.astype(np.float64))[ok].astype(np.float32))
    # 658529 * 104353 = 2^36 + 1, so a*b = 2^-24 + 2^-60 and 1 + a*b lies just above the
    # midpoint between 1 and 1 + 2^-23: the fused result rounds up, while rounding the fp64 sum
    # (which drops 2^-60 and lands on the midpoint) and then to fp32 gives 1.0
    a1 = np.float32(658529 * 2.0 ** -30)
    b1 = np.float32(104353 * 2.0 ** -30)
    assert 658529 * 104353 == 2 ** 36 + 1
    assert (a1.astype(np.float64) * b1 + 1.0).astype(np.float32) == 1.0
    assert oracle.fma32(a1, b1, np.float32(1.0)) == np.float32(1 + 2.0 ** -23)
    assert oracle.fma32(-a1, b1, np.float32(-1.0)) == np.float32(-(1 + 2.0 ** -23))
    assert oracle.fma32(a1, b1, np.float32(-1.0)) == np.float32(-1.0 + 2.0 ** -24)


def test_softmax_routing_against_torch():
    geom = QWEN3
    x = _logits(200, 128, seed=4)
    idx, w = oracle.route(x, None, geom, 1.0)
    p = torch.softmax(x, dim=1)
    top = p.topk(8, dim=1)
    assert torch.equal(torch.from_numpy(idx).long(), top.indices)
    w_ref = top.values / top.values.sum(1, keepdim=True)
    torch.testing.assert_close(torch.from_numpy(w), w_ref, rtol=1e-5, atol=1e-7)
    np.testing.assert_allclose(w.sum(1), 1.0, rtol=1e-5)


@pytest.mark.parametrize("off", [0, 16, 48, 64])
def test_permute_invariants(off):
    geom = SMALL_DS
    x = _logits(500, geom.num_experts, seed=off)
    idx, w = oracle.route(x, _bias(geom.num_experts, off), geom, 2.5)
    p = oracle.permute(idx, w, off, geom.local_experts)
    le = idx - off
    local = (le >= 0) & (le < geom.local_experts)
    hist = np.bincount(le[local], minlength=geom.local_experts)
    np.testing.assert_array_equal(p["counts"], hist)
    np.testing.assert_array_equal(p["offsets"], np.concatenate([[0], np.cumsum(hist)]))
    for e in range(geom.local_experts):
        seg = p["sorted_tok"][p["offsets"][e]:p["offsets"][e + 1]]
        np.testing.assert_array_equal(seg, np.nonzero((le == e).any(1))[0])  # torch.nonzero order
    T, K = idx.shape
    for t in range(T):
        for k in range(K):
            q = p["pair_of"][t, k]
            if local[t, k]:
                assert p["sorted_tok"][q] == t and p["sorted_w"][q] == w[t, k]
                assert p["offsets"][le[t, k]] <= q < p["offsets"][le[t, k] + 1]
            else:
                assert q == -1
    # destinations, by a per-token loop: the token's local pairs sorted by expert go to output
    # row t, then to partial rows t*(k-1), t*(k-1)+1, ...; every destination is used once
    k = min(K, geom.local_experts)
    seen = set()
    for t in range(T):
        mine = sorted((le[t, a], p["pair_of"][t, a]) for a in range(K) if local[t, a])
        for j, (_, q) in enumerate(mine):
            d = int(p["pair_dst"][q])
            assert d == (t if j == 0 else -1 - (t * (k - 1) + j - 1))
            assert d not in seen
            seen.add(d)
    assert len(p["pair_dst"]) == int(local.sum())


def test_dequant_layouts():
    g = torch.Generator().manual_seed(0)
    q = (torch.randn(2, 256, 384, generator=g)).to(torch.float8_e4m3fn)
    s = torch.rand(2, 2, 3, generator=g) + 0.5
    d = oracle.dequant_blocks(q, s)
    for e in range(2):
        for r in (0, 127, 128, 255):
            for c in (0, 127, 128, 383):
                assert d[e, r, c] == q[e, r, c].float() * s[e, r // 128, c // 128]
    hs = torch.randn(5, 256, generator=g).to(torch.float8_e4m3fn)
    hss = torch.rand(2, 5, generator=g) + 0.5  # [H/128, T]
    a = oracle.dequant_activations(hs, hss)
    for t in range(5):
        for c in (0, 127, 128, 255):
            assert a[t, c] == hs[t, c].float() * hss[c // 128, t]


def test_moe_reference_closed_form():
    """Identity weights with distinct block scales: out = sum_k w_k * (a * silu(2a)) exactly
    in the structure, which pins the SwiGLU half order (X1 linear, silu on X2), the transposed
    activation-scale layout and the per-block weight-scale indices."""
    geom = Geometry(256, 256, 64, 16, 4, 4, 2, ROUTING_DS)
    T, H, I, El = 6, 256, 256, 16
    g = torch.Generator().manual_seed(1)
    hs = (torch.rand(T, H, generator=g) * 2 - 1).to(torch.float8_e4m3fn)
    hss = torch.rand(H // 128, T, generator=g) + 0.5
    eye = torch.eye(H)
    w13 = torch.cat([eye[:I], eye[:I]], dim=0).expand(El, 2 * I, H).to(torch.float8_e4m3fn).contiguous()
    # block scales: X1 blocks scale 1, X2 blocks scale 2 -> X2 = 2 * X1
    s13 = torch.ones(El, 2 * I // 128, H // 128)
    s13[:, I // 128:, :] = 2.0
    w2 = eye[:, :I].expand(El, H, I).to(torch.float8_e4m3fn).contiguous()
    s2 = torch.full((El, H // 128, I // 128), 0.5)
    logits = torch.randn(T, 64, generator=g)
    bias = torch.zeros(64, dtype=torch.bfloat16)
    inp = dict(routing_logits=logits, routing_bias=bias, hidden_states=hs, hidden_states_scale=hss,
               gemm1_weights=w13, gemm1_weights_scale=s13, gemm2_weights=w2,
               gemm2_weights_scale=s2, local_expert_offset=0, routed_scaling_factor=2.5)
    out, inter = oracle.moe_reference(inp, geom, return_intermediates=True)
    a = hs.float() * hss.t().repeat_interleave(128, dim=1)
    c = a * torch.nn.functional.silu(2 * a) * 0.5
    idx, w = inter["topk_idx"], inter["topk_w"]
    wl = torch.from_numpy(np.where(idx < El, w, 0)).sum(1)
    expect = (c * wl[:, None]).to(torch.bfloat16)
    torch.testing.assert_close(out.float(), expect.float(), rtol=1e-2, atol=1e-3)
    # swapping the halves would give 2a * silu(a) instead -- make sure the two differ here
    wrong = (2 * a * torch.nn.functional.silu(a) * 0.5 * wl[:, None]).to(torch.bfloat16)
    assert not torch.allclose(out.float(), wrong.float(), rtol=1e-2, atol=1e-3)


def test_synthetic_inputs_shapes_and_quantisation():
    d = jin.make_activations(DS_V3, 16, seed=0)
    assert d["hidden_states"].dtype == torch.float8_e4m3fn and d["hidden_states"].shape == (16, 7168)
    assert d["hidden_states_scale"].shape == (56, 16)
    # per-token 1x128 blocks: the block maximum maps to 448
    q = d["hidden_states"].float().reshape(16, 56, 128).abs().amax(2)
    assert torch.all(q == 448.0)
    w13, s13, w2, s2 = jin.make_weights(Geometry(256, 128, 64, 2, 4, 4, 2, ROUTING_DS), seed=0)
    assert w13.shape == (2, 256, 256) and s13.shape == (2, 2, 2)
    assert w2.shape == (2, 256, 128) and s2.shape == (2, 2, 1)
    blocks = w13.float().reshape(2, 2, 128, 2, 128).abs().amax(dim=(2, 4))
    assert torch.all(blocks == 448.0)
