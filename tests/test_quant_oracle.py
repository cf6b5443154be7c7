"""Pins the activation-quantisation oracle (oracle.quantize_activations) without retyping it.

* The e4m3 rounding is checked against an independent table-driven encoder: all 256 codes are
  decoded from the OCP e4m3fn bit layout (bias 7, subnormals at exponent 0, 0x7f/0xff NaN) and a
  value is encoded as the nearest finite code, ties to the even code.
* Block properties fixed by the rule amax / 448: each block's largest |x| maps to +-448, the
  stored scale is amax / 448, all-zero blocks give scale 0 and zero codes, and every
  dequantised value is within half an e4m3 step of the input.
* Known answers on hand-built rows.
"""
import math

import numpy as np
import pytest
import torch

import oracle

F8 = torch.float8_e4m3fn


def e4m3_table():
    vals = []
    for code in range(256):
        s = -1.0 if code & 0x80 else 1.0
        e = (code >> 3) & 0xF
        m = code & 0x7
        if e == 0xF and m == 0x7:
            vals.append(math.nan)
        elif e == 0:
            vals.append(s * m * 2.0 ** -9)
        else:
            vals.append(s * (1 + m / 8.0) * 2.0 ** (e - 7))
    return np.array(vals)


TABLE = e4m3_table()
FINITE = np.array([c for c in range(256) if not math.isnan(TABLE[c])])


def encode_rne(x: float) -> int:
    """Nearest finite e4m3 code; ties go to the even code (even mantissa)."""
    d = np.abs(TABLE[FINITE] - x)
    best = d.min()
    cands = FINITE[d == best]
    if len(cands) > 1:
        # +0 and -0 both decode to 0: keep the sign of x
        if best == abs(x) and x == 0:
            return 0x80 if math.copysign(1, x) < 0 else 0x00
        even = [c for c in cands if (c & 1) == 0]
        cands = even or cands
        if len(cands) > 1:  # +-0 tie for tiny x: sign of x
            cands = [c for c in cands if (c & 0x80) == (0x80 if x < 0 else 0)] or cands
    return int(cands[0])


def torch_codes(v):
    return torch.tensor(v, dtype=torch.float32).to(F8).view(torch.uint8).numpy()


def test_torch_e4m3_cast_is_round_to_nearest_even():
    rng = np.random.default_rng(0)
    pos = np.sort(TABLE[FINITE][TABLE[FINITE] > 0])
    mids = (pos[:-1] + pos[1:]) / 2  # exact ties between neighbours
    xs = np.concatenate([pos, mids, -mids, rng.uniform(-448, 448, 4000),
                         rng.uniform(-0.02, 0.02, 2000), [0.0, 448.0, -448.0, 2.0 ** -10,
                                                          3 * 2.0 ** -11]])
    xs = xs.astype(np.float32)
    got = torch_codes(xs)
    want = np.array([encode_rne(float(x)) for x in xs], dtype=np.uint8)
    bad = np.nonzero(got != want)[0]
    assert bad.size == 0, [(float(xs[i]), int(got[i]), int(want[i])) for i in bad[:5]]


def test_block_properties_random():
    g = torch.Generator().manual_seed(3)
    x = (torch.randn(37, 640, generator=g) * torch.rand(37, 1, generator=g) * 10).bfloat16()
    x[5, 128:256] = 0  # an all-zero block
    q, s = oracle.quantize_activations(x)
    assert q.dtype == F8 and q.shape == x.shape and s.shape == (5, 37)
    xb = x.float().reshape(37, 5, 128)
    amax = xb.abs().amax(2)
    np.testing.assert_array_equal(s.t().numpy(), (amax / 448.0).numpy())
    assert s[1, 5] == 0 and (q.float().reshape(37, 5, 128)[5, 1] == 0).all()
    qb = q.float().reshape(37, 5, 128)
    nz = amax > 0
    # the block maximum lands on +-448
    top = qb.abs().amax(2)
    assert (top[nz] == 448.0).all()
    # every value within half an e4m3 step (relative 2^-4 for normals, 2^-10 absolute below)
    deq = qb * s.t()[:, :, None]
    err = (deq - xb).abs()
    rel = xb.abs() / torch.where(nz, s.t(), torch.ones_like(amax))[:, :, None]
    step = torch.where(rel >= 2.0 ** -6, 2.0 ** (torch.floor(torch.log2(rel.clamp_min(1e-30))) - 3),
                       torch.full_like(rel, 2.0 ** -9))
    bound = 0.5 * step * s.t()[:, :, None] * 1.0001 + 1e-30
    assert (err <= bound).all()


def test_known_answer_rows():
    # block 0: amax 896 -> scale 2; values 896, -448, 3, 1.125*2 -> codes 448, -224, 1.5, 1.125
    row = torch.zeros(1, 256)
    row[0, 0], row[0, 1], row[0, 2], row[0, 3] = 896.0, -448.0, 3.0, 2.25
    # block 1: all zero
    q, s = oracle.quantize_activations(row.bfloat16())
    assert s[0, 0].item() == 2.0 and s[1, 0].item() == 0.0
    np.testing.assert_array_equal(q.float()[0, :4].numpy(), [448.0, -224.0, 1.5, 1.125])
    assert (q.float()[0, 4:] == 0).all()
