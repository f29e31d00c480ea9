"""Pins the per-token / per-channel restatement (oracle/token_channel.py).

fma32 is checked against rational arithmetic, including products that land exactly
on an fp32 midpoint with a tiny addend on either side (where rounding the float64 sum
first would go wrong); the token scale against the exact quotient m / 448; the token
codes against a rational-arithmetic restatement of activation_token.c on small rows
(zero, tiny, huge, mixed-sign rows) and against the dequantization bound.
"""

import numpy as np
import pytest
import torch

from oracle import e4m3, fp8_codec
from oracle import token_channel as tc

F32 = np.float32


def test_fma32_random_against_rationals():
    rng = np.random.default_rng(1)
    a = rng.standard_normal(3000).astype(F32)
    b = (rng.standard_normal(3000) * 10).astype(F32)
    c = (rng.standard_normal(3000) * np.exp2(rng.integers(-30, 5, 3000))).astype(F32)
    got = tc.fma32(a, b, c)
    for i in range(3000):
        assert got[i] == tc.fma32_exact(a[i], b[i], c[i]), i


@pytest.mark.parametrize("tiny", [0.0, 2.0 ** -60, -(2.0 ** -60)])
def test_fma32_midpoints(tiny):
    # (1 + 2^-12)^2 = 1 + 2^-11 + 2^-24: exactly halfway between two fp32 neighbours
    a = F32(1.0 + 2.0 ** -12)
    c = F32(tiny)
    got = tc.fma32(np.array([a]), np.array([a]), np.array([c]))[0]
    want = tc.fma32_exact(a, a, c)
    assert got == want
    lo, hi = F32(1.0 + 2.0 ** -11), np.nextafter(F32(1.0 + 2.0 ** -11), F32(2.0))
    assert want == (hi if tiny > 0 else lo if tiny < 0 else (lo if (int(np.array(lo).view(np.uint32)) & 1) == 0 else hi))


def test_token_scale_is_near_exact_quotient():
    rng = np.random.default_rng(2)
    m = np.abs(rng.standard_normal(5000) * np.exp2(rng.integers(-20, 20, 5000))).astype(F32)
    s = tc.token_scale(m)
    exact = m.astype(np.float64) / 448.0
    ulp = np.spacing(s).astype(np.float64)
    assert np.all(np.abs(s.astype(np.float64) - exact) <= 0.5 * ulp + 1e-45)
    for i in range(0, 5000, 97):
        want = tc.fma32_exact(tc.fma32_exact(-F32(m[i] * tc.INV448), 448.0, m[i]), tc.INV448, F32(m[i] * tc.INV448))
        assert s[i] == want


def rows():
    rng = np.random.default_rng(3)
    x = (rng.standard_normal((6, 384)) * 3).astype(F32)
    x[1] = 0.0                                          # all-zero row: scale from m = 1
    x[2] *= 1e-30                                       # tiny row (bf16 keeps it)
    x[3] *= 1e30                                        # huge row
    x[4, ::3] = 0.0
    x[5, 7] = -448.0 * 1e3                              # one dominating element
    return torch.tensor(x).bfloat16()


def test_token_quant_against_rationals():
    xb = rows()
    q, s = tc.token_quant(xb)
    for r in range(xb.shape[0]):
        qe, se = tc.token_quant_exact(xb[r].float().numpy())
        assert np.array_equal(q[r], qe), r
        assert s[r] == se, r
    assert s[1] == F32(2.0) * tc.token_scale(np.array([1.0], dtype=F32))[0]
    assert np.all(q[1] & 0x7F == 0)


def test_token_quant_dequantization_bound():
    xb = rows()
    q, s = tc.token_quant(xb)
    x = xb.float().numpy().astype(np.float64)
    # half-range code value = v / 2 with v the OCP rounding of x / s: dec(code) * (2 s) ~ x
    inv = fp8_codec.inverse_table()
    back = e4m3.decode(q).astype(np.float64) * s[:, None].astype(np.float64)
    ocp = e4m3.decode(inv[q]) * (s[:, None].astype(np.float64) / 2.0)
    assert np.array_equal(back, ocp)                          # both views of the same value
    rel = np.abs(back - x) <= np.maximum(np.abs(x) * 2.0 ** -4, s[:, None] * 2.0 ** -9 * 2) + 1e-300
    assert rel.all()


def test_channel_finish_against_rationals():
    """channel_finish.c:9-15 by exact arithmetic: fp32(p * a), then (x0 * w + b) rounded once to fp32 by
    Fraction, then bf16 by torch's RNE cast (independent of the oracle's own bf16 helper)."""
    rng = np.random.default_rng(4)
    p = (rng.standard_normal((6, 48)) * 100).astype(F32)
    p[0, :4] = [0.0, -0.0, 1e-30, -3e38]
    a = rng.random(6).astype(F32)
    w = rng.random(48).astype(F32)
    b = rng.standard_normal(48).astype(F32)
    b[5] = -float(F32(p[0, 5] * a[0]) * w[5])            # near-cancellation
    for bias in (b, None):
        y = tc.channel_finish(p, a, w, bias)
        want = np.empty(p.shape, dtype=F32)
        for i in range(p.shape[0]):
            for j in range(p.shape[1]):
                x0 = F32(p[i, j] * a[i])
                bj = 0.0 if bias is None else float(bias[j])
                want[i, j] = tc.fma32_exact(x0, w[j], F32(bj))
        bits = torch.from_numpy(want).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
        assert np.array_equal(y, bits)
