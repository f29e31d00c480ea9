"""The RMSNorm restatement (oracle/norm.py) against what pins it, on the CPU.

* The reference's own device test (tests/track_a_device_verify.cpp:465-540): its inputs (widths 64 and 576,
  weight_offset 0 and 1, epsilon 1e-5), residual_out bit for bit, norm_out within 2 bf16 ulps of its fp64
  evaluation -- the reference's gate.
* Mathematics: the fixed-order fp64 sum of squares against the exact rational sum rounded once; the inverse
  against a 60-digit evaluation of 1/sqrt (within one fp32 ulp); the +inf argument giving 0 (norm_math.h:22).
* Planted mistakes (a dropped weight_offset, the squares of x instead of the summed rows, a missing epsilon on
  near-zero rows) fail the gate.
"""

import decimal
from fractions import Fraction

import numpy as np
import pytest
import torch

from oracle import norm


def within_gate(got, r, gamma, eps, off):
    ref = torch.from_numpy(norm.fp64_reference(r, gamma, eps, off).astype(np.float32)).to(torch.bfloat16)
    return int(norm.bf16_ulp_diff(got, ref).max())


@pytest.mark.parametrize("width", [64, 576])
@pytest.mark.parametrize("offset", [0.0, 1.0])
def test_reference_device_test_cases(width, offset):
    x, res, gamma = norm.reference_test_inputs(width)
    eps = 1e-5
    assert within_gate(norm.rms_norm(x, gamma, eps, offset), x, gamma, eps, offset) <= norm.GATE_ULPS
    r, n = norm.fused_add_rms_norm(x, res, gamma, eps, offset)
    # residual: the fp32 sum of two bf16 values, computed exactly in fp64 and rounded once to fp32, then RNE
    exact = (x.double() + res.double()).float().to(torch.bfloat16)
    assert torch.equal(r.view(torch.int16), exact.view(torch.int16))
    assert within_gate(n, r, gamma, eps, offset) <= norm.GATE_ULPS


@pytest.mark.parametrize("width", [1, 7, 100, 128, 1000, 4096, 8192])
def test_random_rows_within_gate(width):
    gen = torch.Generator().manual_seed(width)
    x = (torch.randn(3, width, generator=gen) * torch.tensor([1e-3, 1.0, 300.0])[:, None]).bfloat16()
    res = torch.randn(3, width, generator=gen).bfloat16()
    gamma = (torch.rand(width, generator=gen) * 2 - 0.5).bfloat16()
    for off in (0.0, 1.0, -0.25):
        assert within_gate(norm.rms_norm(x, gamma, 1e-6, off), x, gamma, 1e-6, off) <= norm.GATE_ULPS
        r, n = norm.fused_add_rms_norm(x, res, gamma, 1e-6, off)
        assert within_gate(n, r, gamma, 1e-6, off) <= norm.GATE_ULPS


def test_sum_of_squares_is_the_exact_sum_rounded_once():
    gen = torch.Generator().manual_seed(7)
    for width in (5, 333, 2048, 8192):
        x = (torch.randn(2, width, generator=gen) * torch.tensor([0.01, 50.0])[:, None]).bfloat16()
        got = norm.sum_squares(x)
        for i in range(2):
            exact = sum(Fraction(float(v)) ** 2 for v in x[i].float().tolist())
            assert got[i] == np.float32(float(exact)), (width, i)  # float(Fraction) rounds once


def test_inverse_within_one_ulp_and_inf():
    decimal.getcontext().prec = 60
    rng = np.random.default_rng(3)
    ss = np.concatenate([rng.random(200).astype(np.float32) * 10.0 ** rng.integers(-20, 20, 200),
                         np.array([0.0, 1.0, 3.0e38], dtype=np.float32)]).astype(np.float32)
    for width in (1, 576, 8192):
        inv = norm.inverse_rms(ss, width, 1e-6)
        for s, got in zip(ss, inv):
            arg = np.float32(np.float32(s * np.float32(1.0 / np.float32(width))) + np.float32(1e-6))
            want = 1 / decimal.Decimal(float(arg)).sqrt()
            want32 = np.float32(float(want))
            assert abs(int(got.view(np.int32)) - int(want32.view(np.int32))) <= 1, (s, width)
    big = norm.inverse_rms(np.array([np.inf], dtype=np.float32), 64, 1e-5)
    assert big[0] == 0.0


def test_gate_catches_planted_mistakes():
    x, res, gamma = norm.reference_test_inputs(576)
    eps = 1e-5
    # weight_offset dropped
    inv = norm.inverse_rms(norm.sum_squares(x), 576, eps)
    wrong = norm.normalize(x, inv, gamma, 0.0)
    assert within_gate(wrong, x, gamma, eps, 1.0) > norm.GATE_ULPS
    # fused form normalizing with the squares of x instead of the summed rows
    r = norm.fused_add(x, res)
    wrong = norm.normalize(r, norm.inverse_rms(norm.sum_squares(x), 576, eps), gamma, 0.0)
    assert within_gate(wrong, r, gamma, eps, 0.0) > norm.GATE_ULPS
    # epsilon dropped, seen on a near-zero row
    tiny = (torch.ones(1, 64) * 1e-4).bfloat16()
    g = torch.ones(64).bfloat16()
    wrong = norm.normalize(tiny, norm.inverse_rms(norm.sum_squares(tiny), 64, 0.0 + 1e-30), g, 0.0)
    assert within_gate(wrong, tiny, g, 1e-5, 0.0) > norm.GATE_ULPS
