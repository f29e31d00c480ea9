"""The GELU restatement (oracle/gelu.py) against closed forms, on the CPU.

* Exact form: equals x (1 + erf(x / sqrt 2)) / 2 away from the cancellation region, and is the erfc form
  of tests/track_a_device_verify.cpp:274-277.
* Tanh form: its sigmoid evaluation equals x (1 + tanh(sqrt(2/pi) (x + 0.044715 x^3))) / 2, the published
  approximation (a wrong constant fails).
* Special values and the reference test's own inputs.
"""

import math

import numpy as np
import torch

from oracle import gelu


def test_exact_form_matches_erf_identity():
    for x in np.linspace(-3.0, 3.0, 601):
        want = 0.5 * x * (1.0 + math.erf(x / math.sqrt(2.0)))
        got = gelu.gelu_exact(float(x))
        assert abs(got - want) <= 1e-14 * max(1.0, abs(want)), x


def test_tanh_form_matches_published_approximation():
    k = math.sqrt(2.0 / math.pi)
    for x in np.linspace(-6.0, 6.0, 1201):
        want = 0.5 * x * (1.0 + math.tanh(k * (x + 0.044715 * x ** 3)))
        got = gelu.gelu_tanh(float(x))
        # below x = -3 the closed form itself loses digits to 1 + tanh(.) ~ 0
        tol = 1e-13 if x >= -3.0 else 1e-4
        assert abs(got - want) <= tol * max(1e-30, abs(want)), x
    # a planted mistake: sqrt(2/pi) where 2 sqrt(2/pi) belongs in the sigmoid form
    x = 1.0
    wrong = x / (1.0 + math.exp(-k * (x + 0.044715 * x ** 3)))
    assert abs(wrong - gelu.gelu_tanh(x)) > 1e-2


def test_special_values():
    for f in (gelu.gelu_exact, gelu.gelu_tanh):
        assert f(float("inf")) == float("inf")
        assert f(float("-inf")) == 0.0
        assert math.isnan(f(float("nan")))
        assert f(0.0) == 0.0
    assert gelu.gelu_exact(-40.0) == 0.0 or abs(gelu.gelu_exact(-40.0)) < 1e-300


def test_reference_test_input_and_gate_helper():
    x = gelu.reference_test_input()
    assert x.shape == (5, 1152) and x.dtype == torch.bfloat16
    assert float(x[0, 0]) == -6.0 and float(x[1, 0]) == float(torch.tensor((31 - 30) * 0.2).bfloat16())
    ref = gelu.reference_bf16(x)
    assert gelu.within_gate(ref, x) == 0
    off = ref.view(torch.int16).clone()
    off[0, 5] += 2
    assert gelu.within_gate(off.view(torch.bfloat16), x) == 2
