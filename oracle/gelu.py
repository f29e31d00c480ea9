"""CPU restatement of the reference's GELU-and-mul op (test infrastructure only).

gk_gelu_and_mul_bf16_v1 (csrc/tpc/generic_dense/gelu_and_mul_bf16.c:4-49, glue
csrc/host/generic_dense_glue.cpp:424-458): gate_up bf16 [rows, 2W] -> bf16 [rows, W],
out = bf16(gelu(gate) * up) with the product in fp32.  approximate = 0 is the exact GELU,
approximate = 1 the tanh form.  The reference evaluates GELU with its own fp32 polynomials
(csrc/tpc/common/tpc_math_safe.h); its test bounds the op against the fp64 evaluation restated
here (tests/track_a_device_verify.cpp:274-286) to one bf16 ulp (:429-462), which is the gate
the GPU op is held to.

Pinned by: the exact form against Python's math.erfc and the identity 1 - erf; the tanh form's
sigmoid evaluation against 0.5 (1 + tanh(.)) with the published constants sqrt(2/pi) and 0.044715;
the special values (+inf -> +inf, -inf -> 0, NaN -> NaN).  See tests/test_oracle_gelu.py.
"""

import math

import numpy as np
import torch

GATE_ULPS = 1  # tests/track_a_device_verify.cpp:456
SQRT_2_OVER_PI_X2 = 1.59576912160573071176  # 2 * sqrt(2 / pi)


def gelu_exact(x):
    """fp64 exact GELU of a float: x * erfc(-x / sqrt(2)) / 2 (track_a_device_verify.cpp:274-277)."""
    if math.isinf(x):
        return x if x > 0 else 0.0
    if math.isnan(x):
        return x
    return 0.5 * x * math.erfc(-x * 0.70710678118654752440)


def gelu_tanh(x):
    """fp64 tanh-form GELU: x * sigmoid(2 sqrt(2/pi) (x + 0.044715 x^3)) (track_a_device_verify.cpp:279-286)."""
    if math.isinf(x):
        return x if x > 0 else 0.0
    if math.isnan(x):
        return x
    u2 = SQRT_2_OVER_PI_X2 * (x + 0.044715 * x * x * x)
    if u2 >= 0.0:
        return x / (1.0 + math.exp(-u2))
    e = math.exp(u2)
    return x * (e / (1.0 + e))


def gelu_and_mul_f64(gate_up, approximate=False):
    """fp64 [rows, W]: gelu(gate) * up from a bf16 [rows, 2W] tensor."""
    w = gate_up.shape[1] // 2
    g = gate_up[:, :w].double().numpy()
    u = gate_up[:, w:].double().numpy()
    f = np.vectorize(gelu_tanh if approximate else gelu_exact, otypes=[np.float64])
    return f(g) * u


def reference_bf16(gate_up, approximate=False):
    """bf16 of the fp64 value (rounded to fp32 first, as the reference test does)."""
    return torch.from_numpy(gelu_and_mul_f64(gate_up, approximate).astype(np.float32)).to(torch.bfloat16)


def within_gate(got, gate_up, approximate=False):
    """Max bf16-ulp distance to the fp64 value, skipping reference values below FLT_MIN where the op gives 0
    (the test's own exception, track_a_device_verify.cpp:452)."""
    ref32 = torch.from_numpy(gelu_and_mul_f64(gate_up, approximate).astype(np.float32))
    ref = ref32.to(torch.bfloat16)
    ia = got.view(torch.int16).numpy().astype(np.int32)
    ib = ref.view(torch.int16).numpy().astype(np.int32)
    ka = np.where(ia < 0, -32768 - ia, ia)
    kb = np.where(ib < 0, -32768 - ib, ib)
    d = np.abs(ka - kb)
    skip = (ref32.abs().numpy() < np.finfo(np.float32).tiny) & (got.float().numpy() == 0.0)
    both_nan = np.isnan(got.float().numpy()) & np.isnan(ref32.numpy())
    return int(np.where(skip | both_nan, 0, d).max())


def reference_test_input(width=576, rows=5):
    """The gelu_and_mul input of tests/track_a_device_verify.cpp:432-438: bf16 [rows, 2*width]."""
    c = np.arange(2 * width)[None, :]
    r = np.arange(rows)[:, None]
    v = (((c * 17 + r * 31) % 61) - 30).astype(np.float32) * np.float32(0.2)
    return torch.from_numpy(v.astype(np.float32)).to(torch.bfloat16)
