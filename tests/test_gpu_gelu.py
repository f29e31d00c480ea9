"""GELU-and-mul on the GPU (gk_gelu_and_mul_bf16, gk_fp8_gelu_mul_quant_bf16), both forms.

* The reference test's gate (tests/track_a_device_verify.cpp:429-462): every output within one bf16 ulp of
  the fp64 value, on its own input, special values, random and ragged rows, strided input.
* The fused quantizer: codes and scales equal act_quant of the bf16 op output in both layouts and modes.
* The glue's rejection of approximate values other than 0 and 1 (generic_dense_glue.cpp:424-431).
"""

import ctypes

import pytest
import torch

from gaudi_kernels import _native as nat
from gaudi_kernels import ops
from oracle import gelu

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("approximate", [False, True])
def test_reference_input_within_one_ulp(approximate):
    x = gelu.reference_test_input()
    y = ops.gelu_and_mul(x.cuda(), approximate=approximate).cpu()
    assert gelu.within_gate(y, x, approximate) <= gelu.GATE_ULPS


@pytest.mark.parametrize("approximate", [False, True])
def test_special_values(approximate):
    vals = [0.0, -0.0, 1e-6, -1e-6, 0.6249, -0.6249, 0.625, -0.625, 1.249, -1.249, 1.25, -1.25, 3.0, -3.0,
            10.0, -10.0, 15.0, -15.0, 20.0, -20.0, 88.0, -88.0, 100.0, -100.0,
            float("inf"), float("-inf"), float("nan")]
    w = len(vals)
    g = torch.tensor(vals).repeat(2, 1)
    u = torch.ones(2, w)
    u[1] = torch.linspace(-2.0, 2.0, w)
    x = torch.cat([g, u], dim=1).bfloat16()
    y = ops.gelu_and_mul(x.cuda(), approximate=approximate).cpu()
    assert gelu.within_gate(y, x, approximate) <= gelu.GATE_ULPS
    assert float(y[0, vals.index(float("inf"))]) == float("inf")
    assert float(y[0, vals.index(float("-inf"))]) == 0.0


@pytest.mark.parametrize("rows,width", [(1, 128), (37, 14336), (5, 333), (256, 1024), (3, 7)])
@pytest.mark.parametrize("approximate", [False, True])
def test_random_rows_within_one_ulp(rows, width, approximate):
    gen = torch.Generator().manual_seed(rows * 7 + width)
    x = (torch.randn(rows, 2 * width, generator=gen) * 3.0).bfloat16()
    y = ops.gelu_and_mul(x.cuda(), approximate=approximate).cpu()
    assert gelu.within_gate(y, x, approximate) <= gelu.GATE_ULPS


def test_strided_rows():
    rows, width = 6, 1000
    base = (torch.randn(rows, 2 * width + 3, generator=torch.Generator().manual_seed(5)) * 2).bfloat16().cuda()
    x = base[:, 1:2 * width + 1]
    a = ops.gelu_and_mul(x)
    b = ops.gelu_and_mul(x.contiguous())
    assert torch.equal(a.view(torch.int16), b.view(torch.int16))


@pytest.mark.parametrize("rows,width", [(1, 4096), (16, 14336), (5, 333), (40, 1024), (300, 1024)])
@pytest.mark.parametrize("native_half", [False, True])
@pytest.mark.parametrize("approximate", [False, True])
def test_gelu_mul_quant_equals_composition(rows, width, native_half, approximate):
    gen = torch.Generator().manual_seed(rows + width)
    x = (torch.randn(rows, 2 * width, generator=gen) * 2.0).bfloat16().cuda()
    h = ops.gelu_and_mul(x, approximate=approximate)
    m_pad = rows + 3
    q1, s1 = ops.gelu_mul_quant(x, approximate=approximate, native_half=native_half, m_pad=m_pad)
    q2, s2 = ops.act_quant(h, native_half=native_half, m_pad=m_pad)
    assert torch.equal(q1.cpu(), q2.cpu())
    assert torch.equal(s1.cpu().view(torch.int32), s2.cpu().view(torch.int32))
    if rows <= 64:
        p1, t1 = ops.gelu_mul_quant(x, approximate=approximate, native_half=native_half, decode_layout=True)
        p2, t2 = ops.act_quant(h, native_half=native_half, decode_layout=True)
        assert torch.equal(p1.cpu(), p2.cpu()) and torch.equal(t1.cpu().view(torch.int32), t2.cpu().view(torch.int32))


def test_rejections():
    lib = nat.load()
    fake = ctypes.c_void_p(1 << 20)
    assert lib.gk_gelu_and_mul_bf16(fake, 4, 64, 128, fake, 64, 2, None) == nat.GK_UNSUPPORTED_LAYER_CONFIGURATION
    assert lib.gk_gelu_and_mul_bf16(fake, 4, 64, 100, fake, 64, 0, None) == nat.GK_INCOMPATIBLE_INPUT_SIZE
    assert lib.gk_gelu_and_mul_bf16(fake, 4, 64, 128, fake, 32, 1, None) == nat.GK_INCOMPATIBLE_OUTPUT_SIZE
    assert lib.gk_fp8_gelu_mul_quant_bf16(fake, 4, 64, 128, -1, fake, fake, 16, 0, None) == \
        nat.GK_UNSUPPORTED_LAYER_CONFIGURATION
