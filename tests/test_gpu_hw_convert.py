"""The two hardware conversions the kernels use, against the software roundings of
csrc/gk_fp8_math.h that tests/test_math_host.py pins to the oracle:

* the paired fp32 -> bf16 rounding (bf16x2_rne in csrc/gk_fp8_internal.h: gfx950's v_cvt_pk_bf16_f32
  plus a NaN fix-up) against bf16_rne (NaN -> 0x7fc0) on every one of the 2^32 float bit patterns, in
  both positions of the pair.  Every GEMM epilogue, the SiLU/GELU-and-mul ops, the norms, the rank sum
  and the MoE layer's SiLU quantizer and combine round through it;
* the activation quantizer's E4M3 encode (quant_group8: v_cvt_pk_fp8_f32 into both halves of the
  packed word) against e4m3_rne on every fp32 with |v| <= 464, both signs -- the range of the
  quantizer's quotients (|x / s| < 464 as s >= amax / 448 up to two fp32 roundings).
"""

import ctypes
import os

import pytest
import torch

pytestmark = pytest.mark.gpu

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def run_check(name):
    lib = ctypes.CDLL(os.path.join(ROOT, "tests", "csrc", "libgk_probe.so"))
    fn = getattr(lib, name)
    fn.restype = ctypes.c_int
    fn.argtypes = [ctypes.c_void_p, ctypes.c_void_p]
    counts = torch.zeros(2, dtype=torch.int64, device="cuda")
    assert fn(ctypes.c_void_p(counts.data_ptr()), ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)) == 0
    torch.cuda.synchronize()
    return tuple(int(v) for v in counts.cpu())


def test_bf16x2_rne_equals_software_rne_on_all_floats():
    mismatches, checked = run_check("gk_probe_bf16x2_check")
    assert checked == 2 ** 33
    assert mismatches == 0


def test_e4m3_encode_equals_software_rne_up_to_464():
    mismatches, checked = run_check("gk_probe_e4m3_check")
    assert checked == 2 * 0x43E80001
    assert mismatches == 0
