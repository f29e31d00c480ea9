"""The kernels' paired fp32 -> bf16 rounding (bf16x2_rne in csrc/gk_fp8_internal.h: gfx950's
v_cvt_pk_bf16_f32 plus a NaN fix-up) against the software round-to-nearest-even the oracle and
tests/test_math_host.py pin (bf16_rne; NaN -> 0x7fc0), on every one of the 2^32 float bit patterns in
both positions of the pair.  Every GEMM epilogue, the SiLU/GELU-and-mul ops, the norms, the rank sum
and the MoE layer's SiLU quantizer and combine round through it.
"""

import ctypes
import os

import pytest
import torch

from gaudi_kernels import _native as nat

pytestmark = pytest.mark.gpu


def test_bf16x2_rne_equals_software_rne_on_all_floats():
    probe = os.path.join(os.path.dirname(nat.lib_path()), "libgk_probe.so")
    lib = ctypes.CDLL(probe)
    lib.gk_probe_bf16x2_check.restype = ctypes.c_int
    lib.gk_probe_bf16x2_check.argtypes = [ctypes.c_void_p, ctypes.c_void_p]
    counts = torch.zeros(2, dtype=torch.int64, device="cuda")
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    assert lib.gk_probe_bf16x2_check(ctypes.c_void_p(counts.data_ptr()), stream) == 0
    torch.cuda.synchronize()
    mismatches, checked = (int(v) for v in counts.cpu())
    assert checked == 2 ** 33
    assert mismatches == 0
