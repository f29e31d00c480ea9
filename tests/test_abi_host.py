"""Host-side contract of libgk_fp8.so (no GPU needed).

Mirrors the reference's host contract tests (tests/generic_fp8_glue_test.cpp,
tests/generic_dense_guids_test.cpp): the provider loads (dlopen), exports
exactly the declared entry points, enumerates its op names with the
count-query idiom, and rejects bad inputs with the documented status codes
before touching the device (wrong scale grid -> INCOMPATIBLE_INPUT_SIZE, as
generic_fp8_glue_test.cpp:98-100; unknown or conflicting flags ->
UNSUPPORTED_LAYER_CONFIGURATION).  Plans report the variant chosen by M.
"""

import ctypes
import os
import re
import subprocess

import pytest

from gaudi_kernels import _native as nat
from gaudi_kernels import ops

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "gk_fp8.h")

pytestmark = pytest.mark.skipif(not os.path.exists(nat.lib_path()), reason="libgk_fp8.so not built")


def declared():
    text = open(HEADER).read()
    return sorted(set(re.findall(r"^\s*(?:gk_status|uint64_t)\s+(gk_\w+)\s*\(", text, re.MULTILINE)))


def test_exports_match_header():
    out = subprocess.run(["nm", "-D", "--defined-only", nat.lib_path()], check=True, capture_output=True,
                         text=True).stdout
    have = sorted({l.split()[-1] for l in out.splitlines() if " T " in l and l.split()[-1].startswith("gk_")})
    assert have == declared()
    assert sorted(nat.SIGNATURES) == declared()  # the Python binding binds every entry point


def test_load_version_and_ops():
    lib = nat.load()
    assert lib.gk_lib_version() == 1
    names = nat.list_ops()
    assert "gk_fp8_block_gemm_bf16_v1" in names and "gk_fp8_codec_ocp_to_half_v1" in names
    assert len(names) == len(set(names))
    # capacity smaller than the table -> names filled up to capacity + INSUFFICIENT_BUFFER
    cap = ctypes.c_uint32(2)
    arr = (ctypes.c_char_p * 2)()
    assert lib.gk_list_ops(ctypes.byref(cap), arr) == nat.GK_INSUFFICIENT_BUFFER
    assert cap.value == len(names) and arr[0].decode() == names[0]


def test_plan_dispatch_by_m():
    for m in (1, 2, 4, 8, 16):
        v, mp, ws = ops.plan(m, 6144, 4096)
        # quantized-activation scratch: 16 x 4096 codes + 16 x 32 scales
        assert v == nat.GK_VARIANT_DECODE and mp == 16 and ws == 16 * 4096 + 16 * 32 * 4
    for m, want_pad in ((17, 32), (32, 32), (33, 64), (64, 64)):
        v, mp, ws = ops.plan(m, 6144, 4096)
        # one to four 16-token tiles share each weight fragment
        assert v == nat.GK_VARIANT_DECODE and mp == want_pad and ws == want_pad * 4096 + want_pad * 32 * 4
    v, mp, ws = ops.plan(65, 6144, 4096)
    assert v == nat.GK_VARIANT_PREFILL and mp == 256
    v, mp, _ = ops.plan(4096, 7168, 7168)
    assert v == nat.GK_VARIANT_PREFILL and mp == 4096
    v, mp, _ = ops.plan(3, 200, 333)
    assert v == nat.GK_VARIANT_GENERIC and mp == 3  # K % 128 != 0
    assert ops.plan(3, 256, 256, nat.GK_FLAG_FORCE_PREFILL)[0] == nat.GK_VARIANT_PREFILL
    assert ops.plan(3, 256, 256, nat.GK_FLAG_FORCE_GENERIC)[0] == nat.GK_VARIANT_GENERIC


def status_of(fn, *args):
    return fn(*args)


def test_plan_rejections():
    lib = nat.load()
    p = ctypes.c_void_p(256)
    assert lib.gk_fp8_block_gemm_plan(0, 1, 1, 0, p, None, None, None) == nat.GK_INCOMPATIBLE_INPUT_SIZE
    assert lib.gk_fp8_block_gemm_plan(4, 256, 256, 1 << 10, p, None, None, None) == nat.GK_UNSUPPORTED_LAYER_CONFIGURATION
    both = nat.GK_FLAG_FORCE_DECODE | nat.GK_FLAG_FORCE_PREFILL
    assert lib.gk_fp8_block_gemm_plan(4, 256, 256, both, p, None, None, None) == nat.GK_UNSUPPORTED_LAYER_CONFIGURATION
    assert lib.gk_fp8_block_gemm_plan(65, 256, 256, nat.GK_FLAG_FORCE_DECODE, p, None, None, None) == \
        nat.GK_UNSUPPORTED_LAYER_CONFIGURATION
    # misaligned weights cannot take the tiled variants
    assert lib.gk_fp8_block_gemm_plan(4, 256, 256, nat.GK_FLAG_FORCE_DECODE, ctypes.c_void_p(257), None, None,
                                      None) == nat.GK_UNSUPPORTED_LAYER_CONFIGURATION


def test_gemm_rejects_wrong_scale_grid_before_device_use():
    lib = nat.load()
    fake = ctypes.c_void_p(1 << 20)
    ws = ctypes.c_void_p(1 << 21)
    # n = 512, k = 256 -> grid must be 4 x 2; {2, 3}-style mismatch -> INCOMPATIBLE_INPUT_SIZE
    st = lib.gk_fp8_block_gemm_bf16(fake, 4, 256, 256, fake, 512, fake, 2, 3, None, fake, 512, 0, ws, 1 << 20, None)
    assert st == nat.GK_INCOMPATIBLE_INPUT_SIZE
    st = lib.gk_fp8_block_gemm_bf16(fake, 4, 256, 256, fake, 512, fake, 4, 2, None, fake, 100, 0, ws, 1 << 20, None)
    assert st == nat.GK_INCOMPATIBLE_OUTPUT_SIZE
    st = lib.gk_fp8_block_gemm_bf16(fake, 4, 256, 256, fake, 512, fake, 4, 2, None, fake, 512, 0, ws, 16, None)
    assert st == nat.GK_INSUFFICIENT_BUFFER
    st = lib.gk_fp8_block_gemm_bf16(None, 4, 256, 256, fake, 512, fake, 4, 2, None, fake, 512, 0, ws, 1 << 20, None)
    assert st == nat.GK_INVALID_ARGUMENT
    st = lib.gk_fp8_block_gemm_q_bf16(fake, fake, 4, 8, 256, fake, 512, fake, 4, 2, None, fake, 512, 0, None)
    assert st == nat.GK_INCOMPATIBLE_INPUT_SIZE  # m_pad must equal the plan's (16 for decode)


def test_token_channel_gemm_rejects_before_device_use():
    lib = nat.load()
    fake = ctypes.c_void_p(1 << 20)
    f = lib.gk_fp8_token_channel_gemm_bf16
    # x, ldx, m, k, w, n, sw, bias, y, ldy, flags, stream
    assert f(fake, 256, 17, 256, fake, 512, fake, None, fake, 512, 0, None) == nat.GK_INCOMPATIBLE_INPUT_SIZE
    assert f(fake, 256, 4, 200, fake, 512, fake, None, fake, 512, 0, None) == nat.GK_INCOMPATIBLE_INPUT_SIZE
    assert f(fake, 128, 4, 256, fake, 512, fake, None, fake, 512, 0, None) == nat.GK_INCOMPATIBLE_INPUT_SIZE
    assert f(fake, 256, 4, 256, fake, 512, fake, None, fake, 100, 0, None) == nat.GK_INCOMPATIBLE_OUTPUT_SIZE
    assert f(fake, 260, 4, 256, fake, 512, fake, None, fake, 512, 0, None) == nat.GK_INCOMPATIBLE_DATA_TYPE
    assert f(ctypes.c_void_p((1 << 20) + 8), 256, 4, 256, fake, 512, fake, None, fake, 512, 0,
             None) == nat.GK_INCOMPATIBLE_DATA_TYPE
    assert f(fake, 256, 4, 256, fake, 512, fake, None, fake, 512, 1, None) == nat.GK_UNSUPPORTED_LAYER_CONFIGURATION
    assert f(None, 256, 4, 256, fake, 512, fake, None, fake, 512, 0, None) == nat.GK_INVALID_ARGUMENT


def test_codec_rejects_before_device_use():
    lib = nat.load()
    fake = ctypes.c_void_p(1 << 20)
    rounded = ctypes.c_int64(0)
    assert lib.gk_fp8_codec_ocp_to_half(fake, fake, 0, fake, fake, 1, ctypes.byref(rounded), fake, 256,
                                        None) == nat.GK_INCOMPATIBLE_INPUT_SIZE
    assert lib.gk_fp8_codec_ocp_to_half(fake, fake, 16, fake, fake, 1, ctypes.byref(rounded), fake, 8,
                                        None) == nat.GK_INSUFFICIENT_BUFFER
    ws = ctypes.c_size_t(0)
    assert lib.gk_fp8_codec_workspace_bytes(ctypes.byref(ws)) == nat.GK_SUCCESS and ws.value >= 16


def test_no_gpu_means_loud_failure():
    import torch
    if torch.cuda.is_available():
        pytest.skip("GPU present")
    with pytest.raises(RuntimeError):
        ops.require_device()


def test_token_channel_fusion_rule():
    from gaudi_kernels import ops
    assert ops.token_channel_fused_pays(1, 6144, 4096) and ops.token_channel_fused_pays(4, 4096, 14336)
    assert not ops.token_channel_fused_pays(8, 6144, 4096)  # M > 4: the redundant quantizer work dominates
    assert not ops.token_channel_fused_pays(1, 28672, 4096)  # 896 workgroups each reading x twice
