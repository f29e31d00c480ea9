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
    # the MoE layer's packed-expert layout changed: the op is v2, beside its packing op
    assert "gk_fp8_moe_bf16_v2" in names and "gk_fp8_moe_bf16_v1" not in names
    assert "gk_fp8_pack_experts_v1" in names
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


def test_alignment_rejections_before_device_use():
    lib = nat.load()
    fake = ctypes.c_void_p(1 << 20)
    ws = ctypes.c_void_p(1 << 21)
    odd4 = ctypes.c_void_p((1 << 20) + 2)  # 2-byte aligned: not an fp32 buffer
    odd2 = ctypes.c_void_p((1 << 20) + 1)
    # a misaligned fp32 bias, as the channel GEMM and channel finish reject it
    st = lib.gk_fp8_block_gemm_bf16(fake, 4, 256, 256, fake, 512, fake, 4, 2, odd4, fake, 512, 0, ws, 1 << 20, None)
    assert st == nat.GK_INCOMPATIBLE_DATA_TYPE
    st = lib.gk_fp8_block_gemm_q_bf16(fake, fake, 4, 16, 256, fake, 512, fake, 4, 2, odd4, fake, 512, 0, None)
    assert st == nat.GK_INCOMPATIBLE_DATA_TYPE
    # the finite-input check: bf16 x, fp32 scales, the status workspace
    f = lib.gk_fp8_check_inputs
    assert f(odd2, 4, 256, 256, fake, 512, fake, 8, ws, 256, None) == nat.GK_INCOMPATIBLE_DATA_TYPE
    assert f(fake, 4, 256, 256, fake, 512, odd4, 8, ws, 256, None) == nat.GK_INCOMPATIBLE_DATA_TYPE
    assert f(fake, 4, 256, 256, fake, 512, fake, 8, ctypes.c_void_p((1 << 21) + 4), 256,
             None) == nat.GK_INCOMPATIBLE_DATA_TYPE


def test_moe_route_rejections_before_device_use():
    lib = nat.load()
    fake = ctypes.c_void_p(1 << 20)
    rows = ctypes.c_int64(0)
    assert lib.gk_fp8_moe_rows_max(512, 8, 2, ctypes.byref(rows)) == nat.GK_SUCCESS
    f = lib.gk_fp8_moe_route
    # logits, T, E, ld, k, ids, wts, row_of, row_token, rows_max, offsets, stream
    assert f(fake, 512, 8, 8, 2, fake, fake, fake, fake, rows.value - 1, fake, None) == nat.GK_INSUFFICIENT_BUFFER
    assert f(fake, 512, 8, 8, 2, fake, fake, fake, fake, 1 << 40, fake, None) == nat.GK_INCOMPATIBLE_OUTPUT_SIZE
    assert f(fake, 512, 8, 8, 2, fake, fake, fake, ctypes.c_void_p((1 << 20) + 2), rows.value, fake,
             None) == nat.GK_INCOMPATIBLE_DATA_TYPE


@pytest.mark.parametrize("t,h,inter,e,k", [(512, 4096, 14336, 8, 2), (3, 384, 128, 8, 2), (300, 256, 128, 3, 1),
                                           (4500, 11008, 128, 9, 2), (1, 128, 128, 256, 1)])
def test_moe_workspace_is_the_documented_regions(t, h, inter, e, k):
    """gk_fp8_moe_workspace_bytes = the regions include/gk_fp8.h lists for gk_fp8_moe_bf16, in order, each
    from a 256-byte boundary (no bf16 gate_up region: its epilogue writes the SiLU-and-mul codes)."""
    lib = nat.load()
    rows, nbytes = ctypes.c_int64(0), ctypes.c_size_t(0)
    assert lib.gk_fp8_moe_rows_max(t, e, k, ctypes.byref(rows)) == nat.GK_SUCCESS
    r = rows.value
    assert r == (t * k + 255 * e + 255) // 256 * 256
    parts = 2 if (r // 256) * ((h + 255) // 256) < 512 else 1
    sizes = [t * k * 4, t * k * 4, t * k * 4, r * 4, (e + 1) * 4, e * 4, r * h, r * h // 128 * 4, r * inter,
             r * inter // 128 * 4, parts * r * h * 4]
    assert lib.gk_fp8_moe_workspace_bytes(t, h, inter, e, k, ctypes.byref(nbytes)) == nat.GK_SUCCESS
    assert nbytes.value == sum((n + 255) // 256 * 256 for n in sizes)


def test_moe_workspace_rejects_bad_shapes():
    lib = nat.load()
    nbytes = ctypes.c_size_t(0)
    f = lambda *a: lib.gk_fp8_moe_workspace_bytes(*a, ctypes.byref(nbytes))
    assert f(512, 4000, 14336, 8, 2) == nat.GK_INCOMPATIBLE_INPUT_SIZE    # H not a multiple of 128
    assert f(512, 4096, 14300, 8, 2) == nat.GK_INCOMPATIBLE_INPUT_SIZE    # I not a multiple of 128
    assert f(512, 4096, 14336, 257, 2) == nat.GK_INCOMPATIBLE_INPUT_SIZE  # more than 256 experts
    assert f(512, 4096, 14336, 8, 3) == nat.GK_INCOMPATIBLE_INPUT_SIZE    # top_k > 2
    assert f(0, 4096, 14336, 8, 2) == nat.GK_INCOMPATIBLE_INPUT_SIZE      # no tokens
    assert lib.gk_fp8_moe_workspace_bytes(512, 4096, 14336, 8, 2, None) == nat.GK_INVALID_ARGUMENT


def test_rank_sum_rejections_before_device_use():
    """generic_dense_glue_contract_test.cpp:533-584 and the glue's checks (generic_dense_glue.cpp:568-600, 871-895)."""
    lib = nat.load()
    fake = ctypes.c_void_p(1 << 20)
    elems = ctypes.c_int64(0)
    assert lib.gk_rank_sum_infer(16384, 4, ctypes.byref(elems)) == nat.GK_SUCCESS and elems.value == 4096
    for bad in (1, 9):
        assert lib.gk_rank_sum_infer(16384, bad, ctypes.byref(elems)) == nat.GK_UNSUPPORTED_LAYER_CONFIGURATION
    assert lib.gk_rank_sum_infer(3, 4, ctypes.byref(elems)) == nat.GK_INCOMPATIBLE_INPUT_SIZE
    assert lib.gk_rank_sum_infer(10, 4, ctypes.byref(elems)) == nat.GK_INCOMPATIBLE_INPUT_SIZE
    for fn in (lib.gk_rank_sum_f32, lib.gk_rank_sum_bf16):
        assert fn(fake, 16384, 1, fake, 4096, None) == nat.GK_UNSUPPORTED_LAYER_CONFIGURATION
        assert fn(fake, 16384, 9, fake, 4096, None) == nat.GK_UNSUPPORTED_LAYER_CONFIGURATION
        assert fn(fake, 8192, 4, fake, 4096, None) == nat.GK_INCOMPATIBLE_INPUT_SIZE   # mismatched gathered size
        assert fn(fake, 0, 4, fake, 0, None) == nat.GK_INCOMPATIBLE_OUTPUT_SIZE
        assert fn(fake, 4 << 30, 4, fake, 1 << 30, None) == nat.GK_INCOMPATIBLE_OUTPUT_SIZE  # beyond int32
        assert fn(None, 16384, 4, fake, 4096, None) == nat.GK_INVALID_ARGUMENT
    assert lib.gk_rank_sum_f32(ctypes.c_void_p((1 << 20) + 2), 16384, 4, fake, 4096,
                               None) == nat.GK_INCOMPATIBLE_DATA_TYPE
    assert lib.gk_rank_sum_bf16(ctypes.c_void_p((1 << 20) + 1), 16384, 4, fake, 4096,
                                None) == nat.GK_INCOMPATIBLE_DATA_TYPE


def test_kslice_col_offset_rules_before_device_use():
    """The col_offset contract of generic_fp8_glue.hpp:169-176, :245-252 and generic_fp8_glue_test.cpp:196-220."""
    lib = nat.load()
    fake = ctypes.c_void_p(1 << 20)
    ws = ctypes.c_void_p(1 << 21)
    f = lib.gk_fp8_block_gemm_kslice_f32
    # x, m, k, ldx, k_offset, k_len, w, n, scales, rows, cols, partial, ldp, flags, ws, ws_bytes, stream

    def call(k_offset, k_len, k=512, flags=0, ldp=256, ws_bytes=1 << 20, rows=2, cols=None):
        return f(fake, 4, k, k, k_offset, k_len, fake, 256, fake, rows, k // 128 if cols is None else cols, fake, ldp,
                 flags, ws, ws_bytes, None)

    # offset 384 + 256 > 512: rejected as an input size (generic_fp8_glue_test.cpp:216-218)
    assert call(384, 256) == nat.GK_INCOMPATIBLE_INPUT_SIZE
    assert call(100, 256) == nat.GK_UNSUPPORTED_LAYER_CONFIGURATION     # not a multiple of 128
    assert call(-128, 256) == nat.GK_UNSUPPORTED_LAYER_CONFIGURATION
    assert call(0, 0) == nat.GK_INCOMPATIBLE_INPUT_SIZE
    assert call(0, 200) == nat.GK_INCOMPATIBLE_INPUT_SIZE
    assert call(0, 256, k=500) == nat.GK_INCOMPATIBLE_INPUT_SIZE         # K itself a multiple of 128
    assert call(256, 256, cols=2) == nat.GK_INCOMPATIBLE_INPUT_SIZE      # the whole-K scale grid
    assert call(256, 256, ldp=100) == nat.GK_INCOMPATIBLE_OUTPUT_SIZE
    assert call(256, 256, ws_bytes=16) == nat.GK_INSUFFICIENT_BUFFER
    assert call(256, 256, flags=nat.GK_FLAG_FORCE_GENERIC) == nat.GK_UNSUPPORTED_LAYER_CONFIGURATION
    assert f(fake, 4, 512, 512, 256, 256, fake, 256, fake, 2, 4, ctypes.c_void_p((1 << 20) + 2), 256, 0, ws, 1 << 20,
             None) == nat.GK_INCOMPATIBLE_DATA_TYPE


def test_partial_finish_rejections_before_device_use():
    lib = nat.load()
    fake = ctypes.c_void_p(1 << 20)
    f = lib.gk_fp8_partial_finish_bf16
    assert f(fake, 0, 16, 16, None, fake, 16, None) == nat.GK_INCOMPATIBLE_INPUT_SIZE
    assert f(fake, 2, 16, 8, None, fake, 16, None) == nat.GK_INCOMPATIBLE_INPUT_SIZE
    assert f(fake, 2, 16, 16, None, fake, 8, None) == nat.GK_INCOMPATIBLE_OUTPUT_SIZE
    assert f(fake, 2, 16, 16, ctypes.c_void_p((1 << 20) + 2), fake, 16, None) == nat.GK_INCOMPATIBLE_DATA_TYPE
    assert f(None, 2, 16, 16, None, fake, 16, None) == nat.GK_INVALID_ARGUMENT


def test_probe_library_exports_match_its_header():
    """tests/csrc/libgk_probe.so (bench.py's streaming-read ceiling, the hardware conversion checks; not part of
    the library) exports exactly what tests/csrc/gk_probe.h declares."""
    probe = os.path.join(ROOT, "tests", "csrc", "libgk_probe.so")
    if not os.path.exists(probe):
        pytest.skip("libgk_probe.so not built")
    text = open(os.path.join(ROOT, "tests", "csrc", "gk_probe.h")).read()
    want = sorted(set(re.findall(r"^\s*int\s+(gk_\w+)\s*\(", text, re.MULTILINE)))
    out = subprocess.run(["nm", "-D", "--defined-only", probe], check=True, capture_output=True, text=True).stdout
    have = sorted({l.split()[-1] for l in out.splitlines() if " T " in l and l.split()[-1].startswith("gk_")})
    assert have == want == ["gk_probe_bf16x2_check", "gk_probe_e4m3_check", "gk_probe_stream_read"]
    lib = ctypes.CDLL(probe)
    lib.gk_probe_stream_read.restype = ctypes.c_int
    lib.gk_probe_stream_read.argtypes = [ctypes.c_void_p, ctypes.c_size_t, ctypes.c_void_p, ctypes.c_int,
                                         ctypes.c_void_p]
    assert lib.gk_probe_stream_read(ctypes.c_void_p(1 << 20), 17, ctypes.c_void_p(1 << 20), 256, None) == 1
    lib.gk_probe_bf16x2_check.restype = ctypes.c_int
    lib.gk_probe_bf16x2_check.argtypes = [ctypes.c_void_p, ctypes.c_void_p]
    assert lib.gk_probe_bf16x2_check(None, None) == 1
    assert lib.gk_probe_bf16x2_check(ctypes.c_void_p((1 << 20) + 4), None) == 1
    lib.gk_probe_e4m3_check.restype = ctypes.c_int
    lib.gk_probe_e4m3_check.argtypes = [ctypes.c_void_p, ctypes.c_void_p]
    assert lib.gk_probe_e4m3_check(None, None) == 1


def test_noalloc_rejects_beyond_scratch():
    """gk_fp8_block_gemm_bf16_noalloc checks its plan against GK_NOALLOC_SCRATCH_BYTES before any device work:
    a plan needing more scratch returns GK_INSUFFICIENT_BUFFER (fake pointers are never touched; host-only test)."""
    lib = nat.load()
    m, n, k = 8192, 7168, 7168          # 8192 x 56 groups x 132 B > 32 MiB of scratch
    _, _, need = ops.plan(m, n, k)
    assert need > (32 << 20)
    fake = ctypes.c_void_p(1 << 20)
    st = lib.gk_fp8_block_gemm_bf16_noalloc(fake, m, k, k, fake, n, fake, 56, 56, None, fake, n, 0, None)
    assert st == nat.GK_INSUFFICIENT_BUFFER
