"""ctypes binding of libgk_fp8.so (C ABI declared in include/gk_fp8.h).

The library is loaded once per process.  There is no CPU fallback: if the
shared object is missing, or no gfx950 GPU is present, every GPU entry point
raises RuntimeError.
"""

import ctypes
import os
import threading

_LIB_NAME = "libgk_fp8.so"
_lock = threading.Lock()
_lib = None

# gk_status (include/gk_fp8.h)
GK_SUCCESS = 0
GK_INCOMPATIBLE_INPUT_SIZE = 1
GK_INCOMPATIBLE_OUTPUT_SIZE = 2
GK_INCOMPATIBLE_DATA_TYPE = 3
GK_UNSUPPORTED_LAYER_CONFIGURATION = 4
GK_INSUFFICIENT_BUFFER = 5
GK_NODE_NOT_FOUND = 6
GK_INVALID_ARGUMENT = 7
GK_NONFINITE_CODE = 8
GK_INVALID_SCALE = 9
GK_SCALE_OVERFLOW = 10
GK_INEXACT_SCALE = 11
GK_NONFINITE_INPUT = 12
GK_UNSUPPORTED_DEVICE = 13
GK_DEVICE_ERROR = 14

STATUS_NAMES = {
    0: "GK_SUCCESS", 1: "GK_INCOMPATIBLE_INPUT_SIZE", 2: "GK_INCOMPATIBLE_OUTPUT_SIZE",
    3: "GK_INCOMPATIBLE_DATA_TYPE", 4: "GK_UNSUPPORTED_LAYER_CONFIGURATION", 5: "GK_INSUFFICIENT_BUFFER",
    6: "GK_NODE_NOT_FOUND", 7: "GK_INVALID_ARGUMENT", 8: "GK_NONFINITE_CODE", 9: "GK_INVALID_SCALE",
    10: "GK_SCALE_OVERFLOW", 11: "GK_INEXACT_SCALE", 12: "GK_NONFINITE_INPUT", 13: "GK_UNSUPPORTED_DEVICE",
    14: "GK_DEVICE_ERROR",
}

GK_FLAG_NATIVE_HALF = 1
GK_FLAG_FORCE_DECODE = 2
GK_FLAG_FORCE_PREFILL = 4
GK_FLAG_FORCE_GENERIC = 8
GK_FLAG_DECODE_LAYOUT = 16
GK_FLAG_WEIGHT_PACKED = 32
GK_FLAG_ACCUMULATE = 64

GK_VARIANT_DECODE = 1
GK_VARIANT_PREFILL = 2
GK_VARIANT_GENERIC = 3

_c_i64 = ctypes.c_int64
_c_u32 = ctypes.c_uint32
_c_size = ctypes.c_size_t
_c_vp = ctypes.c_void_p
_c_int = ctypes.c_int
_fp = ctypes.c_void_p  # float* passed as address

# name -> (restype, argtypes); must match include/gk_fp8.h
SIGNATURES = {
    "gk_lib_version": (ctypes.c_uint64, []),
    "gk_list_ops": (_c_int, [ctypes.POINTER(_c_u32), ctypes.POINTER(ctypes.c_char_p)]),
    "gk_device_supported": (_c_int, [_c_int]),
    "gk_fp8_codec_workspace_bytes": (_c_int, [ctypes.POINTER(_c_size)]),
    "gk_fp8_codec_ocp_to_half": (_c_int, [_c_vp, _c_vp, _c_i64, _fp, _fp, _c_i64, ctypes.POINTER(_c_i64),
                                          _c_vp, _c_size, _c_vp]),
    "gk_fp8_codec_half_to_ocp": (_c_int, [_c_vp, _c_vp, _c_i64, _fp, _fp, _c_i64, _c_vp, _c_size, _c_vp]),
    "gk_fp8_packed_weight_bytes": (_c_int, [_c_i64, _c_i64, ctypes.POINTER(_c_size)]),
    "gk_fp8_pack_weight": (_c_int, [_c_vp, _c_i64, _c_i64, _c_vp, _c_size, _c_vp]),
    "gk_fp8_pack_experts": (_c_int, [_c_vp, _c_i64, _c_i64, _c_i64, _c_vp, _c_size, _c_vp]),
    "gk_fp8_act_quant_bf16": (_c_int, [_c_vp, _c_i64, _c_i64, _c_i64, _c_vp, _fp, _c_i64, _c_u32, _c_vp]),
    "gk_fp8_block_gemm_plan": (_c_int, [_c_i64, _c_i64, _c_i64, _c_u32, _c_vp, ctypes.POINTER(_c_int),
                                        ctypes.POINTER(_c_i64), ctypes.POINTER(_c_size)]),
    "gk_fp8_block_gemm_bf16": (_c_int, [_c_vp, _c_i64, _c_i64, _c_i64, _c_vp, _c_i64, _fp, _c_i64, _c_i64, _fp,
                                        _c_vp, _c_i64, _c_u32, _c_vp, _c_size, _c_vp]),
    "gk_fp8_block_gemm_bf16_noalloc": (_c_int, [_c_vp, _c_i64, _c_i64, _c_i64, _c_vp, _c_i64, _fp, _c_i64, _c_i64,
                                                _fp, _c_vp, _c_i64, _c_u32, _c_vp]),
    "gk_fp8_block_gemm_q_bf16": (_c_int, [_c_vp, _fp, _c_i64, _c_i64, _c_i64, _c_vp, _c_i64, _fp, _c_i64, _c_i64,
                                          _fp, _c_vp, _c_i64, _c_u32, _c_vp]),
    "gk_fp8_block_gemm_kslice_f32": (_c_int, [_c_vp, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_vp, _c_i64, _fp,
                                              _c_i64, _c_i64, _fp, _c_i64, _c_u32, _c_vp, _c_size, _c_vp]),
    "gk_fp8_partial_finish_bf16": (_c_int, [_fp, _c_i64, _c_i64, _c_i64, _fp, _c_vp, _c_i64, _c_vp]),
    "gk_rank_sum_f32": (_c_int, [_fp, _c_i64, _c_int, _fp, _c_i64, _c_vp]),
    "gk_rank_sum_bf16": (_c_int, [_c_vp, _c_i64, _c_int, _c_vp, _c_i64, _c_vp]),
    "gk_rank_sum_infer": (_c_int, [_c_i64, _c_int, ctypes.POINTER(_c_i64)]),
    "gk_fp8_check_inputs": (_c_int, [_c_vp, _c_i64, _c_i64, _c_i64, _c_vp, _c_i64, _fp, _c_i64, _c_vp, _c_size,
                                     _c_vp]),
    "gk_fp8_token_quant_bf16": (_c_int, [_c_vp, _c_i64, _c_i64, _c_i64, _c_vp, _c_i64, _fp, _c_vp]),
    "gk_fp8_channel_finish_bf16": (_c_int, [_fp, _c_i64, _c_i64, _c_i64, _fp, _fp, _fp, _c_vp, _c_i64, _c_vp]),
    "gk_fp8_channel_gemm_bf16": (_c_int, [_c_vp, _c_i64, _fp, _c_i64, _c_i64, _c_vp, _c_i64, _fp, _fp, _c_vp,
                                          _c_i64, _c_u32, _c_vp]),
    "gk_fp8_token_channel_gemm_bf16": (_c_int, [_c_vp, _c_i64, _c_i64, _c_i64, _c_vp, _c_i64, _fp, _fp, _c_vp,
                                                _c_i64, _c_u32, _c_vp]),
    "gk_silu_and_mul_bf16": (_c_int, [_c_vp, _c_i64, _c_i64, _c_i64, _c_vp, _c_i64, _c_vp]),
    "gk_fp8_silu_mul_quant_bf16": (_c_int, [_c_vp, _c_i64, _c_i64, _c_i64, _c_vp, _fp, _c_i64, _c_u32, _c_vp]),
    "gk_gelu_and_mul_bf16": (_c_int, [_c_vp, _c_i64, _c_i64, _c_i64, _c_vp, _c_i64, _c_int, _c_vp]),
    "gk_fp8_gelu_mul_quant_bf16": (_c_int, [_c_vp, _c_i64, _c_i64, _c_i64, _c_int, _c_vp, _fp, _c_i64, _c_u32,
                                            _c_vp]),
    "gk_rms_norm_bf16": (_c_int, [_c_vp, _c_i64, _c_i64, _c_i64, _c_vp, ctypes.c_float, ctypes.c_float, _c_vp,
                                  _c_i64, _c_vp]),
    "gk_fused_add_rms_norm_bf16": (_c_int, [_c_vp, _c_vp, _c_i64, _c_i64, _c_i64, _c_vp, ctypes.c_float,
                                            ctypes.c_float, _c_vp, _c_vp, _c_i64, _c_vp]),
    "gk_fp8_rms_norm_quant_bf16": (_c_int, [_c_vp, _c_vp, _c_i64, _c_i64, _c_i64, _c_vp, ctypes.c_float,
                                            ctypes.c_float, _c_vp, _c_i64, _c_vp, _fp, _c_i64, _c_u32, _c_vp]),
    "gk_fp8_moe_rows_max": (_c_int, [_c_i64, _c_i64, _c_int, ctypes.POINTER(_c_i64)]),
    "gk_fp8_moe_workspace_bytes": (_c_int, [_c_i64, _c_i64, _c_i64, _c_i64, _c_int, ctypes.POINTER(_c_size)]),
    "gk_fp8_moe_route": (_c_int, [_fp, _c_i64, _c_i64, _c_i64, _c_int, _c_vp, _fp, _c_vp, _c_vp, _c_i64, _c_vp,
                                  _c_vp]),
    "gk_fp8_moe_bf16": (_c_int, [_c_vp, _c_i64, _c_i64, _c_i64, _fp, _c_i64, _c_i64, _c_int, _c_vp, _fp, _c_i64,
                                 _c_vp, _fp, _c_vp, _c_i64, _c_u32, _c_vp, _c_size, _c_vp]),
}


def lib_path():
    return os.path.join(os.path.dirname(os.path.abspath(__file__)), _LIB_NAME)


def load():
    """Load libgk_fp8.so (once) and bind every entry point; raises if it is not built."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is None:
            path = lib_path()
            if not os.path.exists(path):
                raise RuntimeError(f"gaudi_kernels: {path} is not built (run gaudi-kernels_amd/build.py)")
            lib = ctypes.CDLL(path, mode=ctypes.RTLD_LOCAL)
            for name, (res, args) in SIGNATURES.items():
                fn = getattr(lib, name)
                fn.restype = res
                fn.argtypes = args
            _lib = lib
    return _lib


class GkError(RuntimeError):
    def __init__(self, fn, status):
        self.status = status
        super().__init__(f"{fn} failed: {STATUS_NAMES.get(status, status)}")


def check(fn, status):
    if status != GK_SUCCESS:
        raise GkError(fn, status)


def list_ops():
    lib = load()
    count = _c_u32(0)
    check("gk_list_ops", lib.gk_list_ops(ctypes.byref(count), None))
    names = (ctypes.c_char_p * count.value)()
    cap = _c_u32(count.value)
    check("gk_list_ops", lib.gk_list_ops(ctypes.byref(cap), names))
    return [n.decode() for n in names]
