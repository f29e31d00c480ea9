"""MI355X (gfx950) block-FP8 W8A8 GEMM and load-time E4M3 codec.

Drop-in for the block-FP8 path of tracycam/gaudi-kernels: the module paths
``gaudi_kernels.fp8_codec`` (reencode_e4m3fn_half) and
``gaudi_kernels.block_fp8_oracle`` (reference) keep the reference's call
signatures and errors (python/gaudi_kernels/__init__.py:3-5 exports the
codec), now executed by hand-written gfx950 kernels in libgk_fp8.so.
``gaudi_kernels.ops`` holds the asynchronous device-side operations.
"""

from gaudi_kernels.fp8_codec import decode_half_to_ocp, reencode_e4m3fn_half

__all__ = ["reencode_e4m3fn_half", "decode_half_to_ocp"]
