"""CPU oracle for the block-FP8 path -- TEST INFRASTRUCTURE ONLY.

This package restates, on the CPU, the reference algorithm of
``tracycam/gaudi-kernels`` for the block-FP8 W8A8 GEMM and the E4M3 codec.
It is the checker the GPU product is compared against.  Only ``tests/``,
``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of ``bench.py`` may
import it, and only as the checker or the timed CPU baseline: the product
(``gaudi-kernels_amd``) never imports, links or executes anything here.

Modules
-------
``e4m3``        independent OCP E4M3FN encode/decode (bit arithmetic, numpy)
``fp8_codec``   restatement of python/gaudi_kernels/fp8_codec.py:14-53 plus the
                build-defined inverse (half range -> OCP)
``block_fp8``   restatement of python/gaudi_kernels/block_fp8_oracle.py:11-46,
                extended from M=1 to M>=1 (rows are independent)
``moe``         build-defined MoE routing / gather / scatter restatement
``synth``       seeded synthetic inputs shared by tests and bench

How each function is pinned (checked against something other than itself) is
written in its docstring; see tests/test_oracle_*.py for the checks.
"""
