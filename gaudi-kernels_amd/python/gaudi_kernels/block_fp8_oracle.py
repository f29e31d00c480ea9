"""Block-FP8 W8A8 linear with the reference oracle's numerics, executed on the GPU.

Same call signature and errors as python/gaudi_kernels/block_fp8_oracle.py:11-46
of the reference, ``reference(x, weight, scales, *, native_half=False,
bias=None)``, backed by the gfx950 kernels of libgk_fp8.so:

  * activations are quantized per row and 128-column group exactly as the
    reference does (sa = fp32(max(amax, 1e-10)) * fp32(1/448), IEEE divide,
    clamp to +-448, E4M3 round to nearest even) -- bit-identical codes/scales;
  * each 128-K group's fp8 x fp8 dot products are formed by FP8 MFMA and the
    group's original block scales are applied to that group's partial
    (fp32 accumulation), plus bias, rounded to bf16;
  * native_half applies the half-range adaptation of the reference (:31-35):
    activation and weight codes halved with RNE, scales doubled.

Unlike the reference, any M >= 1 is accepted and tensors may be on a ROCm
device (the result stays there) or on the CPU (staged to the current GPU,
the result returned on the CPU).  The output matches the fp64 reference to
max|err| <= 1e-2 * max|ref| and sum|err| / sum|ref| <= 2e-3.
"""

import torch

from gaudi_kernels import ops

ERR_INPUTS = "CPU M1 BF16 activation, original OCP FP8 weight and FP32 scales required"
ERR_GRID = "original block128 scale grid mismatch"
ERR_FINITE = "finite original inputs required"
ERR_BIAS = "CPU bias with N elements required"


def reference(x, weight, scales, *, native_half=False, bias=None):
    placed = all(isinstance(t, torch.Tensor) and t.device.type in ("cpu", "cuda") for t in (x, weight, scales))
    if (not placed or x.dtype != torch.bfloat16 or weight.dtype != torch.float8_e4m3fn
            or scales.dtype != torch.float32 or x.ndim != 2 or weight.ndim != 2
            or x.shape[0] < 1 or x.shape[1] != weight.shape[1]):
        raise ValueError(ERR_INPUTS)
    n, k = weight.shape
    groups = (k + 127) // 128
    if tuple(scales.shape) != ((n + 127) // 128, groups):
        raise ValueError(ERR_GRID)
    on_gpu = x.is_cuda
    device = ops.require_device(x.device if x.is_cuda else weight.device if weight.is_cuda else None)
    xd = x.to(device).contiguous()
    wd = weight.to(device).contiguous()
    sd = scales.to(device).contiguous()
    if not ops.inputs_finite(xd, wd, sd):
        raise ValueError(ERR_FINITE)
    bd = None
    if bias is not None:
        if not isinstance(bias, torch.Tensor) or bias.numel() != n or bias.device.type not in ("cpu", "cuda"):
            raise ValueError(ERR_BIAS)
        bd = bias.reshape(-1).to(device=device, dtype=torch.float32).contiguous()
    y = ops.block_fp8_gemm(xd, wd, sd, bd, native_half=native_half)
    return y if on_gpu else y.cpu()
