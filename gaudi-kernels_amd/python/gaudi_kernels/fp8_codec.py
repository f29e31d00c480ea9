"""Load-time conversion from OCP E4M3FN to Gaudi2 E4M3 half range, on the GPU.

Same call signature, return values and errors as the reference's
python/gaudi_kernels/fp8_codec.py:14-53 (``reencode_e4m3fn_half``), executed
by the gfx950 codec kernel of libgk_fp8.so.  The returned bytes are Gaudi2
half-range bit patterns viewed as torch.float8_e4m3fn storage; each holds the
input value halved, rounded to nearest even on the 2^-9 grid, and the scales
are doubled so that code * scale is preserved except for the rounded codes.

Tensors may live on the CPU (as in the reference; they are staged to the
current GPU and the results returned on the CPU) or on a ROCm device (results
stay there).  ``decode_half_to_ocp`` is the inverse conversion.
"""

import torch

from gaudi_kernels import _native as nat
from gaudi_kernels import ops

ERR_WEIGHT = "expected a nonempty contiguous CPU E4M3FN weight"
ERR_SCALES = "expected nonempty contiguous finite nonnegative CPU FP32 scales"
ERR_OVERFLOW = "doubling FP8 scales overflows FP32"
ERR_NAN = "nonfinite OCP E4M3FN checkpoint code"
ERR_HALF = "half-range E4M3 code has no OCP E4M3FN image"
ERR_INEXACT = "halving FP8 scales is inexact"


def _placed(t):
    return t.device.type in ("cpu", "cuda")


def _validate(weight, scales):
    # fp8_codec.py:21-29, in the same order; finiteness and sign of the scales
    # are checked by the kernel (status word) to avoid a host round trip.
    if (not isinstance(weight, torch.Tensor) or not _placed(weight)
            or weight.dtype != torch.float8_e4m3fn or not weight.is_contiguous()
            or not weight.numel() or weight.requires_grad):
        raise ValueError(ERR_WEIGHT)
    if (not isinstance(scales, torch.Tensor) or not _placed(scales)
            or scales.dtype != torch.float32 or not scales.is_contiguous()
            or not scales.numel() or scales.requires_grad):
        raise ValueError(ERR_SCALES)


def _to_device(weight, scales):
    device = ops.require_device(weight.device if weight.is_cuda else scales.device if scales.is_cuda else None)
    return weight.detach().to(device), scales.detach().to(device), device


def reencode_e4m3fn_half(weight, scales):
    """Return (encoded bytes, doubled FP32 scales, rounded element count).

    Inputs must be contiguous; neither is modified.  Nonfinite checkpoint
    codes and negative, nonfinite or overflowing scales raise ValueError.  The
    shape of each tensor is preserved; layout packing is a separate step.
    """
    _validate(weight, scales)
    w_dev, s_dev, _ = _to_device(weight, scales)
    try:
        codes, s2, rounded = ops.codec_ocp_to_half(w_dev, s_dev)
    except nat.GkError as e:
        msg = {nat.GK_INVALID_SCALE: ERR_SCALES, nat.GK_SCALE_OVERFLOW: ERR_OVERFLOW,
               nat.GK_NONFINITE_CODE: ERR_NAN}.get(e.status)
        if msg is None:
            raise
        raise ValueError(msg) from None
    encoded = codes.view(torch.float8_e4m3fn).reshape(weight.shape)
    s2 = s2.reshape(scales.shape)
    if not weight.is_cuda:
        encoded, s2 = encoded.cpu(), s2.cpu()
    return encoded, s2.contiguous(), rounded


def decode_half_to_ocp(weight, scales):
    """Inverse of reencode_e4m3fn_half: half-range codes -> OCP E4M3FN (value x2, exact), scales / 2.

    Magnitudes 0x77..0x7f (240 and the Gaudi2 specials) have no OCP image at
    twice the value and raise ValueError, as do negative or nonfinite scales
    and scales whose half is an inexact fp32 subnormal.
    """
    _validate(weight, scales)
    w_dev, s_dev, _ = _to_device(weight, scales)
    try:
        codes, s_half = ops.codec_half_to_ocp(w_dev, s_dev)
    except nat.GkError as e:
        msg = {nat.GK_INVALID_SCALE: ERR_SCALES, nat.GK_NONFINITE_CODE: ERR_HALF,
               nat.GK_INEXACT_SCALE: ERR_INEXACT}.get(e.status)
        if msg is None:
            raise
        raise ValueError(msg) from None
    decoded = codes.view(torch.float8_e4m3fn).reshape(weight.shape)
    s_half = s_half.reshape(scales.shape)
    if not weight.is_cuda:
        decoded, s_half = decoded.cpu(), s_half.cpu()
    return decoded, s_half.contiguous()
