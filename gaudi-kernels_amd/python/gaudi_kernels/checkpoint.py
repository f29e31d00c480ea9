"""Checkpoint load path: block-FP8 safetensors weights to persistent device weights.

The checkpoint convention of the block-FP8 path: a linear weight ``<name>.weight``
stored as OCP E4M3FN codes [N, K] next to its fp32 128x128 block-scale grid
``<name>.weight_scale_inv`` [ceil(N/128), ceil(K/128)] (the factor applied to the
codes, code * scale ~ weight -- the ``scales`` argument of
``block_fp8_oracle.reference``, python/gaudi_kernels/block_fp8_oracle.py:11-24).

On MI355X the FP8 MFMA consumes OCP codes directly, so the load path copies codes
and scales to the GPU unchanged and checks them there (no NaN code, finite
nonnegative scales, gk_fp8_check_inputs); the GEMM's ``native_half`` mode applies
the half-range codec in-kernel.  Two options convert at load time on the GPU with
the codec kernels:
  * ``to_half_range=True``: the Gaudi2 half-range bytes and doubled scales of
    python/gaudi_kernels/fp8_codec.py:14-53 (for exchange with a Gaudi2 pipeline);
  * ``from_half_range=True``: a checkpoint already stored in half range is
    brought back to OCP codes (the exact inverse).
Files are read with safetensors (no pickle); tensors are copied one at a time, so
host memory holds at most one tensor beyond the memory map.
"""

from typing import NamedTuple

import torch

from gaudi_kernels import ops

SCALE_SUFFIX = "_scale_inv"


class BlockFP8Weight(NamedTuple):
    codes: torch.Tensor       # device float8_e4m3fn [N, K]
    scales: torch.Tensor      # device float32 [ceil(N/128), ceil(K/128)]
    half_range: bool          # codes are Gaudi2 half-range bytes (scales doubled)
    rounded: int              # codes rounded by the conversion to half range (0 otherwise)


def pair_block_fp8(keys, dtypes):
    """Split checkpoint keys into block-FP8 (weight, scale) pairs and other tensors.

    keys: iterable of tensor names; dtypes: name -> torch dtype.  A weight is an
    float8_e4m3fn tensor whose ``<name>_scale_inv`` companion exists.  Returns
    (pairs {weight_name: scale_name}, others [names]); raises ValueError for an
    fp8 tensor without a scale grid or a scale grid without its weight.
    """
    keys = list(keys)
    keyset = set(keys)
    pairs, others = {}, []
    for k in keys:
        if k.endswith(SCALE_SUFFIX):
            base = k[: -len(SCALE_SUFFIX)]
            if base not in keyset or dtypes[base] != torch.float8_e4m3fn:
                raise ValueError(f"{k}: block-scale grid without an E4M3FN weight {base}")
            continue
        if dtypes[k] == torch.float8_e4m3fn:
            s = k + SCALE_SUFFIX
            if s not in keyset:
                raise ValueError(f"{k}: E4M3FN weight without its block-scale grid {s}")
            pairs[k] = s
        else:
            others.append(k)
    return pairs, others


def _check_grid(name, w, s):
    n, k = w.shape if w.ndim == 2 else (None, None)
    if w.ndim != 2 or s.dtype != torch.float32 or tuple(s.shape) != ((n + 127) // 128, (k + 127) // 128):
        raise ValueError(f"{name}: original block128 scale grid mismatch")


def load_block_fp8(path, device=None, *, names=None, validate=True, to_half_range=False, from_half_range=False):
    """Load a safetensors checkpoint onto the GPU.

    Returns (weights {name: BlockFP8Weight}, tensors {name: device tensor}) for the
    block-FP8 pairs and for every other tensor.  names: optional subset of weight
    or tensor names to load.  validate: reject NaN codes and negative/nonfinite
    scales (ValueError) with one GPU check per weight.
    """
    from safetensors import safe_open

    if to_half_range and from_half_range:
        raise ValueError("to_half_range and from_half_range are exclusive")
    device = ops.require_device(device)
    weights, tensors = {}, {}
    with safe_open(str(path), framework="pt", device="cpu") as f:
        keys = list(f.keys())
        dtypes = {k: f.get_slice(k).get_dtype() for k in keys}
        dtypes = {k: _st_dtype(v) for k, v in dtypes.items()}
        pairs, others = pair_block_fp8(keys, dtypes)
        wanted = set(names) if names is not None else None
        for wname, sname in pairs.items():
            if wanted is not None and wname not in wanted:
                continue
            w = f.get_tensor(wname)
            s = f.get_tensor(sname)
            _check_grid(wname, w, s)
            wd = w.contiguous().to(device, non_blocking=False)
            sd = s.contiguous().to(device, non_blocking=False)
            rounded, half = 0, False
            if from_half_range:
                codes, s_out = ops.codec_half_to_ocp(wd, sd)
                wd, sd = codes.view(torch.float8_e4m3fn), s_out
            if validate and not ops.weights_finite(wd, sd):
                raise ValueError(f"{wname}: NaN code or nonfinite/negative scale")
            if to_half_range:
                codes, s_out, rounded = ops.codec_ocp_to_half(wd, sd)
                wd, sd, half = codes.view(torch.float8_e4m3fn), s_out, True
            weights[wname] = BlockFP8Weight(wd, sd, half, int(rounded))
        for name in others:
            if wanted is not None and name not in wanted:
                continue
            tensors[name] = f.get_tensor(name).to(device)
    return weights, tensors


_ST_DTYPES = {
    "F8_E4M3": torch.float8_e4m3fn, "F32": torch.float32, "BF16": torch.bfloat16, "F16": torch.float16,
    "F64": torch.float64, "I64": torch.int64, "I32": torch.int32, "I16": torch.int16, "I8": torch.int8,
    "U8": torch.uint8, "BOOL": torch.bool, "F8_E5M2": torch.float8_e5m2,
}


def _st_dtype(name):
    if isinstance(name, torch.dtype):
        return name
    return _ST_DTYPES.get(str(name), None)
