"""CPU restatement of the reference's RMSNorm ops (test infrastructure only).

The reference ops gk_rms_norm_bf16_v1 (csrc/tpc/generic_dense/rms_norm_bf16.c:4-53) and
gk_fused_add_rms_norm_bf16_v1 (csrc/tpc/generic_dense/fused_add_rms_norm_bf16.c:4-63), glue
csrc/host/generic_dense_glue.cpp:135-190 (width 1..8192, epsilon finite and > 0, weight_offset
finite), compute per row of bf16 values:

  add        r = bf16_rne(fp32(x) + fp32(residual))          fused_add_rms_norm_bf16.c:17-21
             (residual_out = r; the plain op uses r = x)
  sum        ss = sum of r*r over the row                      :22 v_bf16_mac_acc32_b, norm_math.h:5-15
  inverse    inv = 1 / sqrt(ss * fp32(1 / width) + epsilon)    :24-25, norm_math.h:17-23
  normalize  norm_out = bf16_rne((r * inv) * (gamma + weight_offset)) in fp32    :27-36

The reference accumulates ss in fp32 lanes joined by a compensated reduction (norm_math.h:5-15) and
refines a hardware reciprocal square root by one Newton step (norm_math.h:17-23).  Both aim at the
correctly rounded value; their exact roundings are not documented.  This restatement, and the GPU
kernel that it checks bit for bit, fixes them as:

  ss   the squares in fp64 (exact for bf16 values), summed in fp64 in one fixed order -- 256 threads,
       thread t taking the 8-element chunks t, t + 256, t + 512, ... in turn, element by element; the
       partial sums of each group of 64 threads folded pairwise (p[i] += p[i + s], s = 32, ..., 1),
       then the four group sums folded the same way (s = 2, 1) -- and rounded to fp32 once;
  inv  fp32(1 / sqrt(fp64(fp32(ss * fp32(1 / width)) + epsilon))): the fp32 multiply and add of
       the reference's expression, then an fp64 square root and division rounded to fp32 once
       (within one fp32 ulp of the correctly rounded value; 0 when the argument is +inf, as
       norm_math.h:22);
  norm fp32 products in the reference's order, no fused multiply-add, one RNE to bf16.

The reference's own test (tests/track_a_device_verify.cpp:465-540) checks residual_out bit for bit
and norm_out within 2 bf16 ulps of an fp64 evaluation; `fp64_reference` restates that evaluation and
`GATE_ULPS` its bound.  The 1x128 quantized form of norm_out is block_fp8.act_quant of it.
"""

import numpy as np
import torch

THREADS = 256
CHUNK = 8
MAX_WIDTH = 8192
GATE_ULPS = 2  # tests/track_a_device_verify.cpp:501,539


def _bf16_to_f32(t):
    return t.to(torch.float32).numpy()


def _f32_to_bf16(a):
    return torch.from_numpy(np.ascontiguousarray(a, dtype=np.float32)).to(torch.bfloat16)


def fused_add(x, residual):
    """bf16 [R, W] x, residual -> bf16 residual_out = bf16_rne(fp32 sum) (fused_add_rms_norm_bf16.c:17-21)."""
    return _f32_to_bf16(_bf16_to_f32(x) + _bf16_to_f32(residual))


def sum_squares(r):
    """fp32 [R]: the fixed-order fp64 sum of the squares of bf16 [R, W] rows, rounded to fp32 once."""
    v = _bf16_to_f32(r).astype(np.float64)
    rows, width = v.shape
    passes = -(-width // (THREADS * CHUNK))
    padded = np.zeros((rows, passes * THREADS * CHUNK), dtype=np.float64)
    padded[:, :width] = v * v
    sq = padded.reshape(rows, passes, THREADS, CHUNK)
    part = np.zeros((rows, THREADS), dtype=np.float64)
    for p in range(passes):
        for i in range(CHUNK):
            part = part + sq[:, p, :, i]
    part = part.reshape(rows, THREADS // 64, 64)
    s = 32
    while s >= 1:
        part = part[:, :, :s] + part[:, :, s:2 * s]
        s //= 2
    part = part[:, :, 0]
    s = THREADS // 128
    while s >= 1:
        part = part[:, :s] + part[:, s:2 * s]
        s //= 2
    with np.errstate(over="ignore"):  # a sum past the fp32 range rounds to +inf
        return part[:, 0].astype(np.float32)


def inverse_rms(ss, width, epsilon):
    """fp32 [R]: fp32(1 / sqrt(fp64(fp32(ss * fp32(1/width)) + eps))) with the fp32 steps of :24-25."""
    ss = np.asarray(ss, dtype=np.float32)
    mean = (ss * np.float32(1.0 / np.float32(width))).astype(np.float32)
    arg = (mean + np.float32(epsilon)).astype(np.float32)
    with np.errstate(divide="ignore", invalid="ignore", over="ignore"):
        inv = (1.0 / np.sqrt(arg.astype(np.float64))).astype(np.float32)
    return np.where(np.isposinf(arg), np.float32(0.0), inv)


def normalize(r, inv, gamma, weight_offset):
    """bf16 [R, W] = bf16_rne(fp32(fp32(r * inv) * fp32(gamma + weight_offset)))."""
    rv = _bf16_to_f32(r)
    g = (_bf16_to_f32(gamma) + np.float32(weight_offset)).astype(np.float32)
    with np.errstate(over="ignore", invalid="ignore"):
        n = (rv * inv[:, None]).astype(np.float32)
        n = (n * g[None, :]).astype(np.float32)
    return _f32_to_bf16(n)


def rms_norm(x, gamma, epsilon, weight_offset=0.0):
    """gk_rms_norm_bf16_v1: bf16 [R, W], gamma bf16 [W] -> bf16 [R, W]."""
    inv = inverse_rms(sum_squares(x), x.shape[1], epsilon)
    return normalize(x, inv, gamma, weight_offset)


def fused_add_rms_norm(x, residual, gamma, epsilon, weight_offset=0.0):
    """gk_fused_add_rms_norm_bf16_v1: -> (residual_out bf16 [R, W], norm_out bf16 [R, W])."""
    r = fused_add(x, residual)
    inv = inverse_rms(sum_squares(r), x.shape[1], epsilon)
    return r, normalize(r, inv, gamma, weight_offset)


def fp64_reference(r, gamma, epsilon, weight_offset):
    """fp64 [R, W]: the check of tests/track_a_device_verify.cpp:490-500 (and :530-538 on the summed rows)."""
    v = _bf16_to_f32(r).astype(np.float64)
    ss = (v * v).sum(axis=1)
    rstd = 1.0 / np.sqrt(ss / v.shape[1] + np.float64(np.float32(epsilon)))
    g = _bf16_to_f32(gamma).astype(np.float64) + np.float64(np.float32(weight_offset))
    return v * rstd[:, None] * g[None, :]


def bf16_ulp_diff(a, b):
    """Element-wise distance in bf16 ulps (ordered bit patterns) of two bf16 tensors."""
    ia = a.view(torch.int16).numpy().astype(np.int32)
    ib = b.view(torch.int16).numpy().astype(np.int32)
    ka = np.where(ia < 0, -32768 - ia, ia)
    kb = np.where(ib < 0, -32768 - ib, ib)
    return np.abs(ka - kb)


def reference_test_inputs(width, rows=5):
    """The inputs of tests/track_a_device_verify.cpp:468-477 (x, residual bf16 [rows, width], gamma bf16 [width])."""
    i = np.arange(width * rows)
    x = (((i * 13) % 41) - 20).astype(np.float32) * np.float32(0.125)
    res = (((i * 7) % 29) - 14).astype(np.float32) * np.float32(0.125)
    g = np.float32(0.5) + (np.arange(width) % 9).astype(np.float32) * np.float32(0.1)
    return (_f32_to_bf16(x.reshape(rows, width)), _f32_to_bf16(res.reshape(rows, width)), _f32_to_bf16(g))
