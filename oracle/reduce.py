"""CPU restatement of the row-parallel completion (test infrastructure only).

* ``rank_sum_f32`` / ``rank_sum_bf16`` follow csrc/tpc/generic_dense/rank_sum.c:4-42:
  ``gathered`` holds ``world`` contiguous slices of ``elems`` values (slice r at r * elems);
  the result is ((s_0 + s_1) + s_2) + ... with every addition an IEEE fp32 addition
  (numpy float32, round to nearest even), in rank order.  The bf16 form widens each slice to
  fp32 (exact), sums the same way and rounds the sum once to bf16, nearest even
  (``convert_float128_to_bfloat128(..., SW_RHNE)``, :33-34); NaN -> 0x7FC0.
* ``partial_finish`` is the last step of the decode reduce (reduce_bias.c:42-57):
  bf16(fp32(p + bias)).
* ``gemm_partial_f64`` is the oracle GEMM (oracle.block_fp8, block_fp8_oracle.py:25-41) over a
  K range, before bias and rounding: the fp64 sum over the range's groups of P_g * sa * sw.

Pinned by tests/test_oracle_reduce.py: fp32 additions against exact rational sums, the rank
order against planted inputs whose sum differs under every other order, the bf16 rounding
against torch's fp32 -> bf16 cast (round to nearest even) on ties and specials, and the K-range
partials summing to the whole-K oracle.
"""

import numpy as np
import torch

from oracle import block_fp8


def _slices(gathered, world):
    if world < 2 or world > 8:
        raise ValueError("world_size must be in [2, 8]")
    if gathered.ndim != 1 or gathered.size < world or gathered.size % world:
        raise ValueError("gathered length must be a nonzero multiple of world_size")
    return gathered.reshape(world, -1)


def rank_sum_f32(gathered, world):
    """fp32 [world * elems] -> fp32 [elems], rank order (rank_sum.c:35-39)."""
    s = _slices(np.asarray(gathered, dtype=np.float32), world)
    acc = s[0].copy()
    for r in range(1, world):
        acc = (acc + s[r]).astype(np.float32)
    return acc


def bf16_bits_to_f32(bits):
    return (np.asarray(bits, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def f32_to_bf16_bits(v):
    """fp32 -> bf16 bits, round to nearest even; NaN -> 0x7FC0."""
    b = np.asarray(v, dtype=np.float32).view(np.uint32).astype(np.uint64)
    nan = (b & 0x7FFFFFFF) > 0x7F800000
    r = ((b + 0x7FFF + ((b >> 16) & 1)) >> 16).astype(np.uint16)
    r[nan] = 0x7FC0
    return r


def rank_sum_bf16(gathered_bits, world):
    """bf16 bits [world * elems] -> bf16 bits [elems] (rank_sum.c:23-34)."""
    s = _slices(np.asarray(gathered_bits, dtype=np.uint16), world)
    acc = bf16_bits_to_f32(s[0])
    for r in range(1, world):
        acc = (acc + bf16_bits_to_f32(s[r])).astype(np.float32)
    return f32_to_bf16_bits(acc)


def partial_finish(p, bias=None):
    """fp32 [rows, width] (+ bias [width]) -> bf16 bits, one fp32 addition and one rounding."""
    p = np.asarray(p, dtype=np.float32)
    if bias is not None:
        p = (p + np.asarray(bias, dtype=np.float32)[None, :]).astype(np.float32)
    return f32_to_bf16_bits(p)


def gemm_partial_f64(x, weight, scales, k_offset, k_len, *, native_half=False):
    """fp64 [M, N]: the oracle's sum over groups [k_offset/128, (k_offset + k_len)/128) (no bias, unrounded).

    The 1x128 quantization is per group, so the range's codes and scales are those of the whole row.
    """
    if k_offset % 128 or k_len % 128 or k_len <= 0 or k_offset + k_len > x.shape[1]:
        raise ValueError("K range must be whole 128-groups inside K")
    g0, g1 = k_offset // 128, (k_offset + k_len) // 128
    xs, ws = x[:, k_offset:k_offset + k_len], weight[:, k_offset:k_offset + k_len]
    ss = scales[:, g0:g1].contiguous()
    return block_fp8.reference_f64(xs, ws, ss, native_half=native_half)
