"""The reference's five 1K FP16 GEMM test cases as data + checker (test infrastructure only).

tests/fp8_hybrid_tpcsim_test.cpp:180-380 (cases :388-392) runs the Gaudi2 prefill chain on
generated inputs and accepts it when every output row's bf16 relative L2 error against an FP64
OCP reference is <= 0.01 (:378), with exact zeros on identically zero rows (:369-371).  This
module restates, for this build's tests:

  * the closed-form weights (:211-226: code = ((col*17 + g*31 + i*7) % 118) + 8, sign from row 0
    of x or from a parity pattern), block scales (:207) and bias (:230);
  * the checker (:326-378): per 1x128 group s = fp32(max|x| / 448) (1 for an all-zero group),
    E4M3 RNE of fp32(|x| / s) clamped to 448 (ties to the even code), the FP64 sum with the
    original OCP weights and scales plus bias, rounded once from FP64 to bf16;
  * the per-row relative L2 error.

The activations are the fixture tests/golden/hybrid_gemm_x.npz, written by
tests/golden/make_hybrid_x.py from the reference's generator recipe (:187-201).

Pinned by: tests/test_oracle_hybrid.py -- with the oracle's scale rule the checker (binary-search
RNE, one FP64 -> bf16 rounding) agrees with oracle/block_fp8.reference (torch cast, FP64 -> fp32 ->
bf16) to the last bf16 ulp; the fixture's documented structure; the weight formula on
hand-computed entries; the rounding helpers on ties.
"""

import os

import numpy as np

from oracle import e4m3

FIXTURE = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "tests", "golden",
                       "hybrid_gemm_x.npz")
GATE = 0.01


def load_cases():
    """[(m, n, k, bias, tiny, chunk_groups, x_bits uint16 [m, k])] in the reference's order."""
    d = np.load(FIXTURE)
    return [tuple(int(v) for v in row) + (d[f"x{i}"],) for i, row in enumerate(d["cases"])]


def bf16_to_f32(bits):
    return (np.asarray(bits, dtype=np.uint32) << 16).view(np.float32)


def weights(n, k, x_bits):
    """OCP E4M3 codes uint8 [n, k] and fp32 block scales [n/128, k/128] (:205-226)."""
    groups, blocks = k // 128, n // 128
    nb, g = np.meshgrid(np.arange(blocks), np.arange(groups), indexing="ij")
    scales = ((np.float32(0.5) + np.float32(0.25) * ((nb * 5 + g * 3) % 11).astype(np.float32))
              * np.float32(1e-3)).astype(np.float32)
    col = np.arange(n)[:, None, None]
    gg = np.arange(groups)[None, :, None]
    i = np.arange(128)[None, None, :]
    code = ((col * 17 + gg * 31 + i * 7) % 118 + 8).astype(np.uint8)
    x0 = bf16_to_f32(x_bits[0]).reshape(groups, 128)  # row 0 of x (the reference indexes it without a row)
    prev = np.concatenate([np.zeros((1, 128), np.float32), x0[:-1]])[None]
    same = (prev < 0) == (x0[None] < 0)
    use_x = (gg % 2 == 1) & (i % 5 != 0)
    parity = ((col * 3 + gg * 5 + i) & 1) != 0
    sign = np.where(use_x, same, parity)
    code = np.where(sign, code | 0x80, code).astype(np.uint8)
    return code.reshape(n, k), scales


def bias(n):
    c = np.arange(n)
    return (np.where(c & 1, np.float32(-0.125), np.float32(0.125)) + c.astype(np.float32) * np.float32(1e-4)
            ).astype(np.float32)


def _rne_code(scaled):
    """Magnitude code (0..126) of the OCP E4M3 value nearest to `scaled` (>= 0), ties to the even code."""
    mags = e4m3.decode(np.arange(127, dtype=np.uint8)).astype(np.float64)
    up = np.minimum(np.searchsorted(mags, scaled, side="left"), 126)
    down = np.maximum(up - 1, 0)
    d_down, d_up = scaled - mags[down], mags[up] - scaled
    pick_down = (up > 0) & ((d_down < d_up) | ((d_down == d_up) & (down % 2 == 0)))
    return np.where(pick_down, down, up), mags


def _f64_to_bf16(v):
    """FP64 -> bf16 value, one round to nearest even (normal range)."""
    mant, ex = np.frexp(v)
    return np.ldexp(np.rint(mant * 256.0) / 256.0, ex)


def checker(x_bits, codes, scales, b=None, scale_rule="tpc"):
    """The reference test's FP64 OCP result rounded to bf16 (:326-366), float64 [m, n].

    scale_rule "tpc": the test's group scale fp32(max|x| / 448), 1 for an all-zero group (:341-343);
    "oracle": block_fp8_oracle.py:27, fp32(max(max|x|, 1e-10) * fp32(1/448)) -- the rule this build
    implements.  The two differ by at most one fp32 ulp, which flips an E4M3 code now and then (and by
    far more below 1e-10, where the oracle clamps).
    """
    m, k = x_bits.shape
    x = bf16_to_f32(x_bits).reshape(m, k // 128, 128)
    amax = np.abs(x).max(axis=2, keepdims=True).astype(np.float32)
    if scale_rule == "tpc":
        amax = np.where(amax == 0, np.float32(1.0), amax).astype(np.float32)
        s32 = (amax / np.float32(448.0)).astype(np.float32)
    else:
        s32 = (np.maximum(amax, np.float32(1e-10)) * (np.float32(1.0) / np.float32(448.0))).astype(np.float32)
    scaled = np.minimum(448.0, (np.abs(x) / s32).astype(np.float32).astype(np.float64))
    code, mags = _rne_code(scaled)
    qx = (np.copysign(mags[code] * s32.astype(np.float64), x.astype(np.float64))).reshape(m, k)
    wv = e4m3.decode(codes).astype(np.float64) * np.repeat(np.repeat(scales.astype(np.float64), 128, 0), 128, 1)
    ref = qx @ wv.T
    if b is not None:
        ref = ref + b.astype(np.float64)[None]
    return _f64_to_bf16(ref)


def row_rel_l2(y, ref):
    """Per-row sqrt(sum (y - ref)^2 / sum ref^2); rows with ref == 0 report the raw error sum (must be 0)."""
    y = np.asarray(y, dtype=np.float64)
    err = ((y - ref) ** 2).sum(axis=1)
    den = (ref ** 2).sum(axis=1)
    return np.where(den == 0, err, np.sqrt(err / np.where(den == 0, 1.0, den)))
