"""CPU restatement of the load-time E4M3 codec (test infrastructure only).

Forward: python/gaudi_kernels/fp8_codec.py:14-53 of the reference
(``reencode_e4m3fn_half``): OCP E4M3FN checkpoint codes -> Gaudi2 half-range
E4M3 codes holding value/2 (round to nearest, ties to even), fp32 scales x2,
plus the count of codes that had to be rounded.

Inverse (build-defined; the reference has none): Gaudi2 half-range codes ->
OCP E4M3FN codes holding value*2 (exact), fp32 scales /2.

Pinned by: the reference's own known answers (tests/test_fp8_codec.py:16-68:
an independent nearest-even search over all 254 finite codes, rounded == 16,
the 2x3 fixture, the rejections), by torch's e4m3fn cast of value/2, and by
the round-trip invariants fwd(inv(c)) == c, inv(fwd(c)) == c off the 16
rounded codes.  See tests/test_oracle_codec.py.
"""

import numpy as np

CHUNK = 8 * 1024 * 1024  # fp8_codec.py:45 bounds temporaries per 8 Mi codes


def forward_table():
    """256-entry OCP -> half-range byte table (fp8_codec.py:36-40 closed form)."""
    codes = np.arange(256, dtype=np.uint16)
    m = codes & 0x7F
    half = np.where(m >= 16, m - 8, (m >> 1) + ((m & 1) & ((m >> 1) & 1)))
    return ((codes & 0x80) | half).astype(np.uint8)


def inverse_table():
    """256-entry half-range -> OCP byte table: m <= 7 -> 2m, 8 <= m <= 0x76 -> m + 8.

    Magnitudes 0x77..0x7f have no OCP image at twice the value (0x77 is 240,
    480 > 448; 0x78.. are Gaudi2 inf/NaN); they map to the OCP NaN code and the
    callers reject them.
    """
    codes = np.arange(256, dtype=np.uint16)
    m = codes & 0x7F
    dbl = np.where(m <= 7, 2 * m, m + 8)
    dbl = np.where(m >= 0x77, 0x7F, dbl)
    return ((codes & 0x80) | dbl).astype(np.uint8)


def _check_scales(scales):
    s = np.asarray(scales, dtype=np.float32)
    if s.size == 0 or not np.all(np.isfinite(s)) or np.any(s < 0):
        raise ValueError("expected nonempty contiguous finite nonnegative CPU FP32 scales")
    return s


def reencode_e4m3fn_half(codes, scales):
    """Forward codec on uint8 codes / fp32 scales (numpy arrays).

    Returns (half-range codes, 2*scales, rounded count); raises ValueError on a
    NaN code (fp8_codec.py:48-49) or on scales that overflow when doubled
    (fp8_codec.py:30-32).  Inputs are not modified.
    """
    src = np.asarray(codes, dtype=np.uint8)
    s = _check_scales(scales)
    if src.size == 0:
        raise ValueError("expected a nonempty contiguous CPU E4M3FN weight")
    with np.errstate(over="ignore"):
        s2 = s * np.float32(2.0)
    if not np.all(np.isfinite(s2)):
        raise ValueError("doubling FP8 scales overflows FP32")
    table = forward_table()
    flat = src.reshape(-1)
    out = np.empty_like(flat)
    rounded = 0
    for start in range(0, flat.size, CHUNK):
        raw = flat[start:start + CHUNK]
        mag = raw & 0x7F
        if np.any(mag == 0x7F):
            raise ValueError("nonfinite OCP E4M3FN checkpoint code")
        rounded += int(np.count_nonzero((mag < 16) & ((mag & 1) != 0)))
        out[start:start + raw.size] = table[raw]
    return out.reshape(src.shape), s2, rounded


def decode_half_to_ocp(codes, scales):
    """Inverse codec: half-range codes -> OCP codes (value x2, exact), scales / 2.

    Raises ValueError for magnitudes >= 0x77 (no OCP image).  Halving a scale
    is exact unless the result is an fp32 subnormal and the low significand
    bit is set (biased exponent field 0 or 1); those are rejected so that
    dec(inv(c)) * inv_scale == dec(c) * scale holds exactly.
    """
    src = np.asarray(codes, dtype=np.uint8)
    s = _check_scales(scales)
    if np.any((src & 0x7F) >= 0x77):
        raise ValueError("half-range code has no OCP E4M3FN image")
    bits = s.view(np.uint32)
    if np.any(((bits & 0x7F800000) <= 0x00800000) & ((bits & 1) == 1)):
        raise ValueError("halving FP8 scales is inexact")
    return inverse_table()[src], (s * np.float32(0.5)).astype(np.float32)
