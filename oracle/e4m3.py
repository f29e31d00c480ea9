"""Independent OCP E4M3FN arithmetic in numpy (test infrastructure only).

The reference relies on torch's ``float8_e4m3fn`` cast for every activation
and weight rounding (python/gaudi_kernels/block_fp8_oracle.py:28,32,33).  This
module restates that cast with integer bit operations so that the oracle does
not depend on one library routine alone; tests/test_oracle_e4m3.py pins it
against torch's cast on every tie, every code value and a dense random sweep.

Encoding facts (OCP E4M3FN as published in the OCP 8-bit floating point
specification; tests/test_fp8_codec.py:8-12 of the reference for the magnitude
decode):
  magnitude m = code & 0x7f, e = m >> 3, f = m & 7
  value = (1 + f/8) * 2**(e-7) for e > 0, f * 2**-9 for e == 0
  0x7f / 0xff are NaN; there is no infinity; max finite is 448 (0x7e).
"""

import numpy as np

E4M3_MAX = 448.0


def decode_table():
    """Return the 256-entry float64 table of OCP E4M3FN code values (NaN at 0x7f/0xff)."""
    codes = np.arange(256)
    mag = codes & 0x7F
    e = mag >> 3
    f = mag & 7
    val = np.where(e > 0, (1.0 + f / 8.0) * np.exp2(e.astype(np.float64) - 7.0), f * 2.0 ** -9)
    val = np.where(codes & 0x80, -val, val)
    val[mag == 0x7F] = np.nan
    return val


_DECODE = decode_table()


def decode(codes):
    """uint8 codes (any shape) -> float64 values."""
    return _DECODE[np.asarray(codes, dtype=np.uint8)]


def encode_rne(values):
    """float32 values -> uint8 OCP E4M3FN codes, round to nearest, ties to even.

    Matches torch's ``.to(torch.float8_e4m3fn)``: magnitudes that round above
    448 (i.e. > 464, or exactly 464+ulp and beyond) become NaN (0x7f | sign),
    as does NaN input.  Subnormals use the 2**-9 grid.
    """
    v = np.ascontiguousarray(values, dtype=np.float32)
    bits = v.view(np.uint32)
    sign = ((bits >> 24) & 0x80).astype(np.uint8)
    mbits = bits & np.uint32(0x7FFFFFFF)
    mag = mbits.view(np.float32)
    out = np.zeros(v.shape, dtype=np.uint8)

    is_nan = np.isnan(mag)
    small = mag < np.float32(2.0 ** -6)
    # Subnormal range: nearest multiple of 2**-9, ties to even (np.rint is RNE).
    q = np.rint(np.where(small, mag, 0).astype(np.float64) * 512.0).astype(np.int64)
    sub_code = np.clip(q, 0, 8).astype(np.uint8)  # q == 8 is exactly 2**-6 = code 0x08
    # Normal range: round the fp32 significand to 3 bits, ties to even.
    r = (mbits.astype(np.uint64) + 0x7FFFF + ((mbits.astype(np.uint64) >> 20) & 1)) & 0xFFF00000
    exp = (r >> 23).astype(np.int64) - 127
    man = ((r >> 20) & 7).astype(np.int64)
    norm_code = ((exp + 7) << 3) | man
    over = norm_code > 0x7E  # rounds beyond 448 -> NaN, as torch does
    norm_code = np.clip(norm_code, 0, 0x7F).astype(np.uint8)
    out = np.where(small, sub_code, norm_code).astype(np.uint8)
    out = np.where((~small) & over, np.uint8(0x7F), out)
    out = np.where(is_nan, np.uint8(0x7F), out)
    return (out | sign).astype(np.uint8)
