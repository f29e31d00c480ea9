"""Pin the codec restatement (oracle/fp8_codec.py) with the reference's own known answers.

Known answers come from the reference's tests/test_fp8_codec.py:16-68 (all 254
finite codes against an independent nearest-even search, rounded == 16, the
2x3 fixture, rejections), plus torch's e4m3fn cast of value/2 and round-trip
invariants for the build-defined inverse.
"""

import numpy as np
import pytest
import torch

from oracle import e4m3, fp8_codec


def value(magnitude):
    # Magnitude decode used by the reference's test (test_fp8_codec.py:8-12).
    exponent, mantissa = divmod(magnitude, 8)
    if exponent == 0:
        return mantissa * 2.0 ** -9
    return (1.0 + mantissa / 8.0) * 2.0 ** (exponent - 7)


def nearest_even_half(code):
    """Independent nearest-even search of test_fp8_codec.py:27-35 over Gaudi2 candidates 0..0x77."""
    wanted = value(code & 0x7F) / 2.0
    distance = [abs(value(c) - wanted) for c in range(0x78)]
    best = min(distance)
    ties = [c for c, err in enumerate(distance) if err == best]
    selected = next(c for c in ties if c % 2 == 0) if len(ties) > 1 else ties[0]
    return (code & 0x80) | selected, best


def test_all_finite_codes_against_independent_nearest_even():
    source = np.array([c for c in range(256) if c & 0x7F != 0x7F], dtype=np.uint8)
    scales = np.array([0.0, 0.25, 1.0e30], dtype=np.float32)
    original = source.copy()
    encoded, adjusted, rounded = fp8_codec.reencode_e4m3fn_half(source, scales)
    expected, errors = zip(*(nearest_even_half(int(c)) for c in source))
    assert encoded.tolist() == list(expected)
    assert np.array_equal(source, original)
    assert np.array_equal(adjusted, scales * np.float32(2))
    assert rounded == sum(e != 0 for e in errors) == 16
    assert expected[list(source).index(0x01)] == 0x00
    assert expected[list(source).index(0x81)] == 0x80


def test_codes_equal_torch_cast_of_half_value():
    codes = np.array([c for c in range(256) if c & 0x7F != 0x7F], dtype=np.uint8)
    half = torch.from_numpy(codes).view(torch.float8_e4m3fn).float() * 0.5
    via_torch = half.to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    assert np.array_equal(fp8_codec.forward_table()[codes], via_torch)


def test_nonfinite_codes_and_bad_scales_fail():
    ones = np.ones(1, dtype=np.float32)
    for code in (0x7F, 0xFF):
        w = np.array([0, code], dtype=np.uint8)
        with pytest.raises(ValueError, match="nonfinite"):
            fp8_codec.reencode_e4m3fn_half(w, ones)
        assert w.tolist() == [0, code]
    w = np.zeros(2, dtype=np.uint8)
    for bad in (np.nan, np.inf, -1.0, np.finfo(np.float32).max):
        with pytest.raises(ValueError):
            fp8_codec.reencode_e4m3fn_half(w, np.array([bad], dtype=np.float32))


def test_shape_fixture():
    w = np.array([[0x08, 0x10, 0x78], [0x03, 0x7E, 0x80]], dtype=np.uint8)
    s = np.array([[0.25, 0.5]], dtype=np.float32)
    enc, adj, rounded = fp8_codec.reencode_e4m3fn_half(w, s)
    assert enc.shape == w.shape and adj.shape == s.shape
    assert rounded == 1
    assert enc.tolist() == [[4, 8, 112], [2, 118, 128]]


def test_inverse_round_trips():
    fwd, inv = fp8_codec.forward_table(), fp8_codec.inverse_table()
    halves = np.array([c for c in range(256) if (c & 0x7F) <= 0x76], dtype=np.uint8)
    assert np.array_equal(fwd[inv[halves]], halves)  # fwd(inv(c')) == c' for every m' <= 0x76
    ocp = np.array([c for c in range(256) if c & 0x7F != 0x7F], dtype=np.uint8)
    rounded = ((ocp & 0x7F) < 16) & ((ocp & 1) == 1)
    back = inv[fwd[ocp]]
    assert np.array_equal(back[~rounded], ocp[~rounded])  # exact except the 16 rounded codes
    assert int(rounded.sum()) == 16
    # Doubling is exact: decode(inv(c)) == 2 * decode(c).
    assert np.array_equal(e4m3.decode(inv[halves]), 2 * e4m3.decode(halves))


def test_inverse_rejections():
    s = np.ones(1, dtype=np.float32)
    for code in (0x77, 0x78, 0x7F, 0xF7, 0xFF):
        with pytest.raises(ValueError):
            fp8_codec.decode_half_to_ocp(np.array([code], dtype=np.uint8), s)
    tiny_odd = np.array([1], dtype=np.uint32).view(np.float32)
    with pytest.raises(ValueError):
        fp8_codec.decode_half_to_ocp(np.zeros(1, np.uint8), tiny_odd)
    codes, half = fp8_codec.decode_half_to_ocp(np.array([0x04, 0x84, 0x76], dtype=np.uint8),
                                               np.array([0.5], dtype=np.float32))
    assert codes.tolist() == [0x08, 0x88, 0x7E] and half.tolist() == [0.25]
