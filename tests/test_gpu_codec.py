"""GPU codec parity: the reference's codec tests, run against the gfx950 kernels.

tests/test_fp8_codec.py:16-68 of the reference, restated against
gaudi_kernels.reencode_e4m3fn_half (same signature; CPU tensors in, CPU out),
plus bit-exact sweeps of large device tensors, unaligned views and the
inverse codec against the CPU oracle tables.
"""

import numpy as np
import pytest
import torch

from gaudi_kernels import decode_half_to_ocp, reencode_e4m3fn_half
from oracle import fp8_codec as ofc

pytestmark = pytest.mark.gpu


def value(magnitude):
    exponent, mantissa = divmod(magnitude, 8)
    if exponent == 0:
        return mantissa * 2.0 ** -9
    return (1.0 + mantissa / 8.0) * 2.0 ** (exponent - 7)


def test_all_finite_codes_against_independent_nearest_even():
    source = [code for code in range(256) if code & 0x7F != 0x7F]
    weight = torch.tensor(source, dtype=torch.uint8).view(torch.float8_e4m3fn)
    scales = torch.tensor([0.0, 0.25, 1.0e30], dtype=torch.float32)
    original = weight.view(torch.uint8).clone()
    encoded, adjusted, rounded = reencode_e4m3fn_half(weight, scales)
    expected, errors = [], []
    for code in source:
        wanted = value(code & 0x7F) / 2.0
        distance = [abs(value(c) - wanted) for c in range(0x78)]
        best = min(distance)
        ties = [c for c, e in enumerate(distance) if e == best]
        selected = next(c for c in ties if c % 2 == 0) if len(ties) > 1 else ties[0]
        expected.append((code & 0x80) | selected)
        errors.append(best)
    assert encoded.device.type == "cpu"
    assert encoded.view(torch.uint8).tolist() == expected
    assert torch.equal(weight.view(torch.uint8), original)
    assert torch.equal(adjusted, scales * 2)
    assert rounded == sum(e != 0 for e in errors) == 16
    assert expected[source.index(0x01)] == 0x00 and expected[source.index(0x81)] == 0x80


def test_nonfinite_codes_and_bad_scales_fail():
    scales = torch.ones(1, dtype=torch.float32)
    for code in (0x7F, 0xFF):
        weight = torch.tensor([0, code], dtype=torch.uint8).view(torch.float8_e4m3fn)
        with pytest.raises(ValueError, match="nonfinite"):
            reencode_e4m3fn_half(weight, scales)
        assert weight.view(torch.uint8).tolist() == [0, code]
    weight = torch.zeros(2, dtype=torch.uint8).view(torch.float8_e4m3fn)
    for bad in (float("nan"), float("inf"), -1.0, torch.finfo(torch.float32).max):
        with pytest.raises(ValueError):
            reencode_e4m3fn_half(weight, torch.tensor([bad], dtype=torch.float32))


def test_shape_dtype_and_contiguity():
    weight = torch.tensor([[0x08, 0x10, 0x78], [0x03, 0x7E, 0x80]], dtype=torch.uint8).view(torch.float8_e4m3fn)
    scales = torch.tensor([[0.25, 0.5]], dtype=torch.float32)
    encoded, adjusted, rounded = reencode_e4m3fn_half(weight, scales)
    assert encoded.shape == weight.shape and adjusted.shape == scales.shape
    assert rounded == 1
    assert encoded.view(torch.uint8).tolist() == [[4, 8, 112], [2, 118, 128]]
    with pytest.raises(ValueError):
        reencode_e4m3fn_half(weight.t(), scales)
    with pytest.raises(ValueError):
        reencode_e4m3fn_half(weight, scales.to(torch.float64))


@pytest.mark.parametrize("n", [1, 15, 16, 17, 4095, 1 << 20, (1 << 24) + 3, (1 << 24) + 16 * 5 + 3])
def test_device_sweep_bit_exact(n):
    gen = torch.Generator().manual_seed(n)
    codes = torch.randint(0, 256, (n,), generator=gen, dtype=torch.uint8)
    codes[(codes & 0x7F) == 0x7F] ^= 0x01  # no NaN codes
    scales = torch.rand(max(1, n // 1000), generator=gen)
    d = codes.cuda().view(torch.float8_e4m3fn)
    enc, s2, rounded = reencode_e4m3fn_half(d, scales.cuda())
    want, want_s, want_r = ofc.reencode_e4m3fn_half(codes.numpy(), scales.numpy())
    assert enc.is_cuda and np.array_equal(enc.view(torch.uint8).cpu().numpy(), want)
    assert np.array_equal(s2.cpu().numpy(), want_s) and rounded == want_r


def test_unaligned_views_and_nan_anywhere():
    gen = torch.Generator().manual_seed(9)
    base = torch.randint(0, 256, (100_003,), generator=gen, dtype=torch.uint8)
    base[(base & 0x7F) == 0x7F] = 0x10
    dev = base.cuda()
    view = dev[3:]  # contiguous, not 16-byte aligned
    enc, _, rounded = reencode_e4m3fn_half(view.view(torch.float8_e4m3fn), torch.ones(1, device="cuda"))
    want, _, want_r = ofc.reencode_e4m3fn_half(base[3:].numpy(), np.ones(1, np.float32))
    assert np.array_equal(enc.view(torch.uint8).cpu().numpy(), want) and rounded == want_r
    for pos in (0, 17, 50_000, 100_002):  # NaN code in the vector body and in the tail
        bad = dev.clone()
        bad[pos] = 0xFF
        with pytest.raises(ValueError, match="nonfinite"):
            reencode_e4m3fn_half(bad.view(torch.float8_e4m3fn), torch.ones(1, device="cuda"))


def test_inverse_codec_round_trip_and_rejections():
    halves = torch.tensor([c for c in range(256) if (c & 0x7F) <= 0x76], dtype=torch.uint8)
    s = torch.tensor([0.5, 3.0], dtype=torch.float32)
    ocp, s_half = decode_half_to_ocp(halves.view(torch.float8_e4m3fn), s)
    want, want_s = ofc.decode_half_to_ocp(halves.numpy(), s.numpy())
    assert np.array_equal(ocp.view(torch.uint8).numpy(), want) and np.array_equal(s_half.numpy(), want_s)
    back, s_back, _ = reencode_e4m3fn_half(ocp, s_half)
    assert torch.equal(back.view(torch.uint8), halves) and torch.equal(s_back, s)
    for code in (0x77, 0x7F, 0xF8):
        with pytest.raises(ValueError):
            decode_half_to_ocp(torch.tensor([code], dtype=torch.uint8).view(torch.float8_e4m3fn), s)
    tiny = torch.tensor([1], dtype=torch.int32).view(torch.float32)
    with pytest.raises(ValueError, match="inexact"):
        decode_half_to_ocp(torch.zeros(4, dtype=torch.uint8).view(torch.float8_e4m3fn), tiny)
