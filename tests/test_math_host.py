"""Check the kernels' bit arithmetic (csrc/gk_fp8_math.h) on the CPU against the oracle.

The header is compiled with g++ (tests/csrc/math_check.cpp) -- the same source
the gfx950 kernels include -- and swept against oracle/e4m3.py and
oracle/fp8_codec.py: the E4M3 encoder on ties and a dense sweep, the decoder
on all codes, bf16 rounding, and every SWAR codec primitive on all 256 byte
values in each byte lane.
"""

import ctypes
import os
import subprocess

import numpy as np
import pytest
import torch

from oracle import e4m3, fp8_codec

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
BUILD = os.path.join(ROOT, "tests", "_build")


@pytest.fixture(scope="module")
def mc():
    os.makedirs(BUILD, exist_ok=True)
    so = os.path.join(BUILD, "libmath_check.so")
    src = os.path.join(ROOT, "tests", "csrc", "math_check.cpp")
    subprocess.run(["g++", "-O2", "-std=c++17", "-ffp-contract=off", "-pthread", "-shared", "-fPIC",
                    "-I", os.path.join(ROOT, "gaudi-kernels_amd", "csrc"), src, "-o", so], check=True)
    lib = ctypes.CDLL(so)
    return lib


def _p(a):
    return a.ctypes.data_as(ctypes.c_void_p)


def run_encode(lib, v):
    v = np.ascontiguousarray(v, dtype=np.float32)
    out = np.empty(v.shape, dtype=np.uint8)
    lib.mc_e4m3_rne(_p(v), _p(out), ctypes.c_int64(v.size))
    return out


def test_encoder_matches_oracle(mc):
    vals = e4m3.decode(np.arange(0x7F)).astype(np.float64)
    mids = (vals[:-1] + vals[1:]) / 2
    base = np.concatenate([vals, mids]).astype(np.float32)
    u = base.view(np.uint32)
    near = np.concatenate([(u + d).view(np.float32) for d in (1, 2)] + [(u[u > 2] - d).view(np.float32) for d in (1, 2)])
    rng = np.random.default_rng(1)
    sweep = np.concatenate([base, near, rng.uniform(-448, 448, 2_000_000).astype(np.float32),
                            (np.exp2(rng.uniform(-30, 8.8, 1_000_000)) * rng.choice([-1, 1], 1_000_000)).astype(np.float32)])
    sweep = np.clip(sweep, -448, 448).astype(np.float32)
    sweep = np.concatenate([sweep, -sweep])
    assert np.array_equal(run_encode(mc, sweep), e4m3.encode_rne(sweep))


def test_encoder_stride_sweep_of_all_floats_below_448(mc):
    # every 61st fp32 bit pattern in [0, 448]
    top = np.array([448.0], dtype=np.float32).view(np.uint32)[0]
    pats = np.arange(0, int(top) + 1, 61, dtype=np.uint32)
    v = pats.view(np.float32)
    assert np.array_equal(run_encode(mc, v), e4m3.encode_rne(v))


def test_decoder_all_codes(mc):
    codes = np.array([c for c in range(256) if c & 0x7F != 0x7F], dtype=np.uint8)
    out = np.empty(codes.shape, dtype=np.float32)
    mc.mc_e4m3_value(_p(codes), _p(out), ctypes.c_int64(codes.size))
    assert np.array_equal(out.astype(np.float64), e4m3.decode(codes))


def test_bf16_rounding_matches_torch(mc):
    rng = np.random.default_rng(2)
    v = np.concatenate([rng.standard_normal(1_000_000).astype(np.float32) * 1e3,
                        (np.arange(1 << 16, dtype=np.uint32) << 16 | 0x8000).view(np.float32)])  # ties
    v = v[np.isfinite(v)]
    out = np.empty(v.shape, dtype=np.uint16)
    mc.mc_bf16_rne(_p(v), _p(out), ctypes.c_int64(v.size))
    want = torch.from_numpy(v).bfloat16().view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(out, want)


def swar(lib, op, words):
    words = np.ascontiguousarray(words, dtype=np.uint32)
    out = np.empty(words.shape, dtype=np.uint32)
    lib.mc_swar(ctypes.c_int(op), _p(words), _p(out), ctypes.c_int64(words.size))
    return out


def test_swar_codec_all_bytes_all_lanes(mc):
    rng = np.random.default_rng(3)
    fwd, inv = fp8_codec.forward_table(), fp8_codec.inverse_table()
    for lane in range(4):
        for trial in range(4):
            others = rng.integers(0, 256, (256, 4), dtype=np.uint8)
            others[:, lane] = np.arange(256, dtype=np.uint8)
            words = others.view(np.uint32).reshape(-1)
            b = others
            # forward codec, NaN flags, rounded counts
            got = swar(mc, 0, words).view(np.uint8).reshape(256, 4)
            assert np.array_equal(got, fwd[b])
            nan = swar(mc, 1, words).view(np.uint8).reshape(256, 4)
            assert np.array_equal(nan, np.where((b & 0x7F) == 0x7F, 0x80, 0).astype(np.uint8))
            cnt = swar(mc, 2, words)
            assert np.array_equal(cnt, (((b & 0x7F) < 16) & ((b & 1) == 1)).sum(1))
            # inverse codec and its invalid flags (valid bytes only are compared)
            got_inv = swar(mc, 3, words).view(np.uint8).reshape(256, 4)
            valid = (b & 0x7F) <= 0x76
            assert np.array_equal(got_inv[valid], inv[b][valid])
            bad = swar(mc, 4, words).view(np.uint8).reshape(256, 4)
            assert np.array_equal(bad, np.where(valid, 0, 0x80).astype(np.uint8))


def test_quantizer_division_exhaustive(mc):
    """gk::act_quotient gives the IEEE-division E4M3 code for every bf16 x and bf16 amax >= |x| (2^31 pairs), with
    the correctly rounded reciprocal of the scale and with either of its neighbours (any faithful reciprocal)."""
    mc.mc_div_mismatches.restype = ctypes.c_int64
    assert mc.mc_div_mismatches(ctypes.c_int(min(8, os.cpu_count() or 1))) == 0
