"""Pins of oracle/reduce.py (the rank sum of rank_sum.c:4-42, the partial finish, K-range partials).

* every fp32 addition equals the exact rational sum rounded to nearest even (Fraction arithmetic);
* the rank order: inputs whose sum takes a different value under the reversed order and under
  pairwise summation, so an oracle summing in any other order fails;
* the bf16 rounding equals torch's fp32 -> bf16 cast (nearest even) on ties, near-ties, specials;
* the glue's world-size and size rules (generic_dense_glue.cpp:568-600, 871-895) as the oracle's
  own rejections;
* K-range partials of the oracle GEMM sum to its whole-K value and round to its bf16 output.
"""

from fractions import Fraction

import numpy as np
import pytest
import torch

from oracle import block_fp8, reduce, synth


def round_f32(fr):
    """Exact rational -> nearest fp32 (ties to even), by bracketing with nextafter."""
    v = np.float32(float(fr))  # float(fr) rounds correctly to fp64; refine to fp32 below
    lo = v if Fraction(float(v)) <= fr else np.nextafter(v, np.float32(-np.inf))
    hi = np.nextafter(lo, np.float32(np.inf))
    dlo, dhi = fr - Fraction(float(lo)), Fraction(float(hi)) - fr
    if dlo < dhi:
        return lo
    if dhi < dlo:
        return hi
    return lo if (lo.view(np.uint32) & 1) == 0 else hi


def test_fp32_additions_are_correctly_rounded():
    rng = np.random.default_rng(3)
    for world in range(2, 9):
        g = (rng.standard_normal(world * 64) * np.exp2(rng.integers(-30, 30, world * 64))).astype(np.float32)
        got = reduce.rank_sum_f32(g, world)
        s = g.reshape(world, -1)
        for i in range(s.shape[1]):
            acc = s[0, i]
            for r in range(1, world):
                acc = round_f32(Fraction(float(acc)) + Fraction(float(s[r, i])))
            assert got[i].view(np.uint32) == np.float32(acc).view(np.uint32), (world, i)


def test_rank_order_is_load_bearing():
    t = np.float32(2.0 ** 24)
    g = np.array([t, 1, 1, -t], dtype=np.float32)  # world 4, one element per slice
    assert reduce.rank_sum_f32(g, 4)[0] == 0.0       # ((2^24 + 1) + 1) - 2^24: both +1 round away
    rev = np.float32(np.float32(np.float32(-t + 1) + 1) + t)
    pair = np.float32(np.float32(t + 1) + np.float32(1 - t))
    assert rev == 2.0 and pair == 1.0                # every other order gives another value
    bits = reduce.f32_to_bf16_bits(np.array([256.0, 1.0, 1.0, -256.0], np.float32))
    assert reduce.bf16_bits_to_f32(reduce.rank_sum_bf16(bits, 4))[0] == 2.0  # fp32 sum, then one rounding
    # a one-element-per-rank sum whose fp32 result is a bf16 tie: rounded once, to even
    bits = reduce.f32_to_bf16_bits(np.array([1.0, 2.0 ** -8], np.float32))
    assert reduce.rank_sum_bf16(bits, 2)[0] == 0x3F80


def test_bf16_rounding_matches_torch():
    rng = np.random.default_rng(5)
    base = rng.standard_normal(20000).astype(np.float32)
    u = base.view(np.uint32)
    ties = ((u & 0xFFFF0000) | 0x8000).view(np.float32)
    near = np.concatenate([((u & 0xFFFF0000) | d).view(np.float32) for d in (0x7FFF, 0x8001, 0x0001, 0xFFFF)])
    specials = np.array([0.0, -0.0, np.inf, -np.inf, 3.4028235e38, -3.4028235e38, 1e-45, -1e-45,
                         1.1754942e-38], dtype=np.float32)
    v = np.concatenate([base, ties, near, specials])
    want = torch.from_numpy(v).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(reduce.f32_to_bf16_bits(v), want)
    assert reduce.f32_to_bf16_bits(np.array([np.nan], np.float32))[0] == 0x7FC0


def test_glue_rules():
    g = np.zeros(16384, np.float32)
    assert reduce.rank_sum_f32(g, 4).shape == (4096,)          # generic_dense_glue_contract_test.cpp:537-566
    for bad_world in (1, 9):                                    # :582-584
        with pytest.raises(ValueError):
            reduce.rank_sum_f32(g, bad_world)
    with pytest.raises(ValueError):
        reduce.rank_sum_f32(np.zeros(10, np.float32), 4)        # not a multiple of world
    with pytest.raises(ValueError):
        reduce.rank_sum_f32(np.zeros(3, np.float32), 4)         # fewer values than ranks


def test_partial_finish_is_one_rounding():
    p = np.array([[1.0, 2.0 ** -9, -3.0]], np.float32)
    b = np.array([2.0 ** -8, 1.0, 3.0], np.float32)
    got = reduce.partial_finish(p, b)
    want = torch.from_numpy((p + b).astype(np.float32)).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(got, want)
    assert got[0, 0] == 0x3F80 and got[0, 2] == 0x0000        # 1 + 2^-8 ties to even; -3 + 3 = +0


@pytest.mark.parametrize("native_half", [False, True])
def test_k_range_partials_sum_to_whole_k(native_half):
    m, n, k = 5, 384, 1024
    w, s = synth.weight(n, k, seed=41)
    x = synth.activations(m, k, seed=42)
    whole = block_fp8.reference_f64(x, w, s, native_half=native_half)
    parts = sum(reduce.gemm_partial_f64(x, w, s, off, 256, native_half=native_half) for off in range(0, k, 256))
    assert torch.allclose(parts, whole, rtol=1e-12, atol=1e-12 * float(whole.abs().max()))
    assert torch.equal(whole.to(torch.bfloat16), block_fp8.reference(x, w, s, native_half=native_half))
    with pytest.raises(ValueError):
        reduce.gemm_partial_f64(x, w, s, 384, 768)  # 384 + 768 > 1024
