"""Activation quantization at the E4M3 rounding ties, bit for bit against the oracle.

Random inputs almost never put a quotient x / s exactly on a rounding tie of the E4M3 grid, so this
test builds groups that do (block_fp8_oracle.py:27-28 numerics):
  * exact ties: a group maximum of 448 * 2^e makes s = 2^e exactly, so x = T * 2^e lands on every tie T
    (midpoint of two neighbouring E4M3 values, normal and subnormal grids, both signs), and x one bf16
    step above and below T * 2^e lands beside it;
  * non-power-of-two scales: (x, amax) pairs of bf16 values found by search whose fp32 quotient is
    exactly a tie or one fp32 ulp below it (toward zero).  (A quotient one ulp above a tie never comes
    out of bf16 inputs under this scale rule; the search over 3.3 M candidates finds none.)
The device codes and scales must equal oracle/block_fp8.act_quant (torch's RNE cast) and
act_quant_bits (the independent bit-arithmetic encoder) in both modes and both activation layouts.
"""

import numpy as np
import pytest
import torch

from gaudi_kernels import ops
from oracle import block_fp8, e4m3

pytestmark = pytest.mark.gpu

VALS = e4m3.decode(np.arange(0x7F)).astype(np.float64)          # codes 0x00..0x7E: 0 .. 448
TIES = (VALS[:-1] + VALS[1:]) / 2                                # 126 ties, 2^-10 .. 432
R448 = np.float32(1.0) / np.float32(448.0)


def bf16(v):
    """Nearest bf16 (round to nearest even) of fp32/fp64 values, returned as float32."""
    f = np.asarray(v, np.float32).view(np.uint32).astype(np.uint64)
    return ((f + 0x7FFF + ((f >> 16) & 1)) >> 16 << 16).astype(np.uint32).view(np.float32)


def bf16_step(v, d):
    return (np.asarray(v, np.float32).view(np.uint32).astype(np.int64) + (d << 16)).astype(np.uint32).view(np.float32)


def tie_groups():
    groups = []
    # exact quotients: s = 2^e
    for e in (-9, -4, 0, 3):
        amax = np.float32(448.0 * 2.0 ** e)
        assert np.float32(amax * R448) == np.float32(2.0 ** e)
        on = (TIES * 2.0 ** e).astype(np.float32)
        assert np.array_equal(bf16(on), on)
        for sign in (1, -1):
            for xs in (on, bf16_step(on, 1), bf16_step(on, -1)):
                groups.append(np.concatenate([[amax], sign * np.minimum(xs, amax)]).astype(np.float32))
    # searched pairs: fp32(x / s) == T or T - 1 ulp
    amaxes = np.array([m * 2.0 ** e for e in range(-14, 14) for m in np.arange(128, 256) / 128.0], np.float32)
    s = (amaxes * R448).astype(np.float32)
    by_amax = {}
    for t in TIES:
        t32 = np.float32(t)
        targets = (t32, np.nextafter(t32, np.float32(0)))
        x0 = bf16(t * s.astype(np.float64))
        for d in (-2, -1, 0, 1, 2):
            xb = bf16_step(x0, d)
            ok = (xb > 0) & (xb <= amaxes)
            q = (xb / s).astype(np.float32)
            for i in np.nonzero(ok & ((q == targets[0]) | (q == targets[1])))[0]:
                by_amax.setdefault(i, []).append(xb[i])
    hits = 0
    for i, xs in sorted(by_amax.items()):
        xs = np.unique(np.array(xs, np.float32))
        hits += len(xs)
        for c in range(0, len(xs), 126):
            chunk = xs[c:c + 126]
            signs = np.where(np.arange(len(chunk)) % 2 == 0, 1.0, -1.0).astype(np.float32)
            groups.append(np.concatenate([[amaxes[i]], chunk * signs]).astype(np.float32))
    assert hits > 10000
    return groups


def rows_of(groups, k=4096):
    g_per_row = k // 128
    n_rows = -(-len(groups) // g_per_row)
    x = np.zeros((n_rows, k), np.float32)
    for i, g in enumerate(groups):
        r, c = divmod(i, g_per_row)
        x[r, c * 128: c * 128 + len(g)] = g
    assert np.array_equal(bf16(x), x)
    return torch.from_numpy(x).bfloat16()


@pytest.fixture(scope="module")
def tie_rows():
    return rows_of(tie_groups())


@pytest.mark.parametrize("native_half", [False, True])
def test_quantizer_ties_bit_exact(tie_rows, native_half):
    x = tie_rows
    m, k = x.shape
    want_q, want_sa = block_fp8.act_quant(x, native_half)
    bits_q, bits_sa = block_fp8.act_quant_bits(x.float().numpy(), native_half)
    assert np.array_equal(want_q.numpy(), bits_q) and np.array_equal(want_sa.numpy(), bits_sa)
    q, sa = ops.act_quant(x.cuda(), native_half=native_half, m_pad=m)
    got_q = q.permute(1, 0, 2).reshape(m, k).cpu()
    assert torch.equal(got_q, want_q), int((got_q != want_q).sum())
    assert torch.equal(sa.t().contiguous().cpu().view(torch.int32), want_sa.contiguous().view(torch.int32))
    # the decode fragment layout (16-token tiles) holds the same codes
    for r0 in range(0, min(m, 64), 16):
        xs = x[r0:r0 + 16]
        qp, sap = ops.act_quant(xs.cuda(), native_half=native_half, decode_layout=True)
        got = ops.decode_layout_to_standard(qp).permute(1, 0, 2).reshape(16, k).cpu()[: xs.shape[0]]
        assert torch.equal(got, want_q[r0:r0 + 16])


def test_tie_codes_round_to_even(tie_rows):
    """On the exact ties (s = 2^e) each code is the even neighbour: the reference cast rounds ties to even."""
    x = tie_rows[:1]                                    # row 0 holds the s = 2^-9 groups
    codes, _ = block_fp8.act_quant(x)
    q, _ = ops.act_quant(x.cuda(), m_pad=1)
    got = q.permute(1, 0, 2).reshape(1, -1).cpu()
    assert torch.equal(got, codes)
    c = got[0, 1:127].numpy().astype(np.int64)           # group 0: +T * 2^-9 for the 126 ties
    i = np.arange(126)                                    # tie i lies between codes i and i + 1
    assert np.array_equal(c, np.where(i % 2 == 0, i, i + 1))
