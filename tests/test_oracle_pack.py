"""The packed-weight layout restatement (oracle/pack.py), pinned on the CPU."""

import numpy as np
import pytest

from oracle import pack


@pytest.mark.parametrize("n,k", [(16, 128), (1, 128), (37, 256), (264, 1024)])
def test_round_trip(n, k):
    w = np.random.default_rng(n + k).integers(0, 256, (n, k), dtype=np.uint8)
    p = pack.pack_weight(w)
    assert p.size == (n + 15) // 16 * 16 * k
    assert np.array_equal(pack.unpack_weight(p, n, k), w)
    assert not p[n * k:].any() if n % 16 == 0 else True


def test_marker_positions():
    """Hand-worked addresses: byte (row, col) -> block (row // 16, col // 128), piece (h, l), byte b."""
    n, k = 40, 384
    g_count = k // 128
    for row, col in [(0, 0), (0, 31), (0, 32), (0, 48), (5, 127), (17, 130), (39, 383), (31, 200)]:
        w = np.zeros((n, k), dtype=np.uint8)
        w[row, col] = 0xA5
        p = pack.pack_weight(w)
        t, rr, g, c = row // 16, row % 16, col // 128, col % 128
        q, h, b = c // 32, (c % 32) // 16, c % 16
        addr = (t * g_count + g) * 2048 + h * 1024 + 16 * (16 * q + rr) + b
        assert p[addr] == 0xA5 and np.count_nonzero(p) == 1, (row, col)


def test_padding_rows_zero():
    w = np.full((20, 128), 7, dtype=np.uint8)
    p = pack.pack_weight(w).reshape(2, 1, 2, 4, 16, 16)    # [t, g, h, q, rr, b]
    assert (p[1, :, :, :, 4:, :] == 0).all() and (p[1, :, :, :, :4, :] == 7).all() and (p[0] == 7).all()


def test_rejects_ragged_k():
    with pytest.raises(ValueError):
        pack.pack_weight(np.zeros((16, 100), dtype=np.uint8))
