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


@pytest.mark.parametrize("e,n,k", [(1, 16, 128), (2, 264, 256), (3, 40, 384), (2, 520, 128), (1, 512, 256)])
def test_experts_round_trip(e, n, k):
    w = np.random.default_rng(e + n + k).integers(0, 256, (e, n, k), dtype=np.uint8)
    p = pack.pack_experts(w)
    assert p.size == e * ((n + 15) // 16 * 16 * k)
    assert np.array_equal(pack.unpack_experts(p, e, n, k), w)


def test_experts_marker_blocks():
    """Hand-worked block numbers: one panel of 3 tiles (n = 40, G = 3): row 17, column 130 is tile 1,
    group 1 -> block 1 * 3 + 1 = 4; two panels (n = 264: 16 tiles + 1, G = 2): row 260, column 200 is
    tile 16, group 1 -> block 16 * 2 + 1 * 1 + 0 = 33, and row 20, column 130 (tile 1, group 1) ->
    block 1 * 16 + 1 = 17; the second expert starts one expert size later."""
    for e, n, k, row, col, block in [(1, 40, 384, 17, 130, 4), (1, 264, 256, 260, 200, 33),
                                     (1, 264, 256, 20, 130, 17), (2, 40, 384, 0, 0, 0)]:
        for ex in range(e):
            w = np.zeros((e, n, k), dtype=np.uint8)
            w[ex, row, col] = 0xA5
            p = pack.pack_experts(w)
            c = col % 128
            q, h, b = c // 32, (c % 32) // 16, c % 16
            per = (n + 15) // 16 * 16 * k
            addr = ex * per + block * 2048 + h * 1024 + 16 * (16 * q + row % 16) + b
            assert p[addr] == 0xA5 and np.count_nonzero(p) == 1, (n, row, col, ex)


def test_experts_same_blocks_as_tile_major():
    """Panel p's block for (group g, tile i of the panel) is pack_weight's block (tile 16 p + i, group g)."""
    n, k = 520, 256
    w = np.random.default_rng(9).integers(0, 256, (1, n, k), dtype=np.uint8)
    tm = pack.pack_weight(w[0]).reshape(-1, k // 128, 2048)
    pm = pack.pack_experts(w).reshape(-1, 2048)
    t, g = tm.shape[0], k // 128
    b = 0
    for p0 in range(0, t, 16):
        nbp = min(16, t - p0)
        for gg in range(g):
            for i in range(nbp):
                assert np.array_equal(pm[b], tm[p0 + i, gg])
                b += 1
    assert b == pm.shape[0]
