"""Pin the oracle's E4M3 arithmetic (oracle/e4m3.py) against torch's float8_e4m3fn.

The reference rounds every activation and weight with torch's e4m3fn cast
(block_fp8_oracle.py:28,32,33); the oracle's bit-arithmetic encoder must agree
with that cast on every tie, every code value and a dense sweep, and its
decode table must agree with torch's e4m3fn -> fp32 conversion.
"""

import numpy as np
import torch

from oracle import e4m3


def torch_encode(vals):
    t = torch.from_numpy(np.ascontiguousarray(vals, dtype=np.float32))
    return t.to(torch.float8_e4m3fn).view(torch.uint8).numpy()


def code_values():
    tab = e4m3.decode_table()
    finite = [c for c in range(0x7F)]
    return np.array([tab[c] for c in finite], dtype=np.float64)


def test_decode_table_matches_torch():
    codes = np.array([c for c in range(256) if c & 0x7F != 0x7F], dtype=np.uint8)
    ours = e4m3.decode(codes)
    theirs = torch.from_numpy(codes).view(torch.float8_e4m3fn).float().numpy().astype(np.float64)
    assert np.array_equal(ours, theirs)
    nan = torch.tensor([0x7F, 0xFF], dtype=torch.uint8).view(torch.float8_e4m3fn).float()
    assert torch.isnan(nan).all() and np.isnan(e4m3.decode(np.array([0x7F, 0xFF]))).all()
    assert e4m3.decode(np.array([0x7E]))[0] == 448.0 and e4m3.decode(np.array([0x01]))[0] == 2.0 ** -9


def test_encode_exact_codes_and_ties():
    vals = code_values()
    mids = (vals[:-1] + vals[1:]) / 2  # exactly representable in fp32
    pts = np.concatenate([vals, mids]).astype(np.float32)
    near = []
    for p in pts:
        b = np.array([p], dtype=np.float32).view(np.uint32)[0]
        for d in (-2, -1, 1, 2):
            if p > 0 or d > 0:
                near.append(np.array([b + np.uint32(d) if d > 0 else b - np.uint32(-d)], dtype=np.uint32).view(np.float32)[0])
    pts = np.concatenate([pts, np.array(near, dtype=np.float32)])
    pts = pts[np.abs(pts) <= 470]
    allp = np.concatenate([pts, -pts])
    assert np.array_equal(e4m3.encode_rne(allp), torch_encode(allp))


def test_encode_dense_sweep_and_specials():
    rng = np.random.default_rng(7)
    v = np.concatenate([
        rng.uniform(-500, 500, 1_000_000),
        rng.uniform(-0.02, 0.02, 500_000),
        np.exp2(rng.uniform(-40, 9, 500_000)) * rng.choice([-1, 1], 500_000),
    ]).astype(np.float32)
    assert np.array_equal(e4m3.encode_rne(v), torch_encode(v))
    special = np.array([0.0, -0.0, 448.0, 464.0, 464.0001, 480.0, -480.0, 1e30, np.inf, -np.inf, np.nan,
                        2.0 ** -10, 3 * 2.0 ** -10, 5 * 2.0 ** -10, 2.0 ** -6, 240.0, 232.0], dtype=np.float32)
    ours, theirs = e4m3.encode_rne(special), torch_encode(special)
    # NaN encodings: torch keeps the sign of a NaN input; compare magnitude for those.
    assert np.array_equal(ours & 0x7F, theirs & 0x7F)
    assert np.array_equal(ours[:-1], theirs[:-1])


def test_encode_known_codes():
    # torch 2.10 facts the oracle depends on: ties-to-even on the subnormal
    # grid, 464 -> 448, >= 480 -> NaN, 240 -> 0x77, 232 -> 0x76.
    v = np.array([2.0 ** -10, 3 * 2.0 ** -10, 5 * 2.0 ** -10, 464, 480, 240, 232], dtype=np.float32)
    assert e4m3.encode_rne(v).tolist() == [0x00, 0x02, 0x02, 0x7E, 0x7F, 0x77, 0x76]
