"""CPU restatement of the load-time weight packing (test infrastructure only).

The reference leaves layout packing to the loader (python/gaudi_kernels/fp8_codec.py:19:
"layout packing is a separate step"; the Gaudi2 runtime packs to [G, N, 128],
fp8_hybrid_tpcsim_test.cpp:223).  This build packs into the fragment order of the
gfx950 FP8 matrix instructions (include/gk_fp8.h, gk_fp8_pack_weight): for 16-row
tile t and 128-K group g a 2 KB block whose 16-byte piece (h, l) holds bytes
[128 g + 32 (l // 16) + 16 h, +16) of row 16 t + l % 16, zeros past N.

Written here as one reshape + transpose of the row-major codes (the device kernel
computes each piece's source address instead).  Pinned by: unpack(pack(w)) == w on
ragged shapes, the block/piece positions of hand-placed marker bytes, and, on the
GPU, GEMM results on packed weights bit-identical to those on the row-major codes
(tests/test_gpu_pack.py) -- a misplaced piece changes the matrix-core operands.

Expert weights (include/gk_fp8.h, gk_fp8_pack_experts) hold the same 2 KB blocks in
panel-major order: tiles in panels of 16 (256 rows), panel p's blocks from block
16 G p on, group by group, the panel's nbp = min(16, T - 16 p) tiles side by side.
Pinned by: the round trip, hand-worked block numbers of marker bytes in one- and
two-panel shapes, and the block-for-block relation to pack_weight
(tests/test_oracle_pack.py); on the GPU, MoE layers on packed experts bit-identical
to the row-major ones (tests/test_gpu_moe.py).
"""

import numpy as np


def pack_weight(w):
    """uint8 [N, K] (K % 128 == 0) -> uint8 [ceil(N/16) * 16 * K] in the packed order."""
    w = np.asarray(w, dtype=np.uint8)
    n, k = w.shape
    if k % 128:
        raise ValueError("K must be a multiple of 128")
    t = (n + 15) // 16
    pad = np.zeros((t * 16, k), dtype=np.uint8)
    pad[:n] = w
    # row = 16 t + rr, column = 128 g + 32 q + 16 h + b  ->  [t, g, h, q, rr, b]
    v = pad.reshape(t, 16, k // 128, 4, 2, 16)
    return np.ascontiguousarray(v.transpose(0, 2, 4, 3, 1, 5)).reshape(-1)


def unpack_weight(p, n, k):
    """Inverse of pack_weight: packed bytes -> uint8 [N, K]."""
    t = (n + 15) // 16
    v = np.asarray(p, dtype=np.uint8)[: t * 16 * k].reshape(t, k // 128, 2, 4, 16, 16)
    return np.ascontiguousarray(v.transpose(0, 4, 1, 3, 2, 5)).reshape(t * 16, k)[:n]


def pack_experts(w):
    """uint8 [E, N, K] (K % 128 == 0) -> uint8 [E * ceil(N/16) * 16 * K], each expert panel-major."""
    w = np.asarray(w, dtype=np.uint8)
    e, n, k = w.shape
    t, g = (n + 15) // 16, k // 128
    out = []
    for i in range(e):
        blocks = pack_weight(w[i]).reshape(t, g, 2048)
        for p in range(0, t, 16):
            out.append(blocks[p:p + 16].transpose(1, 0, 2).reshape(-1))  # [g, tile of the panel, 2048]
    return np.concatenate(out)


def unpack_experts(p, e, n, k):
    """Inverse of pack_experts: packed bytes -> uint8 [E, N, K]."""
    t, g = (n + 15) // 16, k // 128
    per = t * g * 2048
    p = np.asarray(p, dtype=np.uint8)
    out = np.empty((e, n, k), dtype=np.uint8)
    for i in range(e):
        blocks = np.empty((t, g, 2048), dtype=np.uint8)
        at = i * per
        for p0 in range(0, t, 16):
            nbp = min(16, t - p0)
            blocks[p0:p0 + nbp] = p[at:at + nbp * g * 2048].reshape(g, nbp, 2048).transpose(1, 0, 2)
            at += nbp * g * 2048
        out[i] = unpack_weight(blocks.reshape(-1), n, k)
    return out
