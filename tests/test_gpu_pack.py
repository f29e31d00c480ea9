"""Load-time weight packing on the GPU (gk_fp8_pack_weight) and the GEMMs on packed weights.

The packed bytes equal oracle/pack.py; every GEMM on packed weights is bit-identical to the
same GEMM on the row-major codes (the decode kernel at one to four token tiles and the 256 x 256
kernel, both modes, bias, ragged N), and the row-major GEMM is pinned to the oracle by the golden
vectors (test_gpu_gemm.py).
"""

import numpy as np
import pytest
import torch

from gaudi_kernels import _native as nat
from gaudi_kernels import ops
from oracle import block_fp8, pack, synth

pytestmark = pytest.mark.gpu


def weights(n, k, seed):
    w, s = synth.weight(n, k, seed)
    return w.cuda(), s.cuda()


@pytest.mark.parametrize("n,k", [(6144, 4096), (1000, 256), (8, 128), (264, 1024)])
def test_pack_bytes(n, k):
    w, _ = weights(n, k, n)
    p = ops.pack_weight(w)
    assert p.shape == (n, k)
    want = pack.pack_weight(w.view(torch.uint8).cpu().numpy())
    assert np.array_equal(p.data.cpu().numpy(), want)


@pytest.mark.parametrize("e,n,k", [(1, 4096, 14336), (3, 264, 256), (2, 40, 384), (8, 768, 512), (2, 520, 128)])
def test_pack_experts_bytes(e, n, k):
    """gk_fp8_pack_experts (panel-major, all experts in one launch) equals oracle/pack.py."""
    w = torch.randint(0, 256, (e, n, k), dtype=torch.uint8, generator=torch.Generator().manual_seed(e * n + k))
    p = ops.pack_experts(w.cuda())
    assert p.shape == (e, n, k)
    assert np.array_equal(p.data.cpu().numpy(), pack.pack_experts(w.numpy()))


CASES = [(1, 6144, 4096), (5, 1000, 256), (16, 28672, 4096), (16, 4096, 14336), (17, 264, 1024),
         (40, 7168, 7168), (64, 6144, 4096), (33, 28672, 512), (100, 1000, 512), (300, 6144, 4096),
         (600, 520, 384)]


@pytest.mark.parametrize("m,n,k", CASES)
@pytest.mark.parametrize("native_half", [False, True])
def test_gemm_packed_bit_identical(m, n, k, native_half):
    w, s = weights(n, k, m + n)
    x = synth.activations(m, k, m).cuda()
    bias = torch.randn(n, device="cuda")
    p = ops.pack_weight(w)
    for b in (None, bias):
        y_row = ops.block_fp8_gemm(x, w, s, b, native_half=native_half)
        y_pack = ops.block_fp8_gemm(x, p, s, b, native_half=native_half)
        assert torch.equal(y_row.view(torch.int16), y_pack.view(torch.int16)), (m, n, k, b is None)


@pytest.mark.parametrize("m", [16, 32, 64])
def test_gemm_q_packed_decode_layout(m):
    n, k = 6144, 4096
    w, s = weights(n, k, 3)
    x = synth.activations(m, k, 3).cuda()
    q, sa = ops.act_quant(x, decode_layout=True)
    p = ops.pack_weight(w)
    y1 = ops.block_fp8_gemm_q(q, sa, m, w, s, decode_layout=True)
    y2 = ops.block_fp8_gemm_q(q, sa, m, p, s, decode_layout=True)
    assert torch.equal(y1.view(torch.int16), y2.view(torch.int16))


def test_packed_vs_oracle():
    m, n, k = 4, 256, 256
    w, s = weights(n, k, 0)
    x = synth.activations(m, k, 0)
    y = ops.block_fp8_gemm(x.cuda(), ops.pack_weight(w), s).cpu()
    ref = block_fp8.reference(x, w.cpu(), s.cpu())
    max_rel, mean_rel = block_fp8.parity(y, ref)
    assert max_rel <= block_fp8.MAX_REL_TOL and mean_rel <= block_fp8.MEAN_REL_TOL


def test_packed_rejections():
    w, s = weights(256, 256, 1)
    x = synth.activations(4, 256, 1).cuda()
    p = ops.pack_weight(w)
    with pytest.raises(nat.GkError):
        ops.block_fp8_gemm(x, p, s, variant="generic")
    with pytest.raises(nat.GkError):
        ops.pack_weight(torch.zeros(16, 200, dtype=torch.uint8, device="cuda"))
    small = ops.PackedWeight(p.data[:1024], 256, 256)
    with pytest.raises(ValueError):
        ops.block_fp8_gemm(x, small, s)
    with pytest.raises(nat.GkError):
        ops.pack_experts(torch.zeros(2, 16, 200, dtype=torch.uint8, device="cuda"))
    lib, buf = nat.load(), torch.empty(2 * 16 * 128, dtype=torch.uint8, device="cuda")
    src = torch.zeros(2, 16, 128, dtype=torch.uint8, device="cuda")
    assert lib.gk_fp8_pack_experts(src.data_ptr(), 2, 16, 128, buf.data_ptr(), buf.numel() - 1, None) \
        == nat.GK_INSUFFICIENT_BUFFER
    assert lib.gk_fp8_pack_experts(src.data_ptr(), 0, 16, 128, buf.data_ptr(), buf.numel(), None) \
        == nat.GK_INCOMPATIBLE_INPUT_SIZE
