"""Decode GEMM with the 1x128 quantizer fused into its activation load (gk_fp8_block_gemm_bf16, M <= 16).

The op fuses the quantizer where its redundant per-workgroup work is small (N = 6144, K = 4096
at every M <= 16; 7168 x 7168 at M <= 12; 28672 x 4096 and 4096 x 14336 at M <= 4; small shapes
at every M) and runs the standalone quantizer otherwise.  Either way it must equal
act_quant followed by the GEMM on the quantized activations bit for bit (same codes, same scales,
same accumulation order), for row-major and packed weights, both modes, with bias, M values that
leave 1-3 clamped rows in a row quad, padded row strides, and activations that are not 16-byte
aligned (always unfused).  The unfused path is pinned to the oracle by the golden vectors.
"""

import pytest
import torch

from gaudi_kernels import ops
from oracle import block_fp8, synth

pytestmark = pytest.mark.gpu


def unfused(x, w, s, bias, native_half):
    q, sa = ops.act_quant(x, native_half=native_half, decode_layout=True)
    return ops.block_fp8_gemm_q(q, sa, x.shape[0], w, s, bias, native_half=native_half, decode_layout=True)


# every fused load step: (NW, R, U) = (8, 2, 4), (8, 1, 2), (2, 2, 2), (16, 1, 1), (8, 2, 1), (8, 1, 1)
@pytest.mark.parametrize("n,k", [(6144, 4096), (4096, 14336), (28672, 4096), (1000, 384), (24, 128), (7168, 7168),
                                 (4096, 7168)])
@pytest.mark.parametrize("native_half", [False, True])
def test_fused_equals_quant_then_gemm(n, k, native_half):
    w, s = synth.weight(n, k, seed=n + k)
    w, s = w.cuda(), s.cuda()
    p = ops.pack_weight(w)
    bias = torch.randn(n, device="cuda")
    for m in (1, 3, 5, 8, 16):
        x = synth.activations(m, k, seed=m).cuda()
        x[0, :128] = 0.0                       # an all-zero group
        x[-1, 130:140] = -0.0                  # negative zeros in a live group (code 0x80)
        if m > 1:
            x[1, 128:256] *= 1e-30             # a tiny group
        for weight in (w, p):
            for b in (None, bias):
                want = unfused(x, weight, s, b, native_half)
                got = ops.block_fp8_gemm(x, weight, s, b, native_half=native_half)
                assert torch.equal(got.view(torch.int16), want.view(torch.int16)), (m, n, k, b is None)


def test_fused_strided_and_unaligned_rows():
    n, k, m = 6144, 4096, 5
    w, s = synth.weight(n, k, seed=9)
    w, s = w.cuda(), s.cuda()
    x = synth.activations(m, k, seed=9).cuda()
    want = unfused(x, w, s, None, False)
    wide = torch.zeros(m, k + 64, dtype=torch.bfloat16, device="cuda")
    wide[:, :k] = x
    assert torch.equal(ops.block_fp8_gemm(wide[:, :k], w, s).view(torch.int16), want.view(torch.int16))
    off = torch.zeros(m * k + 3, dtype=torch.bfloat16, device="cuda")
    xu = off[3:].view(m, k)                    # 6-byte offset rows: the unfused path
    xu.copy_(x)
    assert torch.equal(ops.block_fp8_gemm(xu, w, s).view(torch.int16), want.view(torch.int16))


def test_fused_golden_config1():
    x, w, s = synth.config1()
    y = ops.block_fp8_gemm(x.cuda(), w.cuda(), s.cuda()).cpu()
    ref = block_fp8.reference(x, w, s)
    max_rel, mean_rel = block_fp8.parity(y, ref)
    assert max_rel <= block_fp8.MAX_REL_TOL and mean_rel <= block_fp8.MEAN_REL_TOL
