"""GPU per-token / per-channel W8A8 path against oracle/token_channel.py.

Token quant (activation_token.c): codes and scales bit-exact.  Channel finish
(channel_finish.c): bf16 bits exact.  The fused per-token / per-channel GEMM (MME +
channel finish): within the GEMM gate (max|y - ref| <= 1e-2 max|ref|, sum|y - ref| /
sum|ref| <= 2e-3) of the oracle, whose fp32 product is the exact fp8 dot product
rounded once (the device sums in fp32 inside the matrix cores).
"""

import numpy as np
import pytest
import torch

from gaudi_kernels import ops
from oracle import block_fp8, e4m3, synth
from oracle import token_channel as tc

pytestmark = pytest.mark.gpu


def acts(m, k, seed):
    x = synth.activations(m, k, seed).float()
    if m > 2:
        x[1] = 0.0
        x[2] *= 1e-20
    return x.bfloat16()


@pytest.mark.parametrize("m,k", [(1, 128), (16, 4096), (37, 7168), (300, 256), (5, 14336)])
def test_token_quant_bit_exact(m, k):
    x = acts(m, k, m + k)
    q, s = ops.token_quant(x.cuda())
    want_q, want_s = tc.token_quant(x)
    assert np.array_equal(q.cpu().numpy(), want_q)
    assert np.array_equal(s.cpu().numpy().view(np.uint32), want_s.view(np.uint32))


def test_token_quant_strided():
    x = acts(9, 256, 3)
    wide = torch.zeros(9, 384, dtype=torch.bfloat16)
    wide[:, :256] = x
    qbuf = torch.full((9, 272), 0xAB, dtype=torch.uint8, device="cuda")
    q, s = ops.token_quant(wide.cuda()[:, :256], out=qbuf[:, :256])
    want_q, want_s = tc.token_quant(x)
    assert np.array_equal(qbuf[:, :256].cpu().numpy(), want_q)
    assert torch.all(qbuf[:, 256:].cpu() == 0xAB)


def test_channel_finish_bit_exact():
    gen = torch.Generator().manual_seed(5)
    p = torch.randn(7, 384, generator=gen) * 50
    a = torch.rand(7, generator=gen)
    w = torch.rand(384, generator=gen)
    b = torch.randn(384, generator=gen)
    for bias in (b, None):
        y = ops.channel_finish(p.cuda(), a.cuda(), w.cuda(), None if bias is None else bias.cuda()).cpu()
        want = tc.channel_finish(p.numpy(), a.numpy(), w.numpy(), None if bias is None else bias.numpy())
        assert np.array_equal(y.view(torch.int16).numpy().view(np.uint16), want)


def channel_weight(n, k, seed):
    """Per-output-channel E4M3 weights: s[n] = amax(row) / 448, codes = e4m3(w / s)."""
    gen = torch.Generator().manual_seed(seed)
    w = torch.randn(n, k, generator=gen) * 0.02
    s = w.abs().amax(1).clamp_min(1e-12) / 448.0
    return (w / s[:, None]).clamp(-448, 448).to(torch.float8_e4m3fn), s.float()


@pytest.mark.parametrize("m,n,k", [(1, 6144, 4096), (16, 4096, 14336), (5, 1000, 384), (17, 512, 256),
                                   (300, 768, 1024), (4096, 1024, 1024)])
def test_channel_gemm_vs_oracle(m, n, k):
    x = acts(m, k, 11 + m)
    w, sw = channel_weight(n, k, 12 + n)
    gen = torch.Generator().manual_seed(13)
    bias = torch.randn(n, generator=gen)
    q, sa = ops.token_quant(x.cuda())
    y = ops.channel_gemm(q, sa, w.cuda(), sw.cuda(), bias.cuda()).cpu()
    want_q, want_s = tc.token_quant(x)
    ref = tc.channel_reference(want_q, want_s, w.view(torch.uint8).numpy(), sw.numpy(), bias.numpy())
    ref_t = torch.from_numpy(ref.view(np.int16)).view(torch.bfloat16)
    max_rel, mean_rel = block_fp8.parity(y, ref_t)
    assert max_rel <= block_fp8.MAX_REL_TOL and mean_rel <= block_fp8.MEAN_REL_TOL, (max_rel, mean_rel)
    # and the W8A8 result tracks the bf16 product it approximates
    exact = (x.float() @ (w.float() * sw[:, None]).T + bias).double()
    rel = (y.double() - exact).abs().sum() / exact.abs().sum()
    assert float(rel) < 0.1


def test_channel_gemm_deterministic_and_rejects():
    x = acts(16, 4096, 1)
    w, sw = channel_weight(6144, 4096, 2)
    q, sa = ops.token_quant(x.cuda())
    y1 = ops.channel_gemm(q, sa, w.cuda(), sw.cuda())
    y2 = ops.channel_gemm(q, sa, w.cuda(), sw.cuda())
    assert torch.equal(y1.view(torch.int16), y2.view(torch.int16))
    with pytest.raises(ValueError):
        ops.channel_gemm(q, sa, w.cuda()[:, :2048], sw.cuda())
    with pytest.raises(Exception):
        ops.token_quant(torch.zeros(4, 100, dtype=torch.bfloat16, device="cuda"))  # width % 128


@pytest.mark.parametrize("m", [1, 2, 5, 8, 13, 16])
@pytest.mark.parametrize("n,k", [(6144, 4096), (200, 256), (1000, 768), (4096, 14336), (130, 128)])
def test_fused_token_channel_equals_two_ops(m, n, k):
    """gk_fp8_token_channel_gemm_bf16 (one launch) = token quant + channel GEMM, bit for bit."""
    x = acts(m, k, 31 * m + k).float()
    if m > 3:
        x[3] = -0.0  # an all-(-0) token: the zero-row denominator
        x[0, 5] = 3.0e38 if k > 128 else x[0, 5]  # a huge element
    x = x.bfloat16().cuda()
    w, sw = channel_weight(n, k, 40 + n)
    gen = torch.Generator().manual_seed(41)
    bias = torch.randn(n, generator=gen).cuda()
    wd, swd = w.cuda(), sw.cuda()
    for b in (bias, None):
        q, sa = ops.token_quant(x)
        want = ops.channel_gemm(q, sa, wd, swd, b)
        got = ops.token_channel_gemm(x, wd, swd, b, fused=True)
        assert torch.equal(got.view(torch.int16), want.view(torch.int16)), (m, n, k, b is None)


def test_fused_token_channel_strided_and_fallback():
    x = acts(20, 512, 7)
    wide = torch.zeros(20, 640, dtype=torch.bfloat16)
    wide[:, :512] = x
    xs = wide.cuda()[:, :512]  # row stride 640 elements
    w, sw = channel_weight(384, 512, 8)
    wd, swd = w.cuda(), sw.cuda()
    for m in (1, 16, 20):  # 20 rows: token quant + channel GEMM
        q, sa = ops.token_quant(xs[:m])
        want = ops.channel_gemm(q, sa, wd, swd)
        for fused in (None, True):
            got = ops.token_channel_gemm(xs[:m], wd, swd, fused=fused)
            assert torch.equal(got.view(torch.int16), want.view(torch.int16)), (m, fused)
