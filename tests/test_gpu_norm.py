"""RMSNorm ops on the GPU (gk_rms_norm_bf16, gk_fused_add_rms_norm_bf16, gk_fp8_rms_norm_quant_bf16).

* Bit for bit against the CPU restatement (oracle/norm.py), which fixes the sum and inverse roundings the same
  way, at widths 1..8192, ragged and strided rows, weight_offset 0 / 1 / negative.
* The reference's own gate on its own inputs (tests/track_a_device_verify.cpp:465-540): residual_out exact,
  norm_out within 2 bf16 ulps of an fp64 evaluation.
* The fused quantizer: codes and scales equal act_quant of the bf16 norm output in both layouts and modes; the
  decode GEMM on them equals the op on the normalized rows.
* The glue's rejections (generic_dense_glue.cpp:146-160).
"""

import ctypes

import pytest
import torch

from gaudi_kernels import _native as nat
from gaudi_kernels import ops
from oracle import norm, synth

pytestmark = pytest.mark.gpu


def rows_of(rows, width, seed, scale=1.0):
    gen = torch.Generator().manual_seed(seed)
    return (torch.randn(rows, width, generator=gen) * scale).bfloat16()


def gamma_of(width, seed):
    gen = torch.Generator().manual_seed(seed)
    return (torch.rand(width, generator=gen) * 1.5 - 0.25).bfloat16()


def same(a, b):
    return torch.equal(a.cpu().view(torch.int16), b.cpu().view(torch.int16))


@pytest.mark.parametrize("rows,width", [(1, 1), (5, 7), (3, 64), (5, 576), (17, 1000), (2, 4096), (4, 8192),
                                        (1, 8191), (33, 2048)])
@pytest.mark.parametrize("offset", [0.0, 1.0, -0.25])
def test_bit_exact_vs_restatement(rows, width, offset):
    x = rows_of(rows, width, rows * 100 + width, 3.0)
    res = rows_of(rows, width, rows * 100 + width + 1)
    g = gamma_of(width, width)
    eps = 1e-5
    got = ops.rms_norm(x.cuda(), g.cuda(), eps, offset)
    assert same(got, norm.rms_norm(x, g, eps, offset)), (rows, width, offset)
    r, n = ops.fused_add_rms_norm(x.cuda(), res.cuda(), g.cuda(), eps, offset)
    want_r, want_n = norm.fused_add_rms_norm(x, res, g, eps, offset)
    assert same(r, want_r) and same(n, want_n), (rows, width, offset)


@pytest.mark.parametrize("width", [64, 576])
@pytest.mark.parametrize("offset", [0.0, 1.0])
def test_reference_gate_on_its_inputs(width, offset):
    x, res, g = norm.reference_test_inputs(width)
    eps = 1e-5
    out = ops.rms_norm(x.cuda(), g.cuda(), eps, offset).cpu()
    ref = torch.from_numpy(norm.fp64_reference(x, g, eps, offset).astype("float32")).to(torch.bfloat16)
    assert int(norm.bf16_ulp_diff(out, ref).max()) <= norm.GATE_ULPS
    r, n = ops.fused_add_rms_norm(x.cuda(), res.cuda(), g.cuda(), eps, offset)
    assert same(r, (x.float() + res.float()).bfloat16())
    ref = torch.from_numpy(norm.fp64_reference(r.cpu(), g, eps, offset).astype("float32")).to(torch.bfloat16)
    assert int(norm.bf16_ulp_diff(n.cpu(), ref).max()) <= norm.GATE_ULPS


def test_strided_and_unaligned_rows():
    rows, width = 6, 1000
    base = rows_of(rows, width + 5, 11)
    x = base.cuda()[:, 1:width + 1]          # row stride width + 5, data 2 bytes past 16-byte alignment
    xc = x.contiguous()
    g = gamma_of(width, 12).cuda()
    assert same(ops.rms_norm(x, g, 1e-6, 1.0), ops.rms_norm(xc, g, 1e-6, 1.0))
    rbase = rows_of(rows, width + 5, 13).cuda()
    r = rbase[:, 1:width + 1]
    a = ops.fused_add_rms_norm(x, r, g, 1e-6, 0.0)
    b = ops.fused_add_rms_norm(xc, r.contiguous(), g, 1e-6, 0.0)
    assert same(a[0], b[0]) and same(a[1], b[1])
    # padded output stride leaves the padding alone
    buf = torch.full((rows, width + 8), 7.0, dtype=torch.bfloat16, device="cuda")
    ops.rms_norm(xc, g, 1e-6, 0.0, out=buf[:, :width])
    assert bool((buf[:, width:] == 7.0).all())


def test_special_rows():
    width = 256
    g = torch.ones(width).bfloat16()
    x = torch.zeros(4, width)
    x[1, 3] = 3.0e38                            # sum of squares overflows fp32: inverse 0 (norm_math.h:22)
    x[2] = 1e-30                                # tiny row: epsilon dominates
    x[3, ::2] = -0.0
    x = x.bfloat16()
    got = ops.rms_norm(x.cuda(), g.cuda(), 1e-5, 0.0)
    assert same(got, norm.rms_norm(x, g, 1e-5, 0.0))
    assert float(got[1, 3]) == 0.0 and float(got[1, 0]) == 0.0


@pytest.mark.parametrize("rows,width", [(1, 4096), (5, 333), (16, 7168), (40, 1000), (64, 256), (300, 2048)])
@pytest.mark.parametrize("native_half", [False, True])
def test_norm_quant_equals_composition(rows, width, native_half):
    x = rows_of(rows, width, rows + width, 2.0).cuda()
    res = rows_of(rows, width, rows + width + 1).cuda()
    g = gamma_of(width, width + 3).cuda()
    n = ops.rms_norm(x, g, 1e-6, 1.0)
    m_pad = rows + 5
    q1, s1 = ops.rms_norm_quant(x, g, 1e-6, 1.0, native_half=native_half, m_pad=m_pad)
    q2, s2 = ops.act_quant(n, native_half=native_half, m_pad=m_pad)
    assert torch.equal(q1.cpu(), q2.cpu())
    assert torch.equal(s1.cpu().view(torch.int32), s2.cpu().view(torch.int32))
    r, nr = ops.fused_add_rms_norm(x, res, g, 1e-6, 1.0)
    q3, s3, r3 = ops.rms_norm_quant(x, g, 1e-6, 1.0, residual=res, native_half=native_half, m_pad=m_pad)
    q4, s4 = ops.act_quant(nr, native_half=native_half, m_pad=m_pad)
    assert same(r3, r)
    assert torch.equal(q3.cpu(), q4.cpu()) and torch.equal(s3.cpu().view(torch.int32), s4.cpu().view(torch.int32))
    if rows <= 64:
        p1, t1 = ops.rms_norm_quant(x, g, 1e-6, 1.0, native_half=native_half, decode_layout=True)
        p2, t2 = ops.act_quant(n, native_half=native_half, decode_layout=True)
        assert torch.equal(p1.cpu(), p2.cpu()) and torch.equal(t1.cpu().view(torch.int32), t2.cpu().view(torch.int32))


@pytest.mark.parametrize("m", [1, 16, 48])
def test_decode_gemm_on_norm_codes(m):
    """The QKV chain: normalized and quantized rows fed to the decode GEMM equal the op on the bf16 norm output."""
    k, n = 4096, 6144
    x = rows_of(m, k, m, 2.0).cuda()
    res = rows_of(m, k, m + 1).cuda()
    g = gamma_of(k, 5).cuda()
    w, s = synth.weight(n, k, seed=2000)
    p = ops.pack_weight(w.cuda())
    q, sa, r = ops.rms_norm_quant(x, g, 1e-6, 0.0, residual=res, decode_layout=True)
    y1 = ops.block_fp8_gemm_q(q, sa, m, p, s.cuda(), decode_layout=True)
    _, nrm = ops.fused_add_rms_norm(x, res, g, 1e-6, 0.0)
    y2 = ops.block_fp8_gemm(nrm, p, s.cuda())
    assert same(y1, y2)


def test_rejections():
    lib = nat.load()
    fake = ctypes.c_void_p(1 << 20)
    f = ctypes.c_float
    # epsilon <= 0, non-finite epsilon or offset: unsupported configuration (generic_dense_glue.cpp:150-152)
    for eps, off in ((0.0, 0.0), (-1e-5, 0.0), (float("inf"), 0.0), (1e-5, float("nan"))):
        assert lib.gk_rms_norm_bf16(fake, 4, 64, 64, fake, f(eps), f(off), fake, 64, None) == \
            nat.GK_UNSUPPORTED_LAYER_CONFIGURATION
    # width 0 or > 8192, rows 0, short row stride: input size (:153-155)
    for rows, width, ld in ((4, 0, 64), (4, 8193, 8193), (0, 64, 64), (4, 64, 32)):
        assert lib.gk_rms_norm_bf16(fake, rows, width, ld, fake, f(1e-5), f(0.0), fake, 64, None) == \
            nat.GK_INCOMPATIBLE_INPUT_SIZE
    assert lib.gk_rms_norm_bf16(fake, 4, 64, 64, fake, f(1e-5), f(0.0), fake, 32, None) == \
        nat.GK_INCOMPATIBLE_OUTPUT_SIZE
    assert lib.gk_rms_norm_bf16(ctypes.c_void_p((1 << 20) + 1), 4, 64, 64, fake, f(1e-5), f(0.0), fake, 64,
                                None) == nat.GK_INCOMPATIBLE_DATA_TYPE
    assert lib.gk_fused_add_rms_norm_bf16(fake, None, 4, 64, 64, fake, f(1e-5), f(0.0), fake, fake, 64, None) == \
        nat.GK_INVALID_ARGUMENT
    # quant: decode layout needs m_pad 16, 32 or 64
    assert lib.gk_fp8_rms_norm_quant_bf16(fake, None, 4, 256, 256, fake, f(1e-5), f(0.0), None, 0, fake, fake, 20,
                                          nat.GK_FLAG_DECODE_LAYOUT, None) == nat.GK_INCOMPATIBLE_OUTPUT_SIZE
    with pytest.raises(ValueError):
        ops.rms_norm(torch.zeros(2, 8, device="cuda"), torch.ones(8, device="cuda").bfloat16())
