"""GPU SiLU-and-mul (gk_silu_and_mul_bf16, the reference's gk_silu_and_mul_bf16_v1,
csrc/tpc/generic_dense/silu_and_mul_bf16.c) and its fusion with the 1x128 quantizer
(gk_fp8_silu_mul_quant_bf16) against oracle/moe.py.

The bf16 products come from fp32 exp and division on both sides; where the two fp32
values straddle a bf16 rounding boundary they differ by one bf16 ulp, so the plain op
is checked as: special values bit-exact, every element within one bf16 ulp, and
almost all (>= 1 - 1e-4) bit-exact.  The fused op must equal the composition of the
two GPU ops bit for bit, in both layouts and both modes.
"""

import pytest
import torch

from gaudi_kernels import ops
from oracle import block_fp8, moe

pytestmark = pytest.mark.gpu


def gate_up(rows, width, seed):
    gen = torch.Generator().manual_seed(seed)
    x = torch.randn(rows, 2 * width, generator=gen) * 3
    x[:, : max(1, width // 64)] *= 30      # some large gates (silu(g) ~ g, e^-g underflows)
    return x.bfloat16()


def bf16_ulp_diff(a, b):
    ai, bi = a.view(torch.int16).int(), b.view(torch.int16).int()
    return (ai - bi).abs()


@pytest.mark.parametrize("rows,width", [(1, 128), (37, 14336), (5, 333), (256, 1024), (3, 7)])
def test_silu_and_mul_vs_oracle(rows, width):
    x = gate_up(rows, width, rows * 31 + width)
    y = ops.silu_and_mul(x.cuda()).cpu()
    ref = moe.silu_mul(x)
    assert y.shape == ref.shape == (rows, width)
    d = bf16_ulp_diff(y, ref)
    same_sign = (y.float() * ref.float() >= 0) | (y == 0) | (ref == 0)
    assert bool(same_sign.all())
    assert int(d.max()) <= 1, int(d.max())
    assert float((d != 0).float().mean()) <= 1e-4


def test_silu_and_mul_special_values():
    inf, nan = float("inf"), float("nan")
    g = torch.tensor([0.0, -0.0, -88.0, -100.0, 88.5, 1e-30, -1e-30, 200.0, inf, -inf, nan, 3.0, -87.5, 1.0])
    u = torch.tensor([2.0, 2.0, 5.0, 5.0, 1.0, 1.0, 1.0, -2.0, 1.0, 1.0, 1.0, nan, 1e30, 0.0])
    x = torch.cat([g, u]).reshape(1, -1).bfloat16()
    y = ops.silu_and_mul(x.cuda()).cpu().float()[0]
    ref = moe.silu_mul(x).float()[0]
    assert torch.equal(torch.isnan(y), torch.isnan(ref)), (y, ref)
    ok = torch.isnan(ref) | (y == ref)
    assert bool(ok.all()), (y, ref)
    assert torch.isnan(y[8]) and y[9] == 0 and torch.isnan(y[10]) and torch.isnan(y[11])


def test_silu_and_mul_strided():
    x = gate_up(9, 256, 4)
    wide = torch.zeros(9, 640, dtype=torch.bfloat16)
    wide[:, :512] = x
    out = torch.full((9, 264), 3.0, dtype=torch.bfloat16, device="cuda")
    ops.silu_and_mul(wide.cuda()[:, :512], out=out[:, :256])
    torch.cuda.synchronize()
    assert torch.equal(out[:, :256].cpu(), ops.silu_and_mul(x.cuda()).cpu())
    assert torch.all(out[:, 256:].cpu() == 3.0)


@pytest.mark.parametrize("rows,width", [(1, 4096), (16, 14336), (5, 333), (300, 1024), (40, 1024)])
@pytest.mark.parametrize("native_half", [False, True])
def test_silu_mul_quant_equals_composition(rows, width, native_half):
    xg = gate_up(rows, width, rows + width).cuda()
    h = ops.silu_and_mul(xg)
    m_pad = rows + 3
    q1, s1 = ops.silu_mul_quant(xg, native_half=native_half, m_pad=m_pad)
    q2, s2 = ops.act_quant(h, native_half=native_half, m_pad=m_pad)
    torch.cuda.synchronize()
    assert torch.equal(q1.cpu(), q2.cpu())
    assert torch.equal(s1.cpu().view(torch.int32), s2.cpu().view(torch.int32))
    if rows <= 64:
        p1, t1 = ops.silu_mul_quant(xg, native_half=native_half, decode_layout=True)
        p2, t2 = ops.act_quant(h, native_half=native_half, decode_layout=True)
        assert torch.equal(p1.cpu(), p2.cpu()) and torch.equal(t1.cpu(), t2.cpu())


def test_silu_mul_quant_vs_oracle_and_gemm():
    """Codes against the oracle chain (act_quant of the oracle's products), then the down GEMM on them."""
    rows, width, n = 12, 1024, 512
    x = gate_up(rows, width, 99)
    q, sa = ops.silu_mul_quant(x.cuda(), m_pad=16, decode_layout=True)
    want_codes, want_sa = block_fp8.act_quant(moe.silu_mul(x))
    got = ops.decode_layout_to_standard(q).cpu().permute(1, 0, 2).reshape(16, -1)[:rows]
    assert float((got != want_codes).float().mean()) <= 1e-3
    from oracle import synth
    w, s = synth.weight(n, width, seed=7)
    y = ops.block_fp8_gemm_q(q, sa, rows, w.cuda(), s.cuda(), decode_layout=True).cpu()
    ref = block_fp8.reference(moe.silu_mul(x), w, s)
    max_rel, mean_rel = block_fp8.parity(y, ref)
    assert max_rel <= block_fp8.MAX_REL_TOL and mean_rel <= block_fp8.MEAN_REL_TOL


def test_silu_rejects_bad_shapes():
    with pytest.raises(ValueError):
        ops.silu_and_mul(torch.zeros(3, 7, dtype=torch.bfloat16, device="cuda"))
    with pytest.raises(ValueError):
        ops.silu_and_mul(torch.zeros(3, 8, dtype=torch.float32, device="cuda"))
