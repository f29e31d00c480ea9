"""GPU activation quantization is bit-exact with the oracle (block_fp8_oracle.py:25-28, :31-34)."""

import pytest
import torch

from gaudi_kernels import ops
from oracle import block_fp8

pytestmark = pytest.mark.gpu


def make_x(m, k, seed, kind):
    gen = torch.Generator().manual_seed(seed)
    x = torch.randn(m, k, generator=gen)
    if kind == "outliers":
        cols = torch.randperm(k, generator=gen)[: max(1, k // 100)]
        x[:, cols] *= 20
    elif kind == "mixed":
        x[0, :min(k, 128)] = 0                       # all-zero group
        if m > 1:
            x[1] *= 1e-30                            # tiny row (bf16 keeps it)
        if m > 2:
            x[2] *= 1e30                             # huge row
        if m > 3:
            x[3, ::7] = 0
            x[3, 3::7] = -0.0                        # negative zeros encode to 0x80
    return x.bfloat16()


@pytest.mark.parametrize("m,k", [(1, 4096), (16, 4096), (5, 333), (37, 384), (300, 7168), (2, 14336)])
@pytest.mark.parametrize("kind", ["outliers", "mixed"])
@pytest.mark.parametrize("native_half", [False, True])
def test_act_quant_bit_exact(m, k, kind, native_half):
    x = make_x(m, k, m * 1000 + k, kind)
    m_pad = m + 3
    q, sa = ops.act_quant(x.cuda(), native_half=native_half, m_pad=m_pad)
    want_q, want_sa = block_fp8.act_quant(x, native_half)
    g = (k + 127) // 128
    assert q.shape == (g, m_pad, 128) and sa.shape == (g, m_pad)    # group-major
    q_rows = q.permute(1, 0, 2).reshape(m_pad, g * 128).cpu()
    sa_rows = sa.t().cpu()
    assert torch.equal(q_rows[:m], want_q)
    assert torch.equal(sa_rows[:m].contiguous().view(torch.int32), want_sa.contiguous().view(torch.int32))
    assert int(q_rows[m:].abs().sum()) == 0 and float(sa_rows[m:].abs().sum()) == 0.0


def test_strided_rows():
    x = make_x(8, 1024, 5, "outliers")
    wide = torch.zeros(8, 1536, dtype=torch.bfloat16)
    wide[:, :1024] = x
    q, sa = ops.act_quant(wide.cuda()[:, :1024], m_pad=8)
    want_q, want_sa = block_fp8.act_quant(x)
    assert torch.equal(q.permute(1, 0, 2).reshape(8, 1024).cpu(), want_q) and torch.equal(sa.t().cpu(), want_sa)


@pytest.mark.parametrize("m,k", [(1, 4096), (5, 333), (16, 14336), (16, 128), (17, 1024), (33, 384), (64, 256)])
@pytest.mark.parametrize("native_half", [False, True])
def test_act_quant_decode_layout(m, k, native_half):
    """The decode fragment layout holds the same codes as the standard layout, placed as include/gk_fp8.h says:
    block (group g, token tile t) at (g * m_pad/16 + t) * 2048, piece (h, l) at + h*1024 + 16 l = bytes
    [32 (l // 16) + 16 h, +16) of row 16 t + l % 16; m_pad = 16, 32 or 64 by M."""
    x = make_x(m, k, m * 7 + k, "outliers").cuda()
    qp, sap = ops.act_quant(x, native_half=native_half, decode_layout=True)
    m_pad = 16 * ops.decode_tiles(m)
    qs, sas = ops.act_quant(x, native_half=native_half, m_pad=m_pad)
    assert qp.shape == qs.shape == ((k + 127) // 128, m_pad, 128)
    assert torch.equal(sap.cpu().view(torch.int32), sas.cpu().view(torch.int32))
    flat_p = qp.reshape(-1).cpu()
    std = qs.cpu()
    g_n, tiles = std.shape[0], m_pad // 16
    for g in range(g_n):
        for t in range(tiles):
            for h in range(2):
                for lane in range(64):
                    row, quad = 16 * t + lane % 16, lane // 16
                    at = (g * tiles + t) * 2048 + h * 1024 + 16 * lane
                    assert torch.equal(flat_p[at:at + 16], std[g, row, 32 * quad + 16 * h: 32 * quad + 16 * h + 16])
    assert torch.equal(ops.decode_layout_to_standard(qp).cpu(), std)
    want_q, _ = block_fp8.act_quant(x.cpu(), native_half)
    assert torch.equal(std.permute(1, 0, 2).reshape(m_pad, -1)[:m], want_q)
