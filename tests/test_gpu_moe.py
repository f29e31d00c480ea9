"""GPU block-FP8 MoE layer (gk_fp8_moe_route / gk_fp8_moe_bf16) against oracle/moe.py.

Routing and the expert-sorted row layout are integer/index work: ids,
row_token, row_of and offsets must be bit-exact; the two softmax weights are
fp32 and within a few ulp (the device exp).  The layer output must meet the GEMM
gate (max|y - ref| <= 1e-2 max|ref|, sum|y - ref| / sum|ref| <= 2e-3) at
small sizes in full and at BASELINE.json config 5 (512 tokens, 8 experts, top-2,
H=4096, I=14336) stage by stage on every routed row and end to end on all 512
tokens within the chain bound below, plus the size-independent property that
permuting tokens permutes the output bit-for-bit (every row's arithmetic is
independent of the other rows).
"""

import numpy as np
import pytest
import torch

from gaudi_kernels import _native as nat
from gaudi_kernels import ops
from oracle import block_fp8, moe, synth

pytestmark = pytest.mark.gpu

# End-to-end bound for the two-GEMM chain at config 5.  The GEMM gate holds per
# stage (test_moe_config5_stagewise_parity: each GEMM against the oracle fed
# the device's own input, max 6e-3 / mean 5e-5 measured).  End to end, a one-ulp
# bf16 difference in the gate_up output flips ~6% of the affected E4M3 codes of
# the requantized intermediate (relative step 6-12%), and those flips sum over
# K = 14336 in the down GEMM: measured max 1.628e-2 / mean 1.628e-3 on this
# input (the kernels are deterministic, so this is the one value), inside the
# GEMM gate's mean bound and 1.6x its max bound.  The bound sits just above it,
# so a regression shows.
CHAIN_MAX_REL = 2e-2
CHAIN_MEAN_REL = 2e-3


def check_routing(logits, top_k):
    ids, wts, row_of, row_token, off = ops.moe_route(logits.cuda(), top_k)
    torch.cuda.synchronize()
    ids_ref, w_ref = moe.route(logits.numpy(), top_k)
    rt_ref, _, ro_ref, off_ref, _ = moe.layout(ids_ref, logits.shape[1], 256)
    assert np.array_equal(ids.cpu().numpy(), ids_ref)
    np.testing.assert_allclose(wts.cpu().numpy(), w_ref, rtol=5e-7, atol=0)
    assert np.array_equal(off.cpu().numpy(), off_ref)
    rt = row_token.cpu().numpy()
    assert np.array_equal(rt[: len(rt_ref)], rt_ref)
    assert np.all(rt[len(rt_ref):] == -1)
    assert np.array_equal(row_of.cpu().numpy(), ro_ref)


@pytest.mark.parametrize("t,e,k", [(512, 8, 2), (1, 8, 2), (37, 3, 1), (1000, 256, 2), (3000, 64, 2),
                                   (2048, 2, 2), (5, 1, 1)])
def test_routing_bit_exact(t, e, k):
    gen = torch.Generator().manual_seed(t + e)
    check_routing(torch.randn(t, e, generator=gen), k)


def test_routing_ties_and_skew():
    gen = torch.Generator().manual_seed(9)
    lg = torch.randint(-2, 3, (700, 6), generator=gen).float()   # ties everywhere
    check_routing(lg, 2)
    lg = torch.randn(900, 16, generator=gen)
    lg[:, 3] += 10.0                                              # every token picks expert 3
    check_routing(lg, 2)


def test_routing_oversized_row_buffer_fully_defined():
    # row_token larger than gk_fp8_moe_rows_max: every entry past the layout reads -1
    import ctypes
    t, e, k = 300, 8, 2
    logits = torch.randn(t, e, generator=torch.Generator().manual_seed(11))
    rows = ops.moe_rows_max(t, e, k)
    extra = 3000
    dev = torch.device("cuda")
    lg = logits.to(dev)
    ids = torch.empty((t, k), dtype=torch.int32, device=dev)
    wts = torch.empty((t, k), dtype=torch.float32, device=dev)
    row_of = torch.empty((t, k), dtype=torch.int32, device=dev)
    row_token = torch.full((rows + extra,), 0x5A5A5A5A, dtype=torch.int32, device=dev)
    off = torch.empty(e + 1, dtype=torch.int32, device=dev)
    p = lambda x: ctypes.c_void_p(x.data_ptr())
    st = nat.load().gk_fp8_moe_route(p(lg), t, e, e, k, p(ids), p(wts), p(row_of), p(row_token), rows + extra,
                                     p(off), ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
    assert st == nat.GK_SUCCESS
    ids_ref, _ = moe.route(logits.numpy(), k)
    rt_ref, _, _, _, _ = moe.layout(ids_ref, e, 256)
    rt = row_token.cpu().numpy()
    assert np.array_equal(rt[: len(rt_ref)], rt_ref)
    assert np.all(rt[len(rt_ref):] == -1)


def problem(t, h, inter, e, seed, device="cpu"):
    x = synth.activations(t, h, seed)
    gen = torch.Generator().manual_seed(seed + 1)
    logits = torch.randn(t, e, generator=gen)
    wg, sg, wd, sd = [], [], [], []
    for i in range(e):
        a, b = synth.weight(2 * inter, h, seed=seed + 10 + i, device=device)
        c, d = synth.weight(h, inter, seed=seed + 1000 + i, device=device)
        wg.append(a); sg.append(b); wd.append(c); sd.append(d)
    return x, logits, torch.stack(wg), torch.stack(sg), torch.stack(wd), torch.stack(sd)


def run(x, logits, wg, sg, wd, sd, **kw):
    return ops.moe_block_fp8(x.cuda(), logits.cuda(), wg.cuda(), sg.cuda(), wd.cuda(), sd.cuda(), **kw)


@pytest.mark.parametrize("t,h,inter,e,k", [(64, 256, 384, 4, 2), (200, 512, 256, 8, 2), (3, 384, 128, 8, 2),
                                           (300, 256, 128, 3, 1), (1, 128, 128, 2, 2)])
@pytest.mark.parametrize("native_half", [False, True])
def test_moe_small_full_parity(t, h, inter, e, k, native_half):
    x, logits, wg, sg, wd, sd = problem(t, h, inter, e, seed=t + h + e)
    y = run(x, logits, wg, sg, wd, sd, top_k=k, native_half=native_half).cpu()
    ref = moe.moe_reference(x, logits, wg, sg, wd, sd, top_k=k, native_half=native_half)
    max_rel, mean_rel = block_fp8.parity(y, ref)
    assert max_rel <= block_fp8.MAX_REL_TOL and mean_rel <= block_fp8.MEAN_REL_TOL, (max_rel, mean_rel)


@pytest.mark.parametrize("t,h,inter,e,k", [(300, 512, 384, 4, 2), (200, 384, 256, 3, 2)])
@pytest.mark.parametrize("native_half", [False, True])
def test_moe_packed_experts_bit_identical(t, h, inter, e, k, native_half):
    """Expert weights packed at load time (pack_experts) give the row-major layer's bits; H = 384 leaves
    the down GEMM a last weight panel of 8 tiles."""
    gen = torch.Generator().manual_seed(41)
    x = synth.activations(t, h, seed=42).cuda()
    logits = torch.randn(t, e, generator=gen).cuda()
    wg, sg, wd, sd = [], [], [], []
    for i in range(e):
        a, b = synth.weight(2 * inter, h, seed=50 + i, device="cuda")
        c, d = synth.weight(h, inter, seed=60 + i, device="cuda")
        wg.append(a); sg.append(b); wd.append(c); sd.append(d)
    wg, sg, wd, sd = torch.stack(wg), torch.stack(sg), torch.stack(wd), torch.stack(sd)
    y_row = ops.moe_block_fp8(x, logits, wg, sg, wd, sd, top_k=k, native_half=native_half)
    y_pack = ops.moe_block_fp8(x, logits, ops.pack_experts(wg), sg, ops.pack_experts(wd), sd, top_k=k,
                               native_half=native_half)
    assert torch.equal(y_row.view(torch.int16), y_pack.view(torch.int16))
    with pytest.raises(ValueError):
        ops.moe_block_fp8(x, logits, ops.pack_experts(wg), sg, wd, sd, top_k=k)


def test_moe_strided_output_and_reuse():
    x, logits, wg, sg, wd, sd = problem(96, 256, 256, 4, seed=77)
    xs = torch.zeros(96, 384, dtype=torch.bfloat16)
    xs[:, :256] = x
    out = torch.full((96, 264), 7.0, dtype=torch.bfloat16, device="cuda")
    ws = torch.empty(ops.moe_workspace_bytes(96, 256, 256, 4, 2), dtype=torch.uint8, device="cuda")
    ws.fill_(0xAB)  # stale workspace contents must not matter
    y1 = run(xs[:, :256], logits, wg, sg, wd, sd, out=out[:, :256], workspace=ws)
    y2 = run(x, logits, wg, sg, wd, sd, workspace=ws)
    torch.cuda.synchronize()
    assert torch.equal(y1.cpu(), y2.cpu())
    assert torch.all(out[:, 256:].cpu() == 7.0)


def regions(ws, t, h, inter, e, k):
    """Views of the workspace regions documented for gk_fp8_moe_bf16 (include/gk_fp8.h)."""
    rows = ops.moe_rows_max(t, e, k)
    parts = 2 if (rows // 256) * ((h + 255) // 256) < 512 else 1
    sizes = [("ids", t * k * 4), ("wts", t * k * 4), ("row_of", t * k * 4), ("row_token", rows * 4),
             ("off", (e + 1) * 4), ("cnt", e * 4), ("q1", rows * h), ("sa1", rows * h // 128 * 4),
             ("q2", rows * inter), ("sa2", rows * inter // 128 * 4), ("z", parts * rows * h * 4)]
    out, at = {}, 0
    for name, nbytes in sizes:
        out[name] = ws[at:at + nbytes]
        at += (nbytes + 255) // 256 * 256
    assert at == ops.moe_workspace_bytes(t, h, inter, e, k)
    v = {n: out[n].view(torch.int32) for n in ("ids", "row_of", "row_token", "off", "cnt")}
    v["wts"] = out["wts"].view(torch.float32)
    v["q1"] = out["q1"].reshape(h // 128, rows, 128)
    v["sa1"] = out["sa1"].view(torch.float32).reshape(h // 128, rows)
    v["q2"] = out["q2"].reshape(inter // 128, rows, 128)
    v["sa2"] = out["sa2"].view(torch.float32).reshape(inter // 128, rows)
    zp = out["z"].view(torch.float32).reshape(parts, rows, h)
    z = zp[0].clone()
    for p in range(1, parts):
        z = z + zp[p]                     # fp32, as the combine does
    v["z"] = z.to(torch.bfloat16)
    v["zp"] = zp.clone()                  # the fp32 planes themselves
    v["parts"] = torch.tensor(parts)
    return {n: x.cpu() for n, x in v.items()}


def separate_chain_check(r, rows, w_gu, s_gu, h, inter, native_half=False):
    """The layer's SiLU-and-mul codes and scales on `rows` (one expert's routed rows) against the
    separate chain on the layer's own gathered codes: the dense 256 x 256 GEMM (forced at any row
    count), then the SiLU-and-mul quantizer.  Bit-identical: the dense and grouped forms of that
    kernel give each output element the same arithmetic.  Returns the chain's gate_up output (device)."""
    n = len(rows)
    m_pad = ops.plan(n, 2 * inter, h, nat.GK_FLAG_FORCE_PREFILL)[1]
    q1 = torch.zeros((h // 128, m_pad, 128), dtype=torch.uint8)
    sa1 = torch.zeros((h // 128, m_pad), dtype=torch.float32)
    q1[:, :n], sa1[:, :n] = r["q1"][:, rows], r["sa1"][:, rows]
    gate_up = ops.block_fp8_gemm_q(q1.cuda(), sa1.cuda(), n, w_gu.cuda(), s_gu.cuda(), native_half=native_half,
                                   variant="prefill")
    q_sep, sa_sep = ops.silu_mul_quant(gate_up, native_half=native_half)
    assert torch.equal(r["q2"][:, rows], q_sep.cpu()[:, :n])
    assert torch.equal(r["sa2"][:, rows].view(torch.int32), sa_sep.cpu()[:, :n].view(torch.int32))
    return gate_up


@pytest.mark.parametrize("t,h,inter,e,k", [(300, 512, 384, 4, 2), (200, 384, 256, 3, 2), (70, 256, 128, 5, 1)])
@pytest.mark.parametrize("native_half", [False, True])
@pytest.mark.parametrize("packed", [False, True])
def test_moe_fused_silu_codes_equal_separate_chain(t, h, inter, e, k, native_half, packed):
    """The gate_up epilogue's SiLU-and-mul + 1x128 codes and scales on every routed row against the
    separate kernels (inter 384: the up rows start half-way into a 256-row weight panel)."""
    x, logits, wg, sg, wd, sd = problem(t, h, inter, e, seed=900 + t, device="cuda")
    ws = torch.full((ops.moe_workspace_bytes(t, h, inter, e, k),), 0xC3, dtype=torch.uint8, device="cuda")
    w_gu = ops.pack_experts(wg) if packed else wg
    w_dn = ops.pack_experts(wd) if packed else wd
    ops.moe_block_fp8(x.cuda(), logits.cuda(), w_gu, sg, w_dn, sd, top_k=k, native_half=native_half, workspace=ws)
    r = regions(ws, t, h, inter, e, k)
    ids, row_of = r["ids"].reshape(t, k), r["row_of"].reshape(t, k)
    for x_e in range(e):
        rows = row_of[ids == x_e].long()
        if len(rows):
            separate_chain_check(r, rows, wg[x_e], sg[x_e], h, inter, native_half)


@pytest.mark.timeout(600)
def test_moe_config5_stagewise_parity():
    """Each stage of config 5 against the oracle, fed the device's own input to that stage, on every routed row.

    The layer's gate_up GEMM stores no bf16 output (its epilogue applies the SiLU-and-mul
    and the quantizer), so each expert's gate_up output is recomputed by the dense GEMM on
    the layer's own gathered codes and scales.  gate_up and down: the GEMM gate per expert
    row set; the layer's SiLU-and-mul codes and scales: bit-identical to the separate
    device quantizer on that output (the same per-element arithmetic in both GEMM
    kernels), and equal to the oracle's except where the device exp differs by an ulp;
    combine: bit-exact on the device's z and weights.
    """
    t, h, inter, e, k = 512, 4096, 14336, 8, 2
    x, logits, wg, sg, wd, sd = problem(t, h, inter, e, seed=5000, device="cuda")
    ws = torch.empty(ops.moe_workspace_bytes(t, h, inter, e, k), dtype=torch.uint8, device="cuda")
    y = ops.moe_block_fp8(x.cuda(), logits.cuda(), wg, sg, wd, sd, top_k=k, workspace=ws).cpu()
    r = regions(ws, t, h, inter, e, k)
    ids = r["ids"].reshape(t, k)
    row_of = r["row_of"].reshape(t, k).long()
    assert torch.equal(r["cnt"].long(), torch.bincount(ids.reshape(-1).long(), minlength=e))
    assert int(r["parts"]) == 2  # config 5: the down GEMM splits K
    tokens = torch.arange(t)  # every routed row of every expert
    for x_e in range(e):
        pairs = [(int(tok), s) for tok in tokens for s in range(k) if int(ids[tok, s]) == x_e]
        if not pairs:
            continue
        rows = torch.tensor([int(row_of[tok, s]) for tok, s in pairs])
        toks = torch.tensor([tok for tok, _ in pairs])
        w_gu, s_gu, w_dn, s_dn = wg[x_e].cpu(), sg[x_e].cpu(), wd[x_e].cpu(), sd[x_e].cpu()
        n = len(rows)
        gate_up = separate_chain_check(r, rows, wg[x_e], sg[x_e], h, inter)
        hpre = gate_up.cpu()
        ref_gu = block_fp8.reference(x[toks], w_gu, s_gu, row_chunk=16)
        p_gu = block_fp8.parity(hpre, ref_gu)
        hq = moe.silu_mul(hpre)
        codes, sa = block_fp8.act_quant(hq)
        got_codes = r["q2"][:, rows].permute(1, 0, 2).reshape(n, -1)
        mismatch = (got_codes != codes).float().mean().item()
        got_sa = r["sa2"][:, rows].T
        ref_dn = block_fp8.reference(hq, w_dn, s_dn, row_chunk=16)
        p_dn = block_fp8.parity(r["z"][rows], ref_dn)
        print(f"expert {x_e}: rows {len(rows)} gate_up {p_gu} code mismatch {mismatch:.2e} down {p_dn}", flush=True)
        assert p_gu[0] <= block_fp8.MAX_REL_TOL and p_gu[1] <= block_fp8.MEAN_REL_TOL
        assert mismatch <= 1e-3 and torch.allclose(got_sa, sa, rtol=1e-2, atol=0)
        assert p_dn[0] <= block_fp8.MAX_REL_TOL and p_dn[1] <= block_fp8.MEAN_REL_TOL
    # combine, bit-exact on the device's z and weights
    wts = r["wts"].reshape(t, k)
    z = r["z"].float()
    acc = wts[:, 0:1] * z[row_of[:, 0]]
    for s in range(1, k):
        acc = acc + wts[:, s:s + 1] * z[row_of[:, s]]
    assert torch.equal(y, acc.bfloat16())



@pytest.mark.timeout(600)
def test_moe_config5_packed_bit_identical():
    """Config 5 with experts packed at load time against row-major experts: the SiLU-and-mul codes and
    scales from the gate_up epilogue, the down GEMM's fp32 K-split planes and y agree bit for bit (the
    grouped kernel's two weight layouts)."""
    t, h, inter, e, k = 512, 4096, 14336, 8, 2
    x, logits, wg, sg, wd, sd = problem(t, h, inter, e, seed=5000, device="cuda")
    xg, lg = x.cuda(), logits.cuda()
    nbytes = ops.moe_workspace_bytes(t, h, inter, e, k)
    ws_row = torch.empty(nbytes, dtype=torch.uint8, device="cuda")
    ws_pack = torch.full((nbytes,), 0x5A, dtype=torch.uint8, device="cuda")
    y_row = ops.moe_block_fp8(xg, lg, wg, sg, wd, sd, top_k=k, workspace=ws_row)
    y_pack = ops.moe_block_fp8(xg, lg, ops.pack_experts(wg), sg, ops.pack_experts(wd), sd, top_k=k, workspace=ws_pack)
    torch.cuda.synchronize()
    r_row, r_pack = regions(ws_row, t, h, inter, e, k), regions(ws_pack, t, h, inter, e, k)
    rows = r_row["row_of"].long().reshape(-1)  # every routed row
    assert torch.equal(r_row["row_of"], r_pack["row_of"])
    assert torch.equal(r_row["q2"][:, rows], r_pack["q2"][:, rows])
    assert torch.equal(r_row["sa2"][:, rows].view(torch.int32), r_pack["sa2"][:, rows].view(torch.int32))
    assert torch.equal(r_row["zp"][:, rows].view(torch.int32), r_pack["zp"][:, rows].view(torch.int32))
    assert torch.equal(y_row.view(torch.int16), y_pack.view(torch.int16))


@pytest.mark.timeout(600)
def test_moe_config5_end_to_end_parity_and_permutation():
    t, h, inter, e = 512, 4096, 14336, 8
    x, logits, wg, sg, wd, sd = problem(t, h, inter, e, seed=5000, device="cuda")
    xg, lg = x.cuda(), logits.cuda()
    y = ops.moe_block_fp8(xg, lg, wg, sg, wd, sd, top_k=2)
    perm = torch.randperm(t, generator=torch.Generator().manual_seed(1))
    yp = ops.moe_block_fp8(xg[perm.cuda()].contiguous(), lg[perm.cuda()].contiguous(), wg, sg, wd, sd, top_k=2)
    torch.cuda.synchronize()
    assert torch.equal(yp.cpu(), y.cpu()[perm])
    ids, _ = moe.route(logits.numpy(), 2)
    counts = np.bincount(ids.reshape(-1), minlength=e)
    assert counts.min() > 0 and counts.max() != counts.min()        # uneven, every expert used
    ref = moe.moe_reference(x, logits, wg.cpu(), sg.cpu(), wd.cpu(), sd.cpu(), top_k=2)  # all 512 tokens
    max_rel, mean_rel = block_fp8.parity(y.cpu(), ref)
    print(f"config 5 end to end: max_rel {max_rel:.3e} mean_rel {mean_rel:.3e}", flush=True)
    assert max_rel <= CHAIN_MAX_REL and mean_rel <= CHAIN_MEAN_REL, (max_rel, mean_rel)


def test_moe_rejects_bad_shapes():
    x, logits, wg, sg, wd, sd = problem(8, 256, 128, 2, seed=3)
    with pytest.raises(ValueError):
        run(x, logits, wg[:, :200], sg, wd, sd)
    with pytest.raises(Exception):
        run(x, logits, wg, sg, wd, sd, top_k=3)
