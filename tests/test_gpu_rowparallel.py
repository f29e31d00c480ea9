"""Row-parallel (K-sharded) block-FP8 GEMM on one GPU: K-range fp32 partials, the ordered rank sum, the finish.

* gk_rank_sum_f32 / gk_rank_sum_bf16 (rank_sum.c:4-42) bit-exact against oracle/reduce.py for world
  sizes 2..8, ragged and unaligned lengths, and special values (inf, NaN, -0, subnormals, cancellation);
* config 3's down projection (M=16, N=4096, K=14336) split into W in {2, 4, 8} K shards: each shard's
  fp32 partial (gk_fp8_block_gemm_kslice_f32), gathered, rank-summed and finished, meets the GEMM gate
  against the oracle; each shard's partial meets it against the oracle's fp64 range sum;
* the reference's two chunked chain cases (fp8_hybrid_tpcsim_test.cpp:388,390: 28 and 86 groups per
  chunk) accumulated over K chunks (GK_FLAG_ACCUMULATE) then finished with bias: the test's per-row
  rel-L2 gate and the GEMM gate against the oracle;
* on the LDS-tiled kernel, K ranges accumulated over several calls give the one-call GEMM's bits;
* packed and row-major weights give identical partials; the col_offset rejections.
"""

import numpy as np
import pytest
import torch

from gaudi_kernels import _native as nat
from gaudi_kernels import ops
from oracle import block_fp8, hybrid_case as hc, reduce, synth

pytestmark = pytest.mark.gpu


def assert_gate(y, ref, tag=""):
    max_rel, mean_rel = block_fp8.parity(y, ref)
    assert max_rel <= block_fp8.MAX_REL_TOL and mean_rel <= block_fp8.MEAN_REL_TOL, (tag, max_rel, mean_rel)


def special_f32(n, seed):
    rng = np.random.default_rng(seed)
    v = (rng.standard_normal(n) * np.exp2(rng.integers(-140, 120, n))).astype(np.float32)
    pick = rng.integers(0, 40, n)
    v[pick == 0] = np.inf
    v[pick == 1] = -np.inf
    v[pick == 2] = np.nan
    v[pick == 3] = -0.0
    v[pick == 4] = 1e-45
    v[pick == 5] = 3.0e38
    return v


@pytest.mark.parametrize("world", [2, 3, 4, 5, 6, 7, 8])
@pytest.mark.parametrize("elems", [1, 3, 4, 4099, 65536, 1 << 20])
def test_rank_sum_bit_exact(world, elems):
    g = special_f32(world * elems, seed=world * 1000 + elems % 997)
    got = ops.rank_sum(torch.from_numpy(g).cuda(), world).cpu().numpy()
    want = reduce.rank_sum_f32(g, world)
    same = (got.view(np.uint32) == want.view(np.uint32)) | (np.isnan(got) & np.isnan(want))
    assert same.all(), (world, elems, np.flatnonzero(~same)[:5])
    gb = reduce.f32_to_bf16_bits(special_f32(world * elems, seed=elems + world))
    gotb = ops.rank_sum(torch.from_numpy(gb.view(np.int16)).view(torch.bfloat16).cuda(), world)
    gotb = gotb.view(torch.int16).cpu().numpy().view(np.uint16)
    assert np.array_equal(gotb, reduce.rank_sum_bf16(gb, world)), (world, elems)


def test_rank_sum_unaligned_views():
    world, elems = 4, 1001
    g = special_f32(world * elems + 1, seed=7)
    buf = torch.from_numpy(g).cuda()
    got = ops.rank_sum(buf[1:], world).cpu().numpy()            # 4-byte offset: scalar path
    want = reduce.rank_sum_f32(g[1:], world)
    assert np.array_equal(got.view(np.uint32)[~np.isnan(want)], want.view(np.uint32)[~np.isnan(want)])
    assert np.isnan(got[np.isnan(want)]).all()
    # a planted order dependence: ((2^24 + 1) + 1) - 2^24 = 0 in rank order
    t = 2.0 ** 24
    o = ops.rank_sum(torch.tensor([t, 1.0, 1.0, -t]).cuda(), 4).cpu()
    assert float(o[0]) == 0.0


def shard_partials(x, w, s, world, packed=False):
    k = x.shape[1]
    kl = k // world
    wd = ops.pack_weight(w.cuda()) if packed else w.cuda()
    xd, sd = x.cuda(), s.cuda()
    return torch.stack([ops.block_fp8_gemm_kslice(xd, wd, sd, r * kl, kl) for r in range(world)])


@pytest.mark.parametrize("world", [2, 4, 8])
def test_config3_down_projection_k_sharded(world):
    m, n, k = 16, 4096, 14336
    w, s = synth.weight(n, k, seed=3100)
    x = synth.activations(m, k, seed=3101)
    parts = shard_partials(x, w, s, world)                       # [W, M, N] fp32, one per K shard
    kl = k // world
    for r in (0, world - 1):
        want = reduce.gemm_partial_f64(x, w, s, r * kl, kl)
        assert_gate(parts[r].cpu(), want, f"shard {r}/{world}")
    summed = ops.rank_sum(parts.reshape(-1), world).reshape(m, n)
    sm = summed.cpu().numpy()
    assert np.array_equal(sm.view(np.uint32), reduce.rank_sum_f32(parts.cpu().reshape(-1).numpy(), world)
                          .reshape(m, n).view(np.uint32))
    y = ops.partial_finish(summed)
    assert np.array_equal(y.view(torch.int16).cpu().numpy().view(np.uint16), reduce.partial_finish(sm))
    assert_gate(y.cpu(), block_fp8.reference(x, w, s, row_chunk=16), f"W={world}")
    # packed weights: identical partials
    assert torch.equal(shard_partials(x, w, s, world, packed=True), parts)
    # the bf16 route: each shard finished to bf16, rank-summed in fp32, rounded once
    yb = ops.rank_sum(torch.stack([ops.partial_finish(p) for p in parts]).reshape(-1), world).reshape(m, n)
    assert_gate(yb.cpu(), block_fp8.reference(x, w, s, row_chunk=16), f"W={world} bf16")


@pytest.mark.parametrize("idx", [1, 3])
def test_reference_chunked_cases(idx):
    """fp8_hybrid_tpcsim_test.cpp:389 (K=7168, 28 groups per chunk) and :391 (K=22016, 86 groups per chunk)."""
    m, n, k, with_bias, tiny, chunk, x = hc.load_cases()[idx]
    assert chunk in (28, 86)
    codes, scales = hc.weights(n, k, x)
    b = hc.bias(n) if with_bias else None
    xt = torch.from_numpy(x.astype(np.int16)).view(torch.bfloat16)
    wt = torch.from_numpy(codes).view(torch.float8_e4m3fn)
    st = torch.from_numpy(scales)
    xd, wd, sd = xt.cuda(), wt.cuda(), st.cuda()
    acc = torch.empty((m, n), dtype=torch.float32, device="cuda")
    ck = chunk * 128
    for i, off in enumerate(range(0, k, ck)):
        ops.block_fp8_gemm_kslice(xd, wd, sd, off, min(ck, k - off), out=acc, accumulate=i > 0)
    y = ops.partial_finish(acc, None if b is None else torch.from_numpy(b).cuda())
    yf = y.float().cpu().numpy()
    ref = hc.checker(x, codes, scales, b, scale_rule="oracle")
    rel = hc.row_rel_l2(yf, ref)
    assert np.all(rel <= hc.GATE), rel
    assert np.all(rel[(ref == 0).all(axis=1)] == 0.0)
    assert_gate(y.cpu(), block_fp8.reference(xt, wt, st, bias=None if b is None else torch.from_numpy(b)))


@pytest.mark.parametrize("native_half", [False, True])
def test_prefill_chunks_accumulate_to_one_call_bits(native_half):
    m, n, k = 300, 1000, 3072
    w, s = synth.weight(n, k, seed=55)
    x = synth.activations(m, k, seed=56)
    bias = torch.randn(n, generator=torch.Generator().manual_seed(57)) * 0.1
    xd, wd, sd, bd = x.cuda(), w.cuda(), s.cuda(), bias.cuda()
    one = ops.block_fp8_gemm(xd, wd, sd, bd, native_half=native_half)
    for weight in (wd, ops.pack_weight(wd)):
        acc = torch.empty((m, n), dtype=torch.float32, device="cuda")
        for i, (off, ln) in enumerate(((0, 1024), (1024, 384), (1408, 1664))):
            ops.block_fp8_gemm_kslice(xd, weight, sd, off, ln, native_half=native_half, out=acc, accumulate=i > 0)
        assert torch.equal(ops.partial_finish(acc, bd).view(torch.int16), one.view(torch.int16))
    # decode-sized M: the waves split each range, so the bits depend on the ranges; each is within the gate
    xm = x[:16].contiguous()
    acc = torch.empty((16, n), dtype=torch.float32, device="cuda")
    for i, off in enumerate(range(0, k, 768)):
        ops.block_fp8_gemm_kslice(xm.cuda(), wd, sd, off, 768, native_half=native_half, out=acc, accumulate=i > 0)
    assert_gate(ops.partial_finish(acc, bd).cpu(), block_fp8.reference(xm, w, s, native_half=native_half, bias=bias))


@pytest.mark.parametrize("m", [1, 5, 16, 40, 64, 65, 700])
def test_kslice_partials_against_oracle(m):
    n, k = 640, 2048
    w, s = synth.weight(n, k, seed=m + 3)
    x = synth.activations(m, k, seed=m + 4)
    xd, wd, sd = x.cuda(), w.cuda(), s.cuda()
    for off, ln in ((0, 128), (512, 1024), (1920, 128), (0, 2048)):
        p = ops.block_fp8_gemm_kslice(xd, wd, sd, off, ln)
        assert_gate(p.cpu(), reduce.gemm_partial_f64(x, w, s, off, ln), f"m={m} [{off},+{ln})")
    # row stride of the partial larger than N: the padding stays untouched
    buf = torch.full((m, n + 8), 7.0, dtype=torch.float32, device="cuda")
    ops.block_fp8_gemm_kslice(xd, wd, sd, 256, 256, out=buf[:, :n])
    assert bool((buf[:, n:] == 7.0).all())


def test_kslice_rejections_on_device_tensors():
    x = synth.activations(4, 512, seed=1).cuda()
    w, s = synth.weight(256, 512, seed=2)
    wd, sd = w.cuda(), s.cuda()
    with pytest.raises(nat.GkError) as e:
        ops.block_fp8_gemm_kslice(x, wd, sd, 384, 256)          # 384 + 256 > 512
    assert e.value.status == nat.GK_INCOMPATIBLE_INPUT_SIZE
    with pytest.raises(nat.GkError) as e:
        ops.block_fp8_gemm_kslice(x, wd, sd, 64, 256)
    assert e.value.status == nat.GK_UNSUPPORTED_LAYER_CONFIGURATION
    ops.block_fp8_gemm_kslice(x, wd, sd, 256, 256)               # offset 256, [256, 511]: accepted
