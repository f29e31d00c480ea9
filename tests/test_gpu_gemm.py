"""GPU block-FP8 GEMM parity against the oracle (block_fp8_oracle.py:11-46).

Gate (north star): max|y - ref| <= 1e-2 * max|ref| and
sum|y - ref| / sum|ref| <= 2e-3, on the same seeded inputs.  Covers the
reference's golden vectors, every variant (decode / prefill / generic), the
BASELINE.json decode shapes at full size, the prefill shape at full size through
sampled rows plus size-independent properties (row permutation, exact scale
doubling), ragged shapes with bias, native_half, and untouched output padding.
"""

import pytest
import torch

from gaudi_kernels import block_fp8_oracle as gpu_oracle
from gaudi_kernels import ops
from oracle import block_fp8, synth
from golden_io import load_cases

pytestmark = pytest.mark.gpu

_, CASES = load_cases()
SENTINEL = 0x7E7E  # bf16 bit pattern never produced by these inputs


def assert_parity(y, ref, tag=""):
    max_rel, mean_rel = block_fp8.parity(y, ref)
    print(f"parity {tag}: max_rel {max_rel:.3e} mean_rel {mean_rel:.3e}", flush=True)
    assert max_rel <= block_fp8.MAX_REL_TOL and mean_rel <= block_fp8.MEAN_REL_TOL, (tag, max_rel, mean_rel)
    return max_rel, mean_rel


def run(x, w, s, bias=None, native_half=False, variant=None):
    y = ops.block_fp8_gemm(x.cuda(), w.cuda(), s.cuda(), None if bias is None else bias.cuda(),
                           native_half=native_half, variant=variant)
    return y.cpu()


def variants_for(k, m):
    vs = [None, "generic"]
    if k % 128 == 0:
        vs.append("prefill")
        if m <= 64:
            vs.append("decode")
    return vs


@pytest.mark.parametrize("case", CASES, ids=[c["name"] for c in CASES])
@pytest.mark.parametrize("native_half", [False, True])
def test_golden_vectors(case, native_half):
    want = case["y_half"] if native_half else case["y"]
    for variant in variants_for(case["k"], case["m"]):
        y = run(case["x"], case["w"], case["scales"], case["bias"], native_half, variant)
        assert_parity(y, want, f"{case['name']}/{variant}")


@pytest.mark.parametrize("m", [1, 2, 4, 8, 16])
def test_config2_qkv_decode(m):
    n, k = 6144, 4096
    w, s = synth.weight(n, k, seed=2000)
    x = synth.activations(m, k, seed=2001 + m)
    ref = block_fp8.reference(x, w, s)
    for variant in (None, "prefill"):
        assert_parity(run(x, w, s, variant=variant), ref, f"M={m}/{variant}")


@pytest.mark.parametrize("m", [1, 2, 4, 8, 16])
def test_config2_packed_fused_quantizer_against_oracle(m):
    """The benchmarked path itself -- packed weights, the 1x128 quantizer fused into the decode kernel
    (one launch, gemm_decode_kernel<8,2,4,...,WPACK,XQ,1>) -- against the oracle, not only through
    bit-identity with the unfused and row-major forms."""
    n, k = 6144, 4096
    w, s = synth.weight(n, k, seed=2000)
    x = synth.activations(m, k, seed=2001 + m)
    p = ops.pack_weight(w.cuda())
    assert ops.plan(m, n, k, 32, p.data)[0] == 1  # GK_VARIANT_DECODE on GK_FLAG_WEIGHT_PACKED weights
    y = ops.block_fp8_gemm(x.cuda(), p, s.cuda()).cpu()
    assert_parity(y, block_fp8.reference(x, w, s), f"packed fused M={m}")


@pytest.mark.parametrize("m", [1, 16])
def test_config2_native_half_packed_fused_against_oracle(m):
    """The benchmarked decode form in native_half mode: Gaudi2 half-range codes from the GPU codec, packed, the
    quantizer fused (half-range activation codes, doubled scales), against the oracle's native_half path."""
    n, k = 6144, 4096
    w, s = synth.weight(n, k, seed=2000)
    x = synth.activations(m, k, seed=2101 + m)
    wh, sh, _ = ops.codec_ocp_to_half(w.cuda(), s.cuda())
    y = ops.block_fp8_gemm(x.cuda(), ops.pack_weight(wh), sh, native_half=True).cpu()
    ref = block_fp8.reference(x, wh.cpu().view(torch.float8_e4m3fn), sh.cpu(), native_half=True)
    assert_parity(y, ref, f"native_half packed fused M={m}")


def test_config4_native_half_split_sampled_rows():
    """Config 4 through the split prefill launch in native_half mode (half-range weight codes widened in the
    kernel, doubled scales) on packed weights, against the oracle on 48 sampled rows."""
    m, n, k = 4096, 7168, 7168
    w, s = synth.weight(n, k, seed=4000)
    x = synth.activations(m, k, seed=4101)
    wh, sh, _ = ops.codec_ocp_to_half(w.cuda(), s.cuda())
    y = ops.block_fp8_gemm(x.cuda(), ops.pack_weight(wh), sh, native_half=True)
    rows = torch.randperm(m, generator=torch.Generator().manual_seed(3))[:48].sort().values
    ref = block_fp8.reference(x[rows], wh.cpu().view(torch.float8_e4m3fn), sh.cpu(), native_half=True, row_chunk=16)
    assert_parity(y[rows.cuda()].cpu(), ref, "native_half prefill sampled rows")


def test_config3_packed_against_oracle():
    m = 16
    for (n, k, seed) in ((28672, 4096, 3000), (4096, 14336, 3100)):
        w, s = synth.weight(n, k, seed=seed)
        x = synth.activations(m, k, seed=seed + 1)
        y = ops.block_fp8_gemm(x.cuda(), ops.pack_weight(w.cuda()), s.cuda()).cpu()
        assert_parity(y, block_fp8.reference(x, w, s, row_chunk=16), f"packed N={n} K={k}")


@pytest.mark.parametrize("native_half", [False, True])
def test_config1_as_specified(native_half):
    """BASELINE.json config 1 end to end on the GPU: W [256, 256] N(0, 0.02) seed 0 quantized per 128x128 block
    with scale = blockmax / 240 (Gaudi2 half range), codec forward to half range and inverse back to OCP on the
    GPU, then the GEMM on the round-tripped codes against the oracle on the same codes."""
    from oracle import fp8_codec
    x, w, s = synth.config1()
    assert int(w.view(torch.uint8).bitwise_and(0x7F).max()) <= 0x77         # D = 240 keeps codes <= 0x77
    half, s2, rounded = ops.codec_ocp_to_half(w.cuda(), s.cuda())
    want_half, want_s2, want_rounded = fp8_codec.reencode_e4m3fn_half(w.view(torch.uint8).numpy(), s.numpy())
    assert rounded == want_rounded and torch.equal(half.cpu(), torch.from_numpy(want_half))
    assert torch.equal(s2.cpu(), torch.from_numpy(want_s2))
    back, s_back = ops.codec_half_to_ocp(half, s2)
    want_back, want_s_back = fp8_codec.decode_half_to_ocp(want_half, want_s2)
    assert torch.equal(back.cpu(), torch.from_numpy(want_back)) and torch.equal(s_back.cpu(), torch.from_numpy(want_s_back))
    w_rt = back.cpu().view(torch.float8_e4m3fn)
    # the round trip changes only the codes the forward codec rounds
    changed = int((w_rt.view(torch.uint8) != w.view(torch.uint8)).sum())
    assert changed <= rounded
    for variant in (None, "decode", "prefill", "generic"):
        y = ops.block_fp8_gemm(x.cuda(), back.view(torch.float8_e4m3fn), s_back, native_half=native_half,
                               variant=variant).cpu()
        assert_parity(y, block_fp8.reference(x, w_rt, s_back.cpu(), native_half=native_half), f"config1/{variant}")


def test_config3_mlp_pair_decode():
    m = 16
    for (n, k, seed) in ((28672, 4096, 3000), (4096, 14336, 3100)):
        w, s = synth.weight(n, k, seed=seed)
        x = synth.activations(m, k, seed=seed + 1)
        ref = block_fp8.reference(x, w, s, row_chunk=16)
        assert_parity(run(x, w, s), ref, f"N={n} K={k}")


def test_config4_prefill_sampled_rows_and_invariants():
    m, n, k = 4096, 7168, 7168
    w, s = synth.weight(n, k, seed=4000)
    x = synth.activations(m, k, seed=4001)
    xd, wd, sd = x.cuda(), w.cuda(), s.cuda()
    y = ops.block_fp8_gemm(xd, wd, sd)
    rows = torch.randperm(m, generator=torch.Generator().manual_seed(1))[:48].sort().values
    ref = block_fp8.reference(x[rows], w, s, row_chunk=16)
    assert_parity(y[rows.cuda()].cpu(), ref, "prefill sampled rows")
    # Row permutation permutes the output rows bit for bit.
    perm = torch.randperm(m, generator=torch.Generator().manual_seed(2)).cuda()
    yp = ops.block_fp8_gemm(xd[perm].contiguous(), wd, sd)
    assert torch.equal(yp.view(torch.int16), y[perm].view(torch.int16))
    # Doubling every block scale doubles y exactly.
    y2 = ops.block_fp8_gemm(xd, wd, sd * 2)
    assert torch.equal(y2.view(torch.int16), (y.float() * 2).bfloat16().view(torch.int16))


@pytest.mark.timeout(600)
def test_config4_prefill_all_rows_packed_op():
    """Config 4 in the form bench.py times it: weights packed at load time, the op's 1x128 quantizer, then the
    one-launch split GEMM (256-wide tiles on 4096 columns, 192-wide on 3072) -- every one of the 4096 rows
    against the oracle (64-row chunks of the fp64 restatement: about 5 s on 16 host cores)."""
    m, n, k = 4096, 7168, 7168
    w, s = synth.weight(n, k, seed=4000)
    x = synth.activations(m, k, seed=4001)
    assert ops.plan(m, n, k)[0] == ops.nat.GK_VARIANT_PREFILL
    y = ops.block_fp8_gemm(x.cuda(), ops.pack_weight(w.cuda()), s.cuda()).cpu()
    ref = block_fp8.reference(x, w, s, row_chunk=64)
    assert_parity(y, ref, "config 4, all rows, packed weights")


@pytest.mark.parametrize("m,n,k", [(16, 200, 256), (17, 130, 512), (129, 384, 1024), (300, 1000, 768),
                                   (3, 2048, 2048), (64, 128, 128), (33, 1000, 768), (48, 2048, 1024)])
@pytest.mark.parametrize("native_half", [False, True])
def test_ragged_shapes_with_bias(m, n, k, native_half):
    w, s = synth.weight(n, k, seed=m + n + k)
    x = synth.activations(m, k, seed=m * 7 + 1)
    b = torch.randn(n, generator=torch.Generator().manual_seed(n)) * 0.1
    ref = block_fp8.reference(x, w, s, native_half=native_half, bias=b)
    for variant in variants_for(k, m):
        assert_parity(run(x, w, s, b, native_half, variant), ref, f"{m}x{n}x{k}/{variant}")


def test_output_padding_untouched():
    m, n, k = 20, 200, 512
    w, s = synth.weight(n, k, seed=77)
    x = synth.activations(m, k, seed=78)
    buf = torch.full((m + 2, n + 24), SENTINEL, dtype=torch.int16, device="cuda").view(torch.bfloat16)
    for variant in ("prefill", "generic"):
        buf.view(torch.int16).fill_(SENTINEL)
        out = buf[:m, :n]
        ops.block_fp8_gemm(x.cuda(), w.cuda(), s.cuda(), variant=variant, out=out)
        torch.cuda.synchronize()
        raw = buf.view(torch.int16)
        assert bool((raw[:m, n:] == SENTINEL).all()) and bool((raw[m:] == SENTINEL).all())
        assert_parity(out.cpu(), block_fp8.reference(x, w, s), variant)
    for mm in (1, 5, 16, 17, 20):
        buf.view(torch.int16).fill_(SENTINEL)
        out = buf[:mm, :n]
        ops.block_fp8_gemm(x[:mm].cuda(), w.cuda(), s.cuda(), variant="decode", out=out)
        torch.cuda.synchronize()
        raw = buf.view(torch.int16)
        assert bool((raw[:mm, n:] == SENTINEL).all()) and bool((raw[mm:] == SENTINEL).all())


@pytest.mark.parametrize("m,n", [(300, 203), (256, 200), (40, 1000)])
def test_prefill_epilogue_forms_same_bits(m, n):
    """The prefill tile leaves through LDS as whole-row 16-byte stores when y is 16-byte aligned with a row stride
    that is a multiple of 8, and through per-fragment stores otherwise: both forms write the same bits, only
    inside [M, N] (a ragged last 16-byte chunk included), and match the oracle."""
    k = 512
    w, s = synth.weight(n, k, seed=n + 3)
    x = synth.activations(m, k, seed=m + 4)
    b = torch.randn(n, generator=torch.Generator().manual_seed(5)) * 0.1
    ref = block_fp8.reference(x, w, s, bias=b)
    results = []
    for ld, off in ((n + (-n) % 8 + 8, 0), (n + 3, 0), (n + (-n) % 8 + 8, 1)):  # staged, odd stride, misaligned y
        buf = torch.full((m + 2, ld + 8), SENTINEL, dtype=torch.int16, device="cuda").view(torch.bfloat16)
        flat = buf.view(-1)[off: off + m * ld].view(m, ld)
        out = flat[:, :n]
        ops.block_fp8_gemm(x.cuda(), w.cuda(), s.cuda(), b.cuda(), variant="prefill", out=out)
        torch.cuda.synchronize()
        raw = buf.view(torch.int16).view(-1)
        written = torch.zeros_like(raw, dtype=torch.bool)
        idx = (off + torch.arange(m, device="cuda")[:, None] * ld + torch.arange(n, device="cuda")[None, :]).view(-1)
        written[idx] = True
        assert bool((raw[~written] == SENTINEL).all()), f"ld={ld} off={off}: a write outside [M, N]"
        results.append(out.cpu().view(torch.int16).clone())
        assert_parity(out.cpu(), ref, f"{m}x{n} ld={ld} off={off}")
    assert torch.equal(results[0], results[1]) and torch.equal(results[0], results[2])


def test_drop_in_reference_api_cpu_tensors():
    case = CASES[0]
    y = gpu_oracle.reference(case["x"], case["w"], case["scales"])
    assert y.device.type == "cpu" and y.dtype == torch.bfloat16
    assert_parity(y, case["y"])
    yh = gpu_oracle.reference(case["x"], case["w"], case["scales"], native_half=True)
    assert_parity(yh, case["y_half"])
    with pytest.raises(ValueError, match="grid"):
        gpu_oracle.reference(case["x"], case["w"], case["scales"][:, :1])
    bad = case["scales"].clone()
    bad[0, 0] = float("inf")
    with pytest.raises(ValueError, match="finite"):
        gpu_oracle.reference(case["x"], case["w"], bad)
    badx = case["x"].clone()
    badx[0, 5] = float("nan")
    with pytest.raises(ValueError, match="finite"):
        gpu_oracle.reference(badx, case["w"], case["scales"])
    with pytest.raises(ValueError, match="bias"):
        gpu_oracle.reference(case["x"], case["w"], case["scales"], bias=torch.zeros(3))


@pytest.mark.parametrize("m", [16, 24, 40, 64])
def test_q_entry_point_matches_fused(m):
    n, k = 1024, 2048
    w, s = synth.weight(n, k, seed=5)
    x = synth.activations(m, k, seed=6).cuda()
    for variant in ("decode", "prefill"):
        _, m_pad, _ = ops.plan(m, n, k, {"decode": 2, "prefill": 4}[variant])
        q, sa = ops.act_quant(x, m_pad=m_pad)
        y1 = ops.block_fp8_gemm_q(q, sa, m, w.cuda(), s.cuda(), variant=variant)  # decode: pre-quantized path
        y2 = ops.block_fp8_gemm(x, w.cuda(), s.cuda(), variant=variant)
        assert torch.equal(y1.view(torch.int16), y2.view(torch.int16))
    # decode fragment layout (what the fused op uses internally), both weight modes
    for native_half in (False, True):
        q, sa = ops.act_quant(x, native_half=native_half, decode_layout=True)
        y1 = ops.block_fp8_gemm_q(q, sa, m, w.cuda(), s.cuda(), native_half=native_half, decode_layout=True)
        y2 = ops.block_fp8_gemm(x, w.cuda(), s.cuda(), native_half=native_half)
        assert torch.equal(y1.view(torch.int16), y2.view(torch.int16))
    with pytest.raises(Exception):
        q, sa = ops.act_quant(x, decode_layout=True)
        ops.block_fp8_gemm_q(q, sa, m, w.cuda(), s.cuda(), variant="prefill", decode_layout=True)


@pytest.mark.parametrize("m,n,k", [(16, 6144, 4096), (5, 4096, 14336), (1, 200, 1024), (16, 64, 128),
                                   (7, 1000, 3072), (2, 28672, 512), (16, 16, 256),
                                   (17, 6144, 4096), (32, 4096, 14336), (33, 200, 1024), (64, 28672, 512),
                                   (50, 1000, 3072), (64, 16, 256), (31, 64, 128)])
def test_decode_shapes_deterministic(m, n, k):
    """Every decode workgroup shape the planner picks (R = 1, 2, 4 row tiles; 2-16 waves splitting K; one, two or
    four 16-token tiles; ragged N and M) matches the oracle and reruns bit-identically (fixed-order wave
    reduction)."""
    w, s = synth.weight(n, k, seed=n + k)
    x = synth.activations(m, k, seed=m + 11).cuda()
    wd, sd = w.cuda(), s.cuda()
    y1 = ops.block_fp8_gemm(x, wd, sd)
    y2 = ops.block_fp8_gemm(x, wd, sd)
    assert torch.equal(y1.view(torch.int16), y2.view(torch.int16)), (m, n, k)
    assert_parity(y1.cpu(), block_fp8.reference(x.cpu(), w, s), f"{m}x{n}x{k}")


@pytest.mark.parametrize("native_half", [False, True])
@pytest.mark.parametrize("m", [9, 37])
def test_decode_strided_unaligned_activations(native_half, m):
    """x that is not 16-byte aligned (odd row stride) gives the same bits as a dense copy."""
    n, k = 384, 1024
    w, s = synth.weight(n, k, seed=21)
    x = synth.activations(m, k, seed=22)
    base = torch.zeros((m, k + 1), dtype=torch.bfloat16)
    base[:, 1:] = x
    xs = base.cuda()[:, 1:]          # row stride k + 1, data pointer offset by 2 bytes
    y_strided = ops.block_fp8_gemm(xs, w.cuda(), s.cuda(), native_half=native_half, variant="decode")
    y_dense = ops.block_fp8_gemm(x.cuda(), w.cuda(), s.cuda(), native_half=native_half, variant="decode")
    assert torch.equal(y_strided.view(torch.int16), y_dense.view(torch.int16))
    assert_parity(y_dense.cpu(), block_fp8.reference(x, w, s, native_half=native_half))


@pytest.mark.parametrize("m,n,k", [(20, 24576, 2304), (32, 28672, 384)])
def test_decode_two_tile_narrow_step_shape(m, n, k):
    """Wide N (>= 1536 row tiles) with two token tiles and an odd group count per wave: the planner's
    (NW=2, R=2, U=1, MT=2) shape, for row-major and packed weights (bit-identical to each other)."""
    assert ops.plan(m, n, k)[0] == 1  # GK_VARIANT_DECODE
    w, s = synth.weight(n, k, seed=n + k + 1)
    x = synth.activations(m, k, seed=m + 12)
    wd, sd, xd = w.cuda(), s.cuda(), x.cuda()
    y = ops.block_fp8_gemm(xd, wd, sd)
    yp = ops.block_fp8_gemm(xd, ops.pack_weight(wd), sd)
    assert torch.equal(y.view(torch.int16), yp.view(torch.int16))
    rows = torch.arange(0, m, 3)
    assert_parity(y[rows.cuda()].cpu(), block_fp8.reference(x[rows], w, s), f"{m}x{n}x{k}")


@pytest.mark.parametrize("m,n,native_half", [(4096, 7168, False), (3000, 6000, True)])
def test_prefill_two_tile_widths(m, n, native_half):
    """GEMMs whose 256 x 256 tiles need more than one round over the CUs run their last columns in 192-wide tiles
    (a second launch).  Those columns must equal, bit for bit, a separate GEMM over just those columns (256-wide
    tiles), for row-major and packed weights, and meet the gate against the oracle on sampled rows."""
    k = 1024
    w, s = synth.weight(n, k, seed=n + 5)
    x = synth.activations(m, k, seed=m + 5)
    bias = torch.randn(n, generator=torch.Generator().manual_seed(9)) * 0.1
    xd, wd, sd, bd = x.cuda(), w.cuda(), s.cuda(), bias.cuda()
    y = ops.block_fp8_gemm(xd, wd, sd, bd, native_half=native_half)
    yp = ops.block_fp8_gemm(xd, ops.pack_weight(wd), sd, bd, native_half=native_half)
    assert torch.equal(y.view(torch.int16), yp.view(torch.int16))
    # the narrow tiles take the columns from the last multiple of 256 that keeps the first launch in whole
    # rounds (4096 and 2048 here); compare the columns from a multiple of 128 inside the narrow range
    c0 = (n - 1024) // 128 * 128
    ys = ops.block_fp8_gemm(xd, wd[c0:].contiguous(), sd[c0 // 128:].contiguous(), bd[c0:].contiguous(),
                            native_half=native_half)
    assert torch.equal(y[:, c0:].contiguous().view(torch.int16), ys.view(torch.int16))
    rows = torch.randperm(m, generator=torch.Generator().manual_seed(3))[:40].sort().values
    ref = block_fp8.reference(x[rows], w, s, native_half=native_half, bias=bias)
    assert_parity(y[rows.cuda()].cpu(), ref, f"two widths {m}x{n}")
