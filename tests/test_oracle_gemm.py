"""Pin the GEMM restatement (oracle/block_fp8.py).

* golden vectors written by the reference's own block_fp8_oracle.reference
  (tests/golden/) must be reproduced bit for bit, in both modes;
* an exact rational brute force on tiny inputs must land within one bf16 ulp
  (the reference's only rounding after exact fp64 partials is the final
  fp64 -> fp32 -> bf16 cast), so a dropped term, a wrong sign, a wrong group
  index or a transposed operand fails;
* scaling every block scale by 2 doubles y exactly;
* the batched row form equals the literal per-row form bit for bit.
"""

from fractions import Fraction

import numpy as np
import pytest
import torch

from oracle import block_fp8, e4m3, synth
from golden_io import load_cases

DATA, CASES = load_cases()


def bits(t):
    return t.view(torch.int16)


@pytest.mark.parametrize("case", CASES, ids=[c["name"] for c in CASES])
@pytest.mark.parametrize("native_half", [False, True])
def test_golden_vectors_bit_exact(case, native_half):
    y = block_fp8.reference(case["x"], case["w"], case["scales"], native_half=native_half, bias=case["bias"])
    want = case["y_half"] if native_half else case["y"]
    assert torch.equal(bits(y), bits(want))


def test_golden_provenance():
    assert DATA["reference"].startswith("python/gaudi_kernels/block_fp8_oracle.py")
    assert len(CASES) >= 6


def brute_force(x, w, scales, bias, native_half):
    """Exact rational evaluation of the reference formula for tiny inputs."""
    m, k = x.shape
    n = w.shape[0]
    g = (k + 127) // 128
    qa, sa = block_fp8.act_quant(x, native_half)
    qv = e4m3.decode(qa.numpy())
    wc = w.view(torch.uint8).numpy()
    if native_half:
        wc = e4m3.encode_rne((e4m3.decode(wc) * 0.5).astype(np.float32))
    wv = e4m3.decode(wc)
    sc = scales.numpy().astype(np.float64) * (2.0 if native_half else 1.0)
    out = np.zeros((m, n))
    for r in range(m):
        for c in range(n):
            acc = Fraction(0)
            for gi in range(g):
                part = Fraction(0)
                for i in range(128):
                    kk = gi * 128 + i
                    if kk < k:
                        part += Fraction(float(qv[r, kk])) * Fraction(float(wv[c, kk]))
                acc += part * Fraction(float(sa[r, gi])) * Fraction(float(sc[c // 128, gi]))
            if bias is not None:
                acc += Fraction(float(bias[c]))
            out[r, c] = float(acc)
    return out


@pytest.mark.parametrize("native_half", [False, True])
def test_brute_force_tiny(native_half):
    gen = torch.Generator().manual_seed(3)
    m, n, k = 2, 3, 200
    x = (torch.randn(m, k, generator=gen) * 3).bfloat16()
    x[0, :128] = 0  # all-zero group
    w = (torch.randn(n, k, generator=gen) * 80).clamp(-448, 448).to(torch.float8_e4m3fn)
    s = torch.rand(1, 2, generator=gen) * 1e-2 + 1e-3
    b = torch.randn(n, generator=gen)
    exact = brute_force(x, w, s, b, native_half)
    y = block_fp8.reference(x, w, s, native_half=native_half, bias=b).double().numpy()
    # within one bf16 ulp of the exact value
    ulp = np.exp2(np.floor(np.log2(np.abs(exact))) - 7)
    assert np.all(np.abs(y - exact) <= ulp)


def test_scale_doubling_is_exact():
    x, w, s = synth.config1()
    y1 = block_fp8.reference(x, w, s)
    y2 = block_fp8.reference(x, w, s * 2)
    assert torch.equal(bits(y2), bits((y1.float() * 2).bfloat16()))


def test_batched_equals_rowwise():
    gen = torch.Generator().manual_seed(5)
    x = torch.randn(9, 640, generator=gen).bfloat16()
    w, s = synth.weight(300, 640, seed=11)
    b = torch.randn(300, generator=gen)
    for nh in (False, True):
        y1 = block_fp8.reference(x, w, s, native_half=nh, bias=b, row_chunk=4)
        y2 = block_fp8.reference_rowwise(x, w, s, native_half=nh, bias=b)
        assert torch.equal(bits(y1), bits(y2))


def test_rejections():
    x, w, s = synth.config1()
    with pytest.raises(ValueError, match="grid"):
        block_fp8.reference(x, w, s[:, :1])
    bad = s.clone()
    bad[0, 0] = float("nan")
    with pytest.raises(ValueError, match="finite"):
        block_fp8.reference(x, w, bad)
    with pytest.raises(ValueError, match="bias"):
        block_fp8.reference(x, w, s, bias=torch.zeros(3))
    with pytest.raises(ValueError):
        block_fp8.reference(x.float(), w, s)


def test_config1_plumbing():
    """BASELINE.json config 1 through the oracle (the CPU-runnable case)."""
    x, w, s = synth.config1()
    assert int((w.view(torch.uint8) & 0x7F).max()) <= 0x77  # D = 240 keeps codes in the shared range
    y = block_fp8.reference(x, w, s)
    assert y.shape == (4, 256) and torch.isfinite(y.float()).all()
    # Codec round trip to OCP keeps every code except the rounded low ones.
    from oracle import fp8_codec
    h, s2, rounded = fp8_codec.reencode_e4m3fn_half(w.view(torch.uint8).numpy(), s.numpy())
    back, s1 = fp8_codec.decode_half_to_ocp(h, s2)
    assert np.array_equal(s1, s.numpy())
    changed = int((back != w.view(torch.uint8).numpy()).sum())
    assert changed <= rounded
