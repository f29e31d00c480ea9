"""The reference's five GEMM test cases (tests/fp8_hybrid_tpcsim_test.cpp:388-392) on the GPU.

Inputs: the reference generator's activations (tests/golden/hybrid_gemm_x.npz), closed-form weights,
block scales and bias (oracle/hybrid_case.py).  Gates:
  * the reference's own: per output row, bf16 relative L2 error <= 0.01 against the FP64 checker
    (:366-378), and exact zeros on identically zero rows (:369-371) -- with the checker using the
    block_fp8_oracle scale rule this build implements (the test's TPC chain rounds its group scale
    differently, which flips an occasional code);
  * this build's GEMM gate against oracle/block_fp8.reference, both modes, row-major and packed weights.
The chunked case (:389) splits K across calls of the reference's FP16 chain; one call covers it here
(its activations equal the first case's), run on a padded-stride view of x instead.
"""

import numpy as np
import pytest
import torch

from gaudi_kernels import ops
from oracle import block_fp8, hybrid_case as hc

pytestmark = pytest.mark.gpu

CASES = hc.load_cases()


def tensors(idx):
    m, n, k, with_bias, tiny, chunk, x = CASES[idx]
    codes, scales = hc.weights(n, k, x)
    b = hc.bias(n) if with_bias else None
    xt = torch.from_numpy(x.astype(np.int16)).view(torch.bfloat16)
    wt = torch.from_numpy(codes).view(torch.float8_e4m3fn)
    return x, codes, scales, b, xt, wt, torch.from_numpy(scales), None if b is None else torch.from_numpy(b)


@pytest.mark.parametrize("idx", range(5))
def test_reference_case_gate(idx):
    x, codes, scales, b, xt, wt, st, bt = tensors(idx)
    ref = hc.checker(x, codes, scales, b, scale_rule="oracle")
    xd = xt.cuda()
    if CASES[idx][5]:  # the chunked case: activations in a wider buffer (row stride > K)
        wide = torch.zeros(xt.shape[0], xt.shape[1] + 128, dtype=torch.bfloat16, device="cuda")
        wide[:, : xt.shape[1]] = xd
        xd = wide[:, : xt.shape[1]]
    for weight in (wt.cuda(), ops.pack_weight(wt.cuda())):
        y = ops.block_fp8_gemm(xd, weight, st.cuda(), None if bt is None else bt.cuda()).float().cpu().numpy()
        rel = hc.row_rel_l2(y, ref)
        assert np.all(rel <= hc.GATE), rel
        zero = (ref == 0).all(axis=1)
        assert np.all(rel[zero] == 0.0)
        assert np.all(np.isfinite(y))


@pytest.mark.parametrize("idx", range(5))
@pytest.mark.parametrize("native_half", [False, True])
def test_reference_case_vs_oracle(idx, native_half):
    x, codes, scales, b, xt, wt, st, bt = tensors(idx)
    want = block_fp8.reference(xt, wt, st, native_half=native_half, bias=bt)
    y = ops.block_fp8_gemm(xt.cuda(), wt.cuda(), st.cuda(), None if bt is None else bt.cuda(),
                           native_half=native_half).cpu()
    max_rel, mean_rel = block_fp8.parity(y, want)
    assert max_rel <= block_fp8.MAX_REL_TOL and mean_rel <= block_fp8.MEAN_REL_TOL, (max_rel, mean_rel)
