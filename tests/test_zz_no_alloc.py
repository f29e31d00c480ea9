"""The allocation-free GEMM entry (gk_fp8_block_gemm_bf16_noalloc) against gk_fp8_block_gemm_bf16.

Both are called through the C ABI on the same device buffers; the outputs must be equal bit for bit.
Two calls in a row, the second smaller than the first, so stale scratch contents from the first call
would show in the second; shapes that use the scratch (quantizer then GEMM: the decode variant where
fusing the quantizer does not pay, and the LDS-tiled variant) and the fused decode shape that needs none.
Sizes beyond the scratch are rejected before any device work.
"""

import ctypes

import pytest
import torch

from gaudi_kernels import _native as nat
from gaudi_kernels import ops
from oracle import synth

pytestmark = pytest.mark.gpu


def _p(t):
    return ctypes.c_void_p(t.data_ptr()) if t is not None else None


def both(x, w, s, bias, flags=0):
    lib = nat.load()
    m, k = x.shape
    n = w.shape[0]
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    _, _, ws_bytes = ops.plan(m, n, k, flags, w)
    ws = torch.empty(max(ws_bytes, 256), dtype=torch.uint8, device="cuda")
    y_ref = torch.full((m, n), 1.0, dtype=torch.bfloat16, device="cuda")
    y_na = torch.full((m, n), 2.0, dtype=torch.bfloat16, device="cuda")
    w8 = w.view(torch.uint8)
    nat.check("gk_fp8_block_gemm_bf16",
              lib.gk_fp8_block_gemm_bf16(_p(x), m, k, x.stride(0), _p(w8), n, _p(s), s.shape[0], s.shape[1], _p(bias),
                                         _p(y_ref), n, flags, _p(ws), ws.numel(), stream))
    nat.check("gk_fp8_block_gemm_bf16_noalloc",
              lib.gk_fp8_block_gemm_bf16_noalloc(_p(x), m, k, x.stride(0), _p(w8), n, _p(s), s.shape[0], s.shape[1],
                                                 _p(bias), _p(y_na), n, flags, stream))
    torch.cuda.synchronize()
    return y_ref, y_na


# (first call, second smaller call): decode with the separate quantizer, prefill, fused decode, native_half
SEQUENCES = [
    ((16, 28672, 4096), (9, 28672, 2048)),
    ((1024, 2048, 7168), (300, 2048, 4096)),
    ((4096, 7168, 7168), (70, 512, 1024)),
    ((8, 6144, 4096), (3, 6144, 4096)),
    ((48, 4096, 14336), (20, 4096, 1024)),
]


@pytest.mark.parametrize("seq", SEQUENCES, ids=[f"{a[0]}x{a[1]}x{a[2]}-then-{b[0]}x{b[1]}x{b[2]}" for a, b in SEQUENCES])
@pytest.mark.parametrize("native_half", [False, True])
def test_noalloc_matches_workspace_entry_twice(seq, native_half):
    flags = nat.GK_FLAG_NATIVE_HALF if native_half else 0
    for i, (m, n, k) in enumerate(seq):
        w, s = synth.weight(n, k, seed=n + k + i, device="cuda")
        x = synth.activations(m, k, seed=m + i).cuda()
        bias = (torch.randn(n, generator=torch.Generator().manual_seed(n)) * 0.1).cuda() if i else None
        y_ref, y_na = both(x, w, s, bias, flags)
        assert torch.equal(y_ref.view(torch.int16), y_na.view(torch.int16)), (m, n, k, i)


def test_noalloc_rejects_beyond_scratch():
    lib = nat.load()
    m, n, k = 8192, 7168, 7168          # 8192 x 56 groups x 132 B > 32 MiB of scratch
    _, _, need = ops.plan(m, n, k)
    assert need > (32 << 20)
    fake = ctypes.c_void_p(1 << 20)
    st = lib.gk_fp8_block_gemm_bf16_noalloc(fake, m, k, k, fake, n, fake, 56, 56, None, fake, n, 0, None)
    assert st == nat.GK_INSUFFICIENT_BUFFER
