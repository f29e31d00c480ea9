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


@pytest.mark.parametrize("m,n,k", [(16, 28672, 4096), (8, 6144, 4096), (1024, 2048, 7168)],
                         ids=["decode-scratch", "decode-fused", "prefill"])
def test_noalloc_under_graph_capture(m, n, k):
    """The entry's stated use: a caller that captures it in a HIP graph.  After one eager call (the per-device
    set-up: the scratch's symbol address, the LDS limit of the tiled kernels), the call is captured; each of three
    replays -- with eager work between them, including an eager call of another shape that rewrites the shared
    scratch -- gives the eager result bit for bit."""
    lib = nat.load()
    w, s = synth.weight(n, k, seed=n + k, device="cuda")
    x = synth.activations(m, k, seed=m).cuda()
    w8 = w.view(torch.uint8)
    x_other, (w_other, s_other) = synth.activations(40, 1024, seed=5).cuda(), synth.weight(512, 1024, seed=6, device="cuda")
    y_other = torch.empty((40, 512), dtype=torch.bfloat16, device="cuda")

    def call(xx, ww, ss, y):
        stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
        mm, kk = xx.shape
        nn = ww.shape[0]
        nat.check("gk_fp8_block_gemm_bf16_noalloc",
                  lib.gk_fp8_block_gemm_bf16_noalloc(_p(xx), mm, kk, xx.stride(0), _p(ww.view(torch.uint8)), nn, _p(ss),
                                                     ss.shape[0], ss.shape[1], None, _p(y), nn, 0, stream))

    y_eager = torch.empty((m, n), dtype=torch.bfloat16, device="cuda")
    call(x, w8, s, y_eager)
    torch.cuda.synchronize()
    y_graph = torch.full((m, n), 3.0, dtype=torch.bfloat16, device="cuda")
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        call(x, w8, s, y_graph)
    torch.cuda.synchronize()
    for _ in range(3):
        y_graph.fill_(3.0)
        call(x_other, w_other, s_other, y_other)  # rewrites the scratch between replays
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(y_graph.view(torch.int16), y_eager.view(torch.int16))
