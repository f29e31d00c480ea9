"""Seeded synthetic inputs for the BASELINE.json configurations (test infrastructure only).

The reference ships no generator for the block-FP8 path; these follow the
build-side recipe for BASELINE.json's configs:
  * weights N(0, wstd), a seeded 5% of the 128x128 blocks scaled x8, then per
    block s = amax/D, q = e4m3fn(clamp(W/s, +-D)) with D = 448 (OCP checkpoint
    convention) or 240 (config 1, Gaudi2 half range);
  * activations N(0, 1) with a seeded 1% of the K channels scaled x20;
  * inputs are generated on the CPU with torch.Generator so the GPU path and
    the CPU oracle see identical bits.
"""

import torch


def quantize_weight(w, dmax=448.0):
    """Per-128x128-block E4M3 quantization of an fp32 [N, K] master -> (e4m3fn [N,K], fp32 [NB,G])."""
    n, k = w.shape
    nb, g = (n + 127) // 128, (k + 127) // 128
    wp = torch.zeros(nb * 128, g * 128, dtype=torch.float32, device=w.device)
    wp[:n, :k] = w
    blk = wp.reshape(nb, 128, g, 128)
    amax = blk.abs().amax(dim=(1, 3))
    s = torch.where(amax > 0, amax / dmax, torch.ones_like(amax))
    q = (blk / s[:, None, :, None]).clamp(-dmax, dmax).reshape(nb * 128, g * 128)[:n, :k]
    return q.contiguous().to(torch.float8_e4m3fn), s.float().contiguous()


def weight(n, k, seed, *, wstd=0.02, outlier_frac=0.05, dmax=448.0, device="cpu"):
    gen = torch.Generator(device=device).manual_seed(seed)
    w = torch.randn(n, k, generator=gen, device=device) * wstd
    nb, g = (n + 127) // 128, (k + 127) // 128
    nblk = int(round(outlier_frac * nb * g))
    if nblk:
        pick = torch.randperm(nb * g, generator=gen, device=device)[:nblk]
        mask = torch.ones(nb * g, device=device)
        mask[pick] = 8.0
        mask = mask.reshape(nb, 1, g, 1).expand(nb, 128, g, 128).reshape(nb * 128, g * 128)
        w = w * mask[:n, :k]
    return quantize_weight(w, dmax)


def activations(m, k, seed, *, outlier_frac=0.01, device="cpu"):
    gen = torch.Generator(device=device).manual_seed(seed)
    x = torch.randn(m, k, generator=gen, device=device)
    ncol = int(round(outlier_frac * k))
    if ncol:
        cols = torch.randperm(k, generator=gen, device=device)[:ncol]
        x[:, cols] *= 20.0
    return x.bfloat16()


def config1():
    """W seed 0, N(0, 0.02), D = 240; X N(0, 1) seed 1, M=4, N=K=256."""
    gen = torch.Generator().manual_seed(0)
    w = torch.randn(256, 256, generator=gen) * 0.02
    wq, s = quantize_weight(w, 240.0)
    gen_x = torch.Generator().manual_seed(1)
    x = torch.randn(4, 256, generator=gen_x).bfloat16()
    return x, wq, s
