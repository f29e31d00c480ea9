"""Write golden vectors for block_fp8_oracle.reference from the reference itself.

Run once, in the build container (never on the GPU box), as
    python tests/golden/make_golden.py /root/reference/python
It imports ONLY ``gaudi_kernels.block_fp8_oracle`` from the given reference
tree (python/gaudi_kernels/block_fp8_oracle.py:11-46), because the exact bf16
bits of that function are pinned by no reference test and by no closed form.
The codec is not imported: it is pinned by the reference's known answers.

The reference accepts M == 1 only (block_fp8_oracle.py:16), so each row of a
multi-row case is one reference call.  Inputs and outputs are stored as hex
little-endian bytes in tests/golden/oracle_vectors.json together with the
torch version that produced them.
"""

import json
import os
import sys

import numpy as np


def quantize_weight(torch, w, dmax):
    """Per 128x128 block: s = amax/dmax, q = e4m3fn(clamp(w/s, +-dmax)) (build-side generator)."""
    n, k = w.shape
    nb, g = (n + 127) // 128, (k + 127) // 128
    wp = torch.zeros(nb * 128, g * 128)
    wp[:n, :k] = w
    blk = wp.reshape(nb, 128, g, 128)
    amax = blk.abs().amax(dim=(1, 3))
    s = torch.where(amax > 0, amax / dmax, torch.ones_like(amax))
    q = (blk / s[:, None, :, None]).clamp(-dmax, dmax).reshape(nb * 128, g * 128)[:n, :k]
    return q.contiguous().to(torch.float8_e4m3fn), s.float().contiguous()


def hexs(t):
    return t.contiguous().numpy().tobytes().hex()


def main():
    ref_root = sys.argv[1] if len(sys.argv) > 1 else "/root/reference/python"
    sys.path.insert(0, ref_root)
    import torch
    from gaudi_kernels.block_fp8_oracle import reference  # the only reference import

    rng = np.random.default_rng(20261201)
    cases = []

    def add(name, m, n, k, *, wstd=0.02, dmax=448.0, bias=False, zero_group=False,
            tiny_row=False, outliers=False, codes_from_seed0=False):
        if codes_from_seed0:
            gen = torch.Generator().manual_seed(0)
            w = torch.randn(n, k, generator=gen) * wstd
            w = w.bfloat16().float()
        else:
            w = torch.from_numpy(rng.normal(0.0, wstd, (n, k)).astype(np.float32))
            blocks = ((n + 127) // 128) * ((k + 127) // 128)
            for b in rng.choice(blocks, max(1, blocks // 20), replace=False):
                bn, bg = divmod(int(b), (k + 127) // 128)
                w[bn * 128:(bn + 1) * 128, bg * 128:(bg + 1) * 128] *= 8
        wq, s = quantize_weight(torch, w, dmax)
        x = torch.from_numpy(rng.normal(0.0, 1.0, (m, k)).astype(np.float32))
        if outliers:
            cols = rng.choice(k, max(1, k // 100), replace=False)
            x[:, cols] *= 20
        if zero_group:
            x[0, 128:256] = 0
        if tiny_row and m > 1:
            x[1] = x[1] * 1e-30
        x = x.bfloat16()
        b = torch.from_numpy(rng.normal(0.0, 0.5, n).astype(np.float32)) if bias else None
        case = {
            "name": name, "m": m, "n": n, "k": k,
            "x_bf16": hexs(x.view(torch.int16)),
            "w_e4m3": hexs(wq.view(torch.uint8)),
            "scales_f32": hexs(s),
            "bias_f32": hexs(b) if b is not None else None,
        }
        for native_half in (False, True):
            ys = [reference(x[r:r + 1], wq, s, native_half=native_half, bias=b) for r in range(m)]
            key = "y_bf16_native_half" if native_half else "y_bf16"
            case[key] = hexs(torch.cat(ys, 0).view(torch.int16))
        cases.append(case)

    # BASELINE.json config 1 (CPU plumbing): W seed 0 N(0, 0.02), D = 240, X N(0,1), M=4, N=K=256.
    add("config1", 4, 256, 256, dmax=240.0, codes_from_seed0=True)
    add("ragged_nk", 3, 200, 333, bias=True)
    add("zero_group_tiny_row", 2, 128, 384, zero_group=True, tiny_row=True)
    add("outliers_bias", 2, 256, 512, bias=True, outliers=True)
    add("decode_like", 1, 256, 768, outliers=True)
    add("k_tail_small", 2, 130, 100, bias=True)

    out = {
        "generator": "tests/golden/make_golden.py",
        "reference": "python/gaudi_kernels/block_fp8_oracle.py:11-46",
        "torch": torch.__version__,
        "numpy": np.__version__,
        "cases": cases,
    }
    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "oracle_vectors.json")
    with open(path, "w") as f:
        json.dump(out, f, indent=0)
    print(f"wrote {len(cases)} cases to {path}")


if __name__ == "__main__":
    main()
