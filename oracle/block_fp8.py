"""CPU restatement of the block-FP8 W8A8 oracle (test infrastructure only).

Follows python/gaudi_kernels/block_fp8_oracle.py:11-46 of the reference step
by step, extended from M == 1 to M >= 1 rows (rows are independent in the
reference arithmetic: every quantity it computes is per row).  The weight is
converted to fp64 once per call and rows are processed in chunks so the fp64
partial [G, rows, N] stays bounded.

Numerics (block_fp8_oracle.py line by line):
  :25-26  a = x padded with zeros to G*128 columns, fp32
  :27     sa[g] = fp32(max(amax_g, 1e-10)) * fp32(1/448)          (fp32 multiply)
  :28     qa = e4m3fn_rne(clamp(fp32(a / sa), -448, 448))
  :29-30  w = weight padded to G*128 columns, fp32
  :31-35  native_half: qa = e4m3fn(qa*.5), w = e4m3fn(w*.5), sa*2, scales*2
  :38-39  partial[g, n] = sum_i qa[g,i] * w[n, g*128+i] in fp64 (exact)
  :40-41  y[n] = sum_g partial[g,n] * sa[g] * sw[g,n]  in fp64
  :42-45  + bias (fp64)
  :46     bf16 (torch rounds fp64 -> fp32 -> bf16)

Pinned by: tests/golden/ vectors written by the reference itself (M=1; both
modes, bias, ragged K and N, an all-zero group); the exactness of fp64
partials (closed form, brute force on tiny inputs); torch's e4m3fn cast is
pinned by oracle.e4m3 (bit arithmetic); the batched row form is checked
bit-for-bit against the per-row form.  See tests/test_oracle_gemm.py.
"""

import numpy as np
import torch

from oracle import e4m3

ERR_INPUTS = "CPU BF16 activation, original OCP FP8 weight and FP32 scales required"
ERR_GRID = "original block128 scale grid mismatch"
ERR_FINITE = "finite original inputs required"
ERR_BIAS = "CPU bias with N elements required"


def validate(x, weight, scales, bias=None):
    """The reference's checks (block_fp8_oracle.py:13-24, 43-44), M >= 1."""
    if (x.device.type != "cpu" or weight.device.type != "cpu" or scales.device.type != "cpu"
            or x.dtype != torch.bfloat16 or weight.dtype != torch.float8_e4m3fn
            or scales.dtype != torch.float32 or x.ndim != 2 or weight.ndim != 2
            or x.shape[0] < 1 or x.shape[1] != weight.shape[1]):
        raise ValueError(ERR_INPUTS)
    n, k = weight.shape
    groups = (k + 127) // 128
    if tuple(scales.shape) != ((n + 127) // 128, groups):
        raise ValueError(ERR_GRID)
    if not bool(torch.isfinite(x.float()).all() and torch.isfinite(weight.float()).all()
                and torch.isfinite(scales).all() and (scales >= 0).all()):
        raise ValueError(ERR_FINITE)
    if bias is not None and (bias.device.type != "cpu" or bias.numel() != n):
        raise ValueError(ERR_BIAS)
    return n, k, groups


def act_quant(x, native_half=False):
    """Per-row 1x128 activation quantization exactly as block_fp8_oracle.py:25-28,31-34.

    x: CPU bf16 [M, K].  Returns (qa uint8 codes [M, G*128], sa fp32 [M, G]).
    In native_half mode the codes are e4m3fn(qa*0.5) and the scales sa*2.
    """
    m, k = x.shape
    groups = (k + 127) // 128
    a = torch.zeros((m, groups, 128), dtype=torch.float32)
    a.view(m, -1)[:, :k] = x.float()
    sa = a.abs().amax(-1, keepdim=True).clamp_min(1e-10) * (1.0 / 448.0)
    q = (a / sa).clamp(-448, 448).to(torch.float8_e4m3fn)
    if native_half:
        q = (q.float() * .5).to(torch.float8_e4m3fn)
        sa = sa * 2
    return q.view(torch.uint8).reshape(m, groups * 128), sa.reshape(m, groups)


def act_quant_bits(x_f32, native_half=False):
    """Same quantization in numpy with the bit-arithmetic encoder (independent of torch's cast).

    x_f32: float32 numpy [M, K].  Returns (codes uint8 [M, G*128], sa float32 [M, G]).
    """
    m, k = x_f32.shape
    groups = (k + 127) // 128
    a = np.zeros((m, groups * 128), dtype=np.float32)
    a[:, :k] = x_f32
    a = a.reshape(m, groups, 128)
    amax = np.abs(a).max(-1, keepdims=True)
    sa = np.maximum(amax, np.float32(1e-10)) * np.float32(1.0 / 448.0)
    q = np.clip(a / sa, np.float32(-448), np.float32(448)).astype(np.float32)
    codes = e4m3.encode_rne(q)
    if native_half:
        codes = e4m3.encode_rne((e4m3.decode(codes) * 0.5).astype(np.float32))
        sa = sa * np.float32(2)
    return codes.reshape(m, groups * 128), sa.reshape(m, groups).astype(np.float32)


def reference(x, weight, scales, *, native_half=False, bias=None, row_chunk=64):
    """Row-batched restatement of ``block_fp8_oracle.reference`` (M >= 1). Returns bf16 [M, N]."""
    return _reference(x, weight, scales, native_half, bias, row_chunk, torch.bfloat16)


def reference_f64(x, weight, scales, *, native_half=False, row_chunk=64):
    """The same sum in fp64 before the final rounding (block_fp8_oracle.py:38-41, no bias) -> fp64 [M, N]."""
    return _reference(x, weight, scales, native_half, None, row_chunk, torch.float64)


def _reference(x, weight, scales, native_half, bias, row_chunk, out_dtype):
    n, k, groups = validate(x, weight, scales, bias)
    m = x.shape[0]
    qa, sa = act_quant(x, native_half)
    qa = qa.view(torch.float8_e4m3fn).float().reshape(m, groups, 128)
    w = torch.zeros((n, groups * 128), dtype=torch.float32)
    w[:, :k] = weight.float()
    if native_half:
        w = (w * .5).to(torch.float8_e4m3fn).float()
        scales = scales * 2
    wg = w.reshape(n, groups, 128).permute(1, 2, 0).double()          # [G, 128, N], once per call
    sw = scales.repeat_interleave(128, dim=0)[:n].T.double()           # [G, N]
    bias64 = bias.double().reshape(1, n) if bias is not None else None
    out = torch.empty((m, n), dtype=out_dtype)
    for r0 in range(0, m, row_chunk):
        r1 = min(m, r0 + row_chunk)
        qc = qa[r0:r1].permute(1, 0, 2).double()                        # [G, rows, 128]
        partial = torch.bmm(qc, wg)                                      # [G, rows, N], exact
        sac = sa[r0:r1].T.double().unsqueeze(-1)                         # [G, rows, 1]
        y = (partial * sac * sw.unsqueeze(1)).sum(0)                     # [rows, N]
        if bias64 is not None:
            y = y + bias64
        out[r0:r1] = y.to(out_dtype)
    return out


def reference_rowwise(x, weight, scales, *, native_half=False, bias=None):
    """Literal M=1 form of block_fp8_oracle.py:25-46 applied row by row (slow; for pinning)."""
    n, k, groups = validate(x, weight, scales, bias)
    rows = []
    for r in range(x.shape[0]):
        xr = x[r:r + 1]
        a = torch.zeros((groups, 128), dtype=torch.float32)
        a.view(-1)[:k] = xr.float().view(-1)
        sa = a.abs().amax(-1, keepdim=True).clamp_min(1e-10) * (1.0 / 448.0)
        qa = (a / sa).clamp(-448, 448).to(torch.float8_e4m3fn).float()
        w = torch.zeros((n, groups * 128), dtype=torch.float32)
        w[:, :k] = weight.float()
        sc = scales
        if native_half:
            qa = (qa * .5).to(torch.float8_e4m3fn).float()
            w = (w * .5).to(torch.float8_e4m3fn).float()
            sa = sa * 2
            sc = sc * 2
        wg = w.reshape(n, groups, 128).permute(1, 2, 0).double()
        partial = torch.bmm(qa.double().unsqueeze(1), wg).squeeze(1)
        sw = sc.repeat_interleave(128, dim=0)[:n].T.double()
        y = (partial * sa.double() * sw).sum(0, keepdim=True)
        if bias is not None:
            y = y + bias.double()
        rows.append(y.to(torch.bfloat16))
    return torch.cat(rows, 0)


def parity(y, ref):
    """(max|y-ref| / max|ref|, sum|y-ref| / sum|ref|) in fp64 -- the gate metrics."""
    y64 = y.double().cpu()
    r64 = ref.double().cpu()
    diff = (y64 - r64).abs()
    den_max = float(r64.abs().max()) if r64.numel() else 0.0
    den_sum = float(r64.abs().sum()) if r64.numel() else 0.0
    max_rel = float(diff.max()) / den_max if den_max > 0 else float(diff.max()) if diff.numel() else 0.0
    mean_rel = float(diff.sum()) / den_sum if den_sum > 0 else float(diff.sum())
    return max_rel, mean_rel


MAX_REL_TOL = 1e-2   # max|y - ref| <= 1e-2 * max|ref|  (north star)
MEAN_REL_TOL = 2e-3  # sum|y - ref| / sum|ref| <= 2e-3    (north star)
