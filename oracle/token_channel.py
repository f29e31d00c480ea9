"""CPU restatement of the per-token / per-channel W8A8 path (test infrastructure only).

Reference: csrc/tpc/block_fp8_framework/activation_token.c:4-26 with
activation_quant_common.h:3-30 (token quant) and channel_finish.c:2-18 (the
epilogue on the MME's fp32 product).  The arithmetic is restated step for step
in IEEE fp32, with an exact fp32 fused multiply-add (``fma32``) where the TPC
code uses v_f32_mac_b:

  m   = max |x| over the row, 1 for an all-zero row            (activation_token.c:9-16)
  s0  = fp32(m * fp32(1/448));  s = fma(fma(-s0, 448, m), fp32(1/448), s0)   (common.h:3-7)
  r   = fp32(1 / s)                                            (IEEE; the TPC reciprocal's
                                                                rounding is not documented)
  q0  = fp32(x * r);  z = fma(fma(-q0, s, x), r, q0)           (common.h:10-12)
  code = E4M3 RNE of min(|z|, 448) with x's sign, halved into the Gaudi2 half range
         (value / 2, RNE on the half-range grid: the codec rule)    (common.h:13-21, 23-29)
  scale = 2 s                                                  (activation_token.c:24)
  y   = bf16(fma(fp32(P * a), w, b))                           (channel_finish.c:9-15)

Pinned by: fma32 against exact rational arithmetic on random and tie-forcing
inputs; the scale against the exact quotient m / 448 (within half an ulp) and
rational arithmetic; the codes against a rational-arithmetic restatement on
small inputs, the codec table and the dequantization bound.  See
tests/test_oracle_token.py.
"""

from fractions import Fraction

import numpy as np

from oracle import e4m3, fp8_codec

F32 = np.float32
INV448 = F32(1.0) / F32(448.0)


def fma32(a, b, c):
    """Exact fp32 fused multiply-add on float32 arrays (a*b + c rounded once, RNE)."""
    a = np.asarray(a, dtype=F32).astype(np.float64)
    b = np.asarray(b, dtype=F32).astype(np.float64)
    c = np.asarray(c, dtype=F32).astype(np.float64)
    p = a * b                                   # exact: 24 x 24 bits
    s = p + c
    t = s - p
    e = (p - (s - t)) + (c - t)                 # TwoSum: p + c == s + e exactly
    r = s.astype(F32)
    # s is rounded to fp32 correctly unless it sits exactly on an fp32 midpoint
    # and e says which side the exact value is on.
    rd = r.astype(np.float64)
    toward = np.where(s > rd, np.inf, -np.inf).astype(F32)
    other = np.nextafter(r, toward)
    mid = (rd + other.astype(np.float64)) * 0.5
    on_mid = (rd != s) & (mid == s) & (e != 0)
    up = e > 0
    fix = np.where(up, np.maximum(r, other), np.minimum(r, other))
    return np.where(on_mid, fix, r).astype(F32)


def fma32_exact(a, b, c):
    """Scalar fp32 fma by rational arithmetic (for pinning fma32)."""
    v = Fraction(float(F32(a))) * Fraction(float(F32(b))) + Fraction(float(F32(c)))
    return _round_f32(v)


def _round_f32(v):
    """Fraction -> nearest fp32 (ties to even), for finite normal-range values."""
    if v == 0:
        return F32(0.0)
    f = F32(float(v))                           # float64 rounding first ...
    # ... then correct the (rare) double rounding by comparing against neighbours
    best = f
    for cand in (np.nextafter(f, F32(-np.inf)), f, np.nextafter(f, F32(np.inf))):
        if abs(Fraction(float(cand)) - v) < abs(Fraction(float(best)) - v):
            best = cand
        elif abs(Fraction(float(cand)) - v) == abs(Fraction(float(best)) - v) and cand != best:
            if (int(np.asarray(cand).view(np.uint32)) & 1) == 0:
                best = cand
    return F32(best)


def token_scale(m):
    """activation_quant_common.h:3-7 on fp32 row maxima."""
    m = np.asarray(m, dtype=F32)
    s0 = (m * INV448).astype(F32)
    res = fma32(-s0, F32(448.0), m)
    return fma32(res, INV448, s0)


def token_quant(x):
    """x: bf16 torch tensor or fp32 array [rows, width] -> (half-range codes uint8, scales fp32 [rows])."""
    xf = np.asarray(x.float().numpy() if hasattr(x, "float") else x, dtype=F32)
    m = np.abs(xf).max(axis=1)
    m = np.where(m == 0, F32(1.0), m).astype(F32)
    s = token_scale(m)
    r = (F32(1.0) / s).astype(F32)
    sc, rc = s[:, None], r[:, None]
    q0 = (xf * rc).astype(F32)
    z = fma32(fma32(-q0, sc, xf), rc, q0)
    zc = np.minimum(np.abs(z), F32(448.0)) * np.where(np.signbit(xf), F32(-1.0), F32(1.0))
    ocp = e4m3.encode_rne(zc.astype(F32))
    ocp = np.where(np.signbit(xf), ocp | 0x80, ocp & 0x7F).astype(np.uint8)   # the sign of x, also for 0
    half = fp8_codec.forward_table()[ocp]
    return half.astype(np.uint8), (s * F32(2.0)).astype(F32)


def channel_finish(partial, act, w, bias=None):
    """channel_finish.c:9-15: bf16(fma(fp32(p * a), w, b)) -> uint16 bf16 bits."""
    p = np.asarray(partial, dtype=F32)
    x0 = (p * np.asarray(act, dtype=F32)[:, None]).astype(F32)
    b = np.zeros(p.shape[1], dtype=F32) if bias is None else np.asarray(bias, dtype=F32)
    y = fma32(x0, np.broadcast_to(np.asarray(w, dtype=F32), p.shape), np.broadcast_to(b, p.shape))
    return _bf16_bits(y)


def channel_reference(q, sa, w, sw, bias=None):
    """Per-token / per-channel GEMM: exact fp8 products summed in fp64, rounded to fp32, then channel_finish.
    q: uint8 codes [M, K] (OCP or half-range bytes, read as OCP values), w: codes [N, K] -> bf16 bits [M, N]."""
    qv = e4m3.decode(np.asarray(q, dtype=np.uint8))
    wv = e4m3.decode(np.asarray(w, dtype=np.uint8))
    p = (qv @ wv.T).astype(F32)
    return channel_finish(p, sa, sw, bias)


def _bf16_bits(v):
    b = np.asarray(v, dtype=F32).view(np.uint32).astype(np.uint64)
    nan = (b & 0x7FFFFFFF) > 0x7F800000
    r = ((b + 0x7FFF + ((b >> 16) & 1)) >> 16) & 0xFFFF
    return np.where(nan, 0x7FC0, r).astype(np.uint16)


def token_quant_exact(xrow):
    """One row by rational arithmetic (slow; for pinning token_quant on small inputs)."""
    xs = [F32(v) for v in np.asarray(xrow, dtype=F32)]
    m = max(abs(v) for v in xs)
    m = F32(1.0) if m == 0 else m
    s0 = F32(m * INV448)
    s = fma32_exact(fma32_exact(-s0, 448.0, m), INV448, s0)
    r = F32(F32(1.0) / s)
    codes = []
    for x in xs:
        q0 = F32(x * r)
        z = fma32_exact(fma32_exact(-q0, s, x), r, q0)
        zc = min(abs(z), F32(448.0))
        c = int(e4m3.encode_rne(np.array([zc], dtype=F32))[0]) & 0x7F
        if np.signbit(x):
            c |= 0x80
        codes.append(int(fp8_codec.forward_table()[c]))
    return np.array(codes, dtype=np.uint8), F32(s * F32(2.0))
