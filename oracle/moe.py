"""CPU restatement of the block-FP8 MoE layer (test infrastructure only).

The reference has no MoE, routing, gather/scatter or collective code for the
block-FP8 path.  The MoE layer benchmarked here is therefore build-defined, from
the reference's own pieces:

  route    top-k (k = 1 or 2) experts per token by router logit; ties go to the
           lower expert index.  Combine weights = softmax over the k selected
           logits (fp32).
  rows     every (token, slot) pair is one row; rows are ordered by expert,
           then by token (stable).  Each expert's rows start at a padded
           offset (multiple of `row_align`) so that GEMM row tiles never mix
           experts; padding rows carry no token.
  gate_up  y_e = block_fp8_oracle.reference(x[rows of e], W_gu[e], S_gu[e])
           -- python/gaudi_kernels/block_fp8_oracle.py:11-46, bf16 out.
  act      h = bf16(silu(gate) * up) in fp32, gate = first half of the
           columns, up = second half, silu(g) = g / (1 + exp(-g)), g <= -88
           -> 0, NaN -> NaN, +inf -> NaN (the reference's Newton-refined
           quotient computes -inf + inf there); only the product is rounded
           -- the semantics of the reference's fused SiLU-and-mul kernel
           (csrc/tpc/generic_dense/silu_and_mul_bf16.c:4-15, 15-16).
  down     z_e = block_fp8_oracle.reference(h, W_dn[e], S_dn[e]), bf16.
  combine  y[t] = bf16(sum_k w[t, k] * z[row(t, k)]) in fp32, k ascending.

Pinned by: the routing is checked against an explicit per-token loop and
brute-force tie cases; the GEMMs are block_fp8.reference (pinned by the
reference's golden vectors); silu_mul against an fp64 evaluation.  See
tests/test_oracle_moe.py.
"""

import numpy as np
import torch

from oracle import block_fp8


def route(logits, top_k=2):
    """(ids int64 [T, k], weights fp32 [T, k]) -- top-k by logit, ties to the lower expert."""
    lg = np.asarray(logits, dtype=np.float32)
    t, e = lg.shape
    if not 1 <= top_k <= min(2, e):
        raise ValueError("top_k must be 1 or 2 and at most the expert count")
    ids = np.empty((t, top_k), dtype=np.int64)
    work = lg.copy()
    for k in range(top_k):
        ids[:, k] = np.argmax(work, axis=1)          # first occurrence: lower index on ties
        work[np.arange(t), ids[:, k]] = -np.inf
    sel = lg[np.arange(t)[:, None], ids]             # [T, k] fp32
    ex = np.exp((sel - sel[:, :1]).astype(np.float32)).astype(np.float32)
    w = (ex / ex.sum(axis=1, keepdims=True)).astype(np.float32)
    return ids, w


def route_loop(logits, top_k=2):
    """Literal per-token restatement of `route` (for pinning)."""
    lg = np.asarray(logits, dtype=np.float32)
    ids, ws = [], []
    for row in lg:
        chosen = []
        for _ in range(top_k):
            best = None
            for j, v in enumerate(row):
                if j in chosen:
                    continue
                if best is None or v > row[best]:
                    best = j
            chosen.append(best)
        sel = np.array([row[j] for j in chosen], dtype=np.float32)
        ex = np.exp(sel - sel[0]).astype(np.float32)
        ids.append(chosen)
        ws.append((ex / ex.sum()).astype(np.float32))
    return np.array(ids, dtype=np.int64), np.array(ws, dtype=np.float32)


def layout(ids, n_experts, row_align=256):
    """Expert-sorted row layout.

    Returns (row_token int64 [R], row_slot int64 [R], row_of int64 [T, k],
    offsets int64 [E+1] (padded starts), counts int64 [E]) where R is the
    padded row count; padding rows have row_token = -1.
    """
    t, k = ids.shape
    counts = np.bincount(ids.reshape(-1), minlength=n_experts).astype(np.int64)
    padded = (counts + row_align - 1) // row_align * row_align
    offsets = np.concatenate([[0], np.cumsum(padded)]).astype(np.int64)
    rows = int(offsets[-1])
    row_token = np.full(rows, -1, dtype=np.int64)
    row_slot = np.full(rows, -1, dtype=np.int64)
    row_of = np.empty((t, k), dtype=np.int64)
    fill = offsets[:-1].copy()
    for tok in range(t):                 # token order -> stable within each expert
        for slot in range(k):
            e = ids[tok, slot]
            r = fill[e]
            fill[e] += 1
            row_token[r] = tok
            row_slot[r] = slot
            row_of[tok, slot] = r
    return row_token, row_slot, row_of, offsets, counts


def silu_mul(gate_up):
    """bf16 [R, 2W] -> bf16 [R, W]: bf16(silu(g) * u) in fp32 (csrc/tpc/generic_dense/silu_and_mul_bf16.c)."""
    g = gate_up[:, : gate_up.shape[1] // 2].float()
    u = gate_up[:, gate_up.shape[1] // 2:].float()
    s = g / (1.0 + torch.exp(-g))
    s = torch.where(g <= -88.0, torch.zeros_like(s), s)
    s = torch.where(g == float("inf"), torch.full_like(s, float("nan")), s)  # silu_and_mul_bf16.c:8-9
    return (s * u).to(torch.bfloat16)


def silu_mul_f64(gate_up):
    g = gate_up[:, : gate_up.shape[1] // 2].double()
    u = gate_up[:, gate_up.shape[1] // 2:].double()
    s = torch.where(g <= -88.0, torch.zeros_like(g), g / (1.0 + torch.exp(-g)))
    return s * u


def moe_reference(x, logits, w_gu, s_gu, w_dn, s_dn, *, top_k=2, tokens=None, native_half=False):
    """bf16 [T, H] MoE output (rows `tokens` only when given, in that order).

    x bf16 [T, H]; logits fp32 [T, E]; w_gu e4m3fn [E, 2I, H], s_gu fp32 [E, ceil(2I/128), ceil(H/128)];
    w_dn e4m3fn [E, H, I], s_dn fp32 [E, ceil(H/128), ceil(I/128)].
    Combine: y = w_0 * z_0 (+ w_1 * z_1), each product and the sum rounded to fp32, then bf16.
    native_half: both GEMMs in the reference's native_half mode (block_fp8_oracle.py:31-35).
    """
    ids, wts = route(logits.numpy() if isinstance(logits, torch.Tensor) else logits, top_k)
    t = x.shape[0]
    sel = np.arange(t) if tokens is None else np.asarray(tokens)
    z = {}
    for e in sorted(set(ids[sel].reshape(-1).tolist())):
        pairs = [(int(tok), k) for tok in sel for k in range(top_k) if ids[tok, k] == e]
        rows = torch.tensor([tok for tok, _ in pairs])
        h = silu_mul(block_fp8.reference(x[rows], w_gu[e], s_gu[e], native_half=native_half, row_chunk=16))
        ze = block_fp8.reference(h, w_dn[e], s_dn[e], native_half=native_half, row_chunk=16).float()
        for pair, zr in zip(pairs, ze):
            z[pair] = zr
    out = torch.empty((len(sel), w_dn.shape[1]), dtype=torch.float32)
    for i, tok in enumerate(sel):
        acc = torch.tensor(float(wts[tok, 0]), dtype=torch.float32) * z[(int(tok), 0)]
        for k in range(1, top_k):
            acc = acc + torch.tensor(float(wts[tok, k]), dtype=torch.float32) * z[(int(tok), k)]
        out[i] = acc
    return out.to(torch.bfloat16)
