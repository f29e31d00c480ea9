"""Pins the CPU restatement of the block-FP8 MoE layer (oracle/moe.py).

The reference has no MoE code, so nothing here is a golden vector: routing is
pinned by an explicit per-token loop and hand-worked tie cases, the layout by
its invariants (a permutation of the (token, slot) pairs, stable within each
expert, segments aligned), SiLU-and-mul by an fp64 evaluation and its
special cases (csrc/tpc/generic_dense/silu_and_mul_bf16.c:4-15), and the whole
layer by a literal per-token evaluation through block_fp8.reference_rowwise.
"""

import numpy as np
import pytest
import torch

from oracle import block_fp8, moe, synth


@pytest.mark.parametrize("t,e,k", [(200, 8, 2), (64, 3, 1), (50, 2, 2), (33, 16, 2)])
def test_route_matches_loop(t, e, k):
    rng = np.random.default_rng(t * 31 + e)
    lg = rng.standard_normal((t, e)).astype(np.float32)
    ids, w = moe.route(lg, k)
    ids2, w2 = moe.route_loop(lg, k)
    assert np.array_equal(ids, ids2)
    assert np.array_equal(w, w2)
    assert np.all(lg[np.arange(t), ids[:, 0]] == lg.max(1))
    if k == 2:
        assert np.all(ids[:, 0] != ids[:, 1])
        assert np.all(w[:, 0] >= w[:, 1])
    np.testing.assert_allclose(w.sum(1), 1.0, rtol=0, atol=2e-7)


def test_route_ties_go_to_lower_index():
    lg = np.array([[1, 1, 1, 1], [0, 2, 2, 1], [3, 0, 3, 3], [-1, -1, 5, -1]], dtype=np.float32)
    ids, w = moe.route(lg, 2)
    assert ids.tolist() == [[0, 1], [1, 2], [0, 2], [2, 0]]
    assert w[0].tolist() == [0.5, 0.5] and w[1].tolist() == [0.5, 0.5] and w[2].tolist() == [0.5, 0.5]
    # softmax of (5, -1): 1 / (1 + e^-6)
    assert abs(float(w[3, 0]) - 1.0 / (1.0 + np.exp(-6.0))) < 1e-7
    ids2, _ = moe.route_loop(lg, 2)
    assert np.array_equal(ids, ids2)
    # integer logits over a small range: ties everywhere
    rng = np.random.default_rng(5)
    lg = rng.integers(-2, 3, size=(300, 6)).astype(np.float32)
    assert np.array_equal(moe.route(lg, 2)[0], moe.route_loop(lg, 2)[0])


@pytest.mark.parametrize("align", [256, 16])
def test_layout_invariants(align):
    rng = np.random.default_rng(7)
    t, e, k = 300, 8, 2
    ids, _ = moe.route(rng.standard_normal((t, e)).astype(np.float32), k)
    ids[:40] = [0, 1]  # skew the counts
    row_token, row_slot, row_of, off, counts = moe.layout(ids, e, align)
    assert np.all(off % align == 0) and off[0] == 0
    assert np.array_equal(counts, np.bincount(ids.reshape(-1), minlength=e))
    for x in range(e):
        seg = row_token[off[x]:off[x + 1]]
        live = seg[: counts[x]]
        assert np.all(seg[counts[x]:] == -1)
        assert np.array_equal(live, np.sort(np.nonzero((ids == x).any(1))[0]))  # stable: token order
        assert np.all(ids[live, row_slot[off[x]:off[x] + counts[x]]] == x)
    # every (token, slot) pair appears exactly once, and row_of inverts row_token
    assert np.array_equal(row_token[row_of], np.repeat(np.arange(t)[:, None], k, 1))
    assert np.array_equal(row_slot[row_of], np.tile(np.arange(k), (t, 1)))
    assert (row_token >= 0).sum() == t * k


def test_layout_empty_expert():
    ids = np.array([[2, 0], [2, 0], [0, 2]])
    row_token, _, row_of, off, counts = moe.layout(ids, 4, 256)
    assert counts.tolist() == [3, 0, 3, 0]
    assert off.tolist() == [0, 256, 256, 512, 512]
    assert row_token[:4].tolist() == [0, 1, 2, -1] and row_token[256:259].tolist() == [0, 1, 2]
    assert row_of.tolist() == [[256, 0], [257, 1], [2, 258]]


def test_silu_mul_against_fp64_and_special_cases():
    gen = torch.Generator().manual_seed(3)
    gu = (torch.randn(64, 512, generator=gen) * 6).bfloat16()
    got = moe.silu_mul(gu).double()
    want = moe.silu_mul_f64(gu)
    # one bf16 rounding of a value within a few fp32 ulps of the fp64 result
    assert torch.all((got - want).abs() <= want.abs() * 2.0 ** -8 + 1e-30)
    inf, nan = float("inf"), float("nan")
    g = torch.tensor([[0.0, -88.0, -100.0, 200.0, 1.0, -87.5, inf, -inf, nan]]).bfloat16()
    u = torch.tensor([[3.0, 5.0, 5.0, 2.0, 1.0, 1e30, 1.0, 1.0, 1.0]]).bfloat16()
    out = moe.silu_mul(torch.cat([g, u], 1)).float()[0]
    assert out[0] == 0 and out[1] == 0 and out[2] == 0
    assert out[3] == float(torch.tensor(400.0).bfloat16())                  # silu(g) = g for large g
    assert out[4] == float(torch.tensor(1.0 / (1.0 + np.exp(-1.0))).bfloat16())
    assert out[5] != 0                                                       # -87.5 is above the cutoff
    # silu_and_mul_bf16.c:8-12: +inf -> (-inf + inf) = NaN; -inf <= -88 -> 0; NaN passes through
    assert torch.isnan(out[6]) and out[7] == 0 and torch.isnan(out[8])


def _small_problem(t, h, inter, e, seed):
    x = synth.activations(t, h, seed)
    gen = torch.Generator().manual_seed(seed + 1)
    logits = torch.randn(t, e, generator=gen)
    wg, sg, wd, sd = [], [], [], []
    for i in range(e):
        a, b = synth.weight(2 * inter, h, seed=seed + 10 + i)
        c, d = synth.weight(h, inter, seed=seed + 100 + i)
        wg.append(a); sg.append(b); wd.append(c); sd.append(d)
    return x, logits, torch.stack(wg), torch.stack(sg), torch.stack(wd), torch.stack(sd)


@pytest.mark.parametrize("top_k", [1, 2])
def test_moe_reference_against_per_token_evaluation(top_k):
    x, logits, wg, sg, wd, sd = _small_problem(12, 256, 128, 4, 40 + top_k)
    y = moe.moe_reference(x, logits, wg, sg, wd, sd, top_k=top_k)
    ids, w = moe.route_loop(logits.numpy(), top_k)
    for t in range(x.shape[0]):
        acc = None
        for k in range(top_k):
            e = int(ids[t, k])
            hpre = block_fp8.reference_rowwise(x[t:t + 1], wg[e], sg[e])
            g, u = hpre[:, :128].float(), hpre[:, 128:].float()
            h = (g / (1.0 + torch.exp(-g)) * u).bfloat16()
            z = block_fp8.reference_rowwise(h, wd[e], sd[e]).float()[0]
            p = torch.tensor(float(w[t, k]), dtype=torch.float32) * z
            acc = p if acc is None else acc + p
        assert torch.equal(y[t], acc.bfloat16()), t
    # the `tokens` selection returns the same rows
    sel = [7, 2, 11]
    assert torch.equal(moe.moe_reference(x, logits, wg, sg, wd, sd, top_k=top_k, tokens=sel), y[sel])
