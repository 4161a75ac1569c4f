"""Pins the oracle's canonical router/grouping functions (kernels/drama.cu:317-468,744-778).

Checks against float64 restatements, special cases whose answer the mathematics fixes
(one-hot, ties, E == topk, exact small-integer sums) and brute force.
"""
import numpy as np

import oracle as O
import synth


def test_rmsnorm_canon_vs_float64():
    rng = np.random.default_rng(0)
    for K in (2048, 512, 4096):
        x = rng.normal(0, 1, K).astype(np.float32)
        nw = (1 + rng.normal(0, 0.1, K)).astype(np.float32)
        xn = O.rmsnorm(x, nw, 1e-6)
        ref = x.astype(np.float64) / np.sqrt(np.mean(x.astype(np.float64) ** 2) + 1e-6) * nw
        np.testing.assert_allclose(xn, ref, rtol=2e-6, atol=1e-7)
    np.testing.assert_array_equal(O.rmsnorm(x, None, 1e-6), x)


def test_dot_canon_exact_small_integers_and_float64():
    rng = np.random.default_rng(1)
    K = 2048
    w = rng.integers(-8, 9, K).astype(np.float32)
    x = rng.integers(-8, 9, K).astype(np.float32)
    wb = synth.f32_to_bf16(w)
    assert O.lib().or_dot_bf16_canon(wb.ctypes.data, x.ctypes.data, K) == float(np.dot(w.astype(np.int64), x.astype(np.int64)))
    W = synth.f32_to_bf16(rng.normal(0, 0.02, (64, K)).astype(np.float32))
    xr = rng.normal(0, 1, K).astype(np.float32)
    out = np.empty(64, np.float32)
    O.lib().or_router_logits(W.ctypes.data, xr.ctypes.data, 64, K, out.ctypes.data)
    ref = synth.bf16_to_f32(W).astype(np.float64) @ xr.astype(np.float64)
    np.testing.assert_allclose(out, ref, rtol=0, atol=2e-5)
    # a transposed/shifted chunk mapping would still be exact on constants; a wrong element
    # pairing is caught here: element k of w pairs with element k of x
    one_hot = np.zeros(K, np.float32)
    for k in (0, 7, 8, 511, 512, 2047):
        one_hot[:] = 0
        one_hot[k] = 1
        assert O.lib().or_dot_bf16_canon(W[3].ctypes.data, one_hot.ctypes.data, K) == synth.bf16_to_f32(W[3])[k]


def test_softmax_topk_special_cases():
    E, topk = 256, 8
    # one-hot: the hot expert gets (almost) all the mass and comes first
    l = np.full(E, -10, np.float32)
    l[77] = 10.0
    idx, w = O.softmax_topk(l, E, topk)
    assert idx[0] == 77
    np.testing.assert_array_equal(idx[1:], np.arange(7))  # remaining ties break to low indices
    # all equal: first topk indices, equal weights 1/topk exactly
    idx, w = O.softmax_topk(np.zeros(E, np.float32), E, topk)
    np.testing.assert_array_equal(idx, np.arange(8))
    np.testing.assert_array_equal(w, np.full(8, 0.125, np.float32))
    # E == topk: everything selected, sorted by logit desc, weights = softmax
    rng = np.random.default_rng(2)
    l8 = rng.normal(0, 1, 8).astype(np.float32)
    idx, w = O.softmax_topk(l8, 8, 8)
    np.testing.assert_array_equal(idx, np.argsort(-l8, kind="stable"))
    sm = np.exp(l8 - l8.max())
    sm /= sm.sum()
    np.testing.assert_allclose(w, sm[idx], rtol=1e-6)
    assert abs(float(w.astype(np.float64).sum()) - 1.0) < 1e-6


def test_softmax_topk_brute_force():
    rng = np.random.default_rng(3)
    for trial in range(200):
        E = int(rng.choice([8, 16, 64, 200, 256]))
        topk = int(min(E, rng.choice([1, 2, 8, 32])))
        l = rng.normal(0, 2, E).astype(np.float32)
        if trial % 5 == 0:
            l = np.round(l * 2) / 2  # many exact ties
        idx, w = O.softmax_topk(l, E, topk)
        # selection is the (logit desc, index asc) order, -0 just below +0
        order = sorted(range(E), key=lambda e: (-float(l[e]), bool(np.signbit(l[e])), e))[:topk]
        np.testing.assert_array_equal(idx, order)
        p = np.exp(l.astype(np.float64) - l.max())
        p /= p.sum()
        np.testing.assert_allclose(w, p[idx] / p[idx].sum(), rtol=2e-6)


def test_router_topk_full():
    rng = np.random.default_rng(4)
    E, K = 256, 2048
    W = synth.f32_to_bf16(rng.normal(0, 0.02, (E + 1, K)).astype(np.float32))
    x = rng.normal(0, 1, K).astype(np.float32)
    nw = (1 + rng.normal(0, 0.1, K)).astype(np.float32)
    logits, idx, w, sg = O.router_topk(W, x, nw, 1e-6, E, 8)
    xn64 = x.astype(np.float64) / np.sqrt(np.mean(x.astype(np.float64) ** 2) + 1e-6) * nw
    ref = synth.bf16_to_f32(W).astype(np.float64) @ xn64
    np.testing.assert_allclose(logits, ref, atol=2e-5)
    assert sg == logits[E]
    sel, _ = O.softmax_topk(logits[:E].copy(), E, 8)
    np.testing.assert_array_equal(idx, sel)
    rows = O.router_logits_rows(synth.f32_to_bf16(x)[None, :].copy(), W, 1, E + 1, K)
    np.testing.assert_allclose(rows[0], synth.bf16_to_f32(W).astype(np.float64) @ synth.bf16_to_f32(synth.f32_to_bf16(x)),
                               atol=2e-5)


def test_moe_topk_rows_matches_single_row():
    rng = np.random.default_rng(5)
    rows, E = 40, 256
    logits = rng.normal(0, 1, (rows, E + 3)).astype(np.float32)
    idx, w, sg = O.moe_topk(logits, rows, E, 8, E + 3)
    for r in range(rows):
        i1, w1 = O.softmax_topk(logits[r, :E].copy(), E, 8)
        np.testing.assert_array_equal(idx[r * 8:(r + 1) * 8], i1)
        np.testing.assert_array_equal(w[r * 8:(r + 1) * 8], w1)
        assert sg[r] == logits[r, E]


def test_group_invariants_and_brute_force():
    rng = np.random.default_rng(6)
    for n, E in ((2400, 256), (17, 4), (1, 1), (0, 8), (8192, 256)):
        idx = rng.integers(0, E, n).astype(np.int32)
        counts, offsets, slot_of = O.moe_group(idx, E)
        np.testing.assert_array_equal(counts, np.bincount(idx, minlength=E))
        np.testing.assert_array_equal(offsets, np.concatenate([[0], np.cumsum(counts)[:-1]]).astype(np.int32))
        assert counts.sum() == n
        assert np.array_equal(np.sort(slot_of), np.arange(n))
        # brute force: stable sort by expert
        perm = np.argsort(idx, kind="stable")
        expect = np.empty(n, np.int32)
        expect[perm] = np.arange(n)
        np.testing.assert_array_equal(slot_of, expect)


def test_softmax_topk_signed_zero_and_infinities():
    """-0 ranks just below +0 (key order), -inf is a number above NaN; weights stay exact."""
    l = np.full(16, -np.inf, np.float32)
    l[3], l[9] = -0.0, 0.0
    idx, w = O.softmax_topk(l, 16, 3)
    assert list(idx) == [9, 3, 0]
    np.testing.assert_array_equal(w, np.array([0.5, 0.5, 0.0], np.float32))


def test_softmax_topk_nan_logits_pick_distinct_valid_experts():
    """NaN logits rank below every number, picks never leave [0, E) and never repeat."""
    for E in (256, 16, 8):
        l = np.full(E, np.nan, np.float32)
        idx, w = O.softmax_topk(l, E, 8)
        np.testing.assert_array_equal(idx, np.arange(8))
        l = np.random.default_rng(E).normal(0, 1, E).astype(np.float32)
        l[[1, 3]] = np.nan  # NaN poisons the sum (every weight is NaN), not the selection
        idx, w = O.softmax_topk(l, E, 8)
        assert len(set(idx.tolist())) == 8 and idx.min() >= 0 and idx.max() < E
        if E > 10:
            assert 1 not in idx and 3 not in idx
