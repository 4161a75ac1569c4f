"""Pins the oracle's MoE value functions (tools/reference.py:331-351, kernels/drama.cu:470-968)
with an independent float64 numpy restatement (dequantisation written with numpy bit
operations, dense matmuls) and invariants the mathematics fixes: a single expert of weight
1 with the shared gate at -inf is a plain SwiGLU MLP, permuting expert storage and remapping
indices changes nothing, an all-zero expert contributes nothing, the prefill expert path on
one token equals the decode path on the bf16-rounded input."""
import numpy as np
import pytest

import oracle as O
import synth

H, I = 2048, 512


def np_dequant_q4(q, sm, kind):
    """numpy restatement: low nibble is element 2b, high nibble 2b+1; w = q * scale + min."""
    N = q.shape[0]
    nib = np.empty((N, q.shape[1] * 2), np.float32)
    nib[:, 0::2] = q & 15
    nib[:, 1::2] = q >> 4
    s = synth.dec(sm[..., 0], kind)
    m = synth.dec(sm[..., 1], kind)
    g = nib.reshape(N, -1, 64)
    return (g * s[..., None] + m[..., None]).reshape(N, -1).astype(np.float64)


def np_dequant_q8(q, s, kind, group):
    N, K = q.shape
    sc = synth.dec(s, kind).reshape(N, -1)
    return (q.astype(np.float64).reshape(N, K // group, group) * sc[..., None]).reshape(N, K)


def np_dequant_fp8(w8, s, kind):
    N, K = w8.shape
    v = synth.E4M3[w8].astype(np.float64)
    sc = synth.dec(s, kind).reshape(N // 128, K // 128).astype(np.float64)
    return v * np.repeat(np.repeat(sc, 128, 0), 128, 1)


def np_silu(v):
    return v / (1 + np.exp(-v))


def np_moe_decode(L, x, idx, wts, sg, res, nw):
    xn = O.rmsnorm(x, nw, 1e-6).astype(np.float64) if nw is not None else x.astype(np.float64)
    acts = []
    for e in idx:
        if L["kind"] == "q4":
            gu = np_dequant_q4(L["gu_q"][e], L["gu_s"][e], L["sc_kind"])
            d = np_dequant_q4(L["d_q"][e], L["d_s"][e], L["sc_kind"])
        else:
            gu = np_dequant_fp8(L["gu_q"][e], L["gu_s"][e], L["sc_kind"])
            d = np_dequant_fp8(L["d_q"][e], L["d_s"][e], L["sc_kind"])
        h = gu @ xn
        acts.append((np_silu(h[:I]) * h[I:], d))
    sgu = np_dequant_q8(L["sgu_q"], L["sgu_s"], L["sh_kind"], L["sh_group_gu"])
    sd = np_dequant_q8(L["sd_q"], L["sd_s"], L["sh_kind"], L["sh_group_d"])
    hs = sgu @ xn
    sact = np_silu(hs[:I]) * hs[I:]
    y = res.astype(np.float64) + 1 / (1 + np.exp(-float(sg))) * (sd @ sact.astype(np.float32).astype(np.float64))
    for w, (a, d) in zip(wts, acts):
        y += float(w) * (d @ a.astype(np.float32).astype(np.float64))
    return y


@pytest.fixture(scope="module", params=[("cfg", "q4"), ("ref", "q4"), ("cfg", "fp8"), ("ref", "fp8")])
def layer(request):
    fmt, kind = request.param
    return synth.make_layer(7, E=12, fmt=fmt, kind=kind)


def test_decode_vs_numpy_restatement(layer):
    rng = np.random.default_rng(8)
    x = rng.normal(0, 1, H).astype(np.float32)
    res = rng.normal(0, 1, H).astype(np.float32)
    _, idx, wts, sg = O.router_topk(layer["router"], x, layer["nw"], 1e-6, layer["E"], 8)
    act, y = O.moe_decode(layer, x, idx, wts, sg, res, H, I, 8, nw=layer["nw"], eps=1e-6)
    ref = np_moe_decode(layer, x, idx, wts, sg, res, layer["nw"])
    np.testing.assert_allclose(y, ref, rtol=1e-5, atol=1e-5)


def test_single_expert_is_swiglu_mlp():
    L = synth.make_layer(9, E=8, fmt="cfg")
    rng = np.random.default_rng(10)
    x = rng.normal(0, 1, H).astype(np.float32)
    idx = np.array([3, 0, 1, 2, 4, 5, 6, 7], np.int32)
    wts = np.array([1, 0, 0, 0, 0, 0, 0, 0], np.float32)
    zero = np.zeros(H, np.float32)
    act, y = O.moe_decode(L, x, idx, wts, -np.inf, zero, H, I, 8)
    gu = np_dequant_q4(L["gu_q"][3], L["gu_s"][3], L["sc_kind"])
    d = np_dequant_q4(L["d_q"][3], L["d_s"][3], L["sc_kind"])
    h = gu @ x.astype(np.float64)
    np.testing.assert_allclose(y, d @ (np_silu(h[:I]) * h[I:]), rtol=1e-5, atol=1e-5)


def test_expert_storage_permutation_invariance():
    L = synth.make_layer(11, E=10, fmt="ref")
    rng = np.random.default_rng(12)
    x = rng.normal(0, 1, H).astype(np.float32)
    _, idx, wts, sg = O.router_topk(L["router"], x, L["nw"], 1e-6, 10, 8)
    _, y = O.moe_decode(L, x, idx, wts, sg, x, H, I, 8, nw=L["nw"], eps=1e-6)
    perm = rng.permutation(10)
    P = dict(L)
    for k in ("gu_q", "gu_s", "d_q", "d_s"):
        P[k] = np.ascontiguousarray(L[k][perm])
    inv = np.argsort(perm).astype(np.int32)
    _, y2 = O.moe_decode(P, x, inv[idx], wts, sg, x, H, I, 8, nw=L["nw"], eps=1e-6)
    np.testing.assert_allclose(y2, y, rtol=1e-6, atol=1e-6)


def test_zero_expert_contributes_nothing():
    L = synth.make_layer(13, E=9, fmt="cfg")
    Z = dict(L)
    for k in ("d_q", "d_s"):
        Z[k] = L[k].copy()
    Z["d_q"][2] = 0
    Z["d_s"][2] = 0  # scale 0, min 0
    rng = np.random.default_rng(14)
    x = rng.normal(0, 1, H).astype(np.float32)
    idx = np.array([2, 0, 1, 3, 4, 5, 6, 7], np.int32)
    wts = np.full(8, 0.125, np.float32)
    _, y = O.moe_decode(Z, x, idx, wts, 0.0, x, H, I, 8)
    wts2 = wts.copy()
    wts2[0] = 0
    _, y2 = O.moe_decode(Z, x, idx, wts2, 0.0, x, H, I, 8)
    np.testing.assert_array_equal(y, y2)


def test_prefill_expert_path_equals_decode_rows_on_one_token():
    L = synth.make_layer(15, E=6, fmt="cfg")
    rng = np.random.default_rng(16)
    xb = synth.f32_to_bf16(rng.normal(0, 1, (1, H)).astype(np.float32))
    counts = np.array([0, 0, 1, 0, 0, 0], np.int32)
    offsets = np.array([0, 0, 0, 1, 1, 1], np.int32)
    act, yp = O.moe_prefill_experts(L, xb, offsets, counts, 6, H, I)
    gu = np_dequant_q4(L["gu_q"][2], L["gu_s"][2], L["sc_kind"])
    d = np_dequant_q4(L["d_q"][2], L["d_s"][2], L["sc_kind"])
    h = gu @ synth.bf16_to_f32(xb[0]).astype(np.float64)
    a = synth.bf16_to_f32(synth.f32_to_bf16((np_silu(h[:I]) * h[I:]).astype(np.float32)))
    np.testing.assert_array_equal(act[0], synth.f32_to_bf16(a))
    np.testing.assert_allclose(yp[0], d @ a.astype(np.float64), rtol=1e-5, atol=1e-5)


def test_prefill_layer_matches_per_row_composition():
    """or_moe_prefill_layer == x + sigmoid(sg) shared + sum_k w_k expert_k, row by row."""
    L = synth.make_layer(17, E=16, fmt="cfg")
    rng = np.random.default_rng(18)
    rows, topk = 5, 8
    hn = synth.f32_to_bf16(rng.normal(0, 1, (rows, H)).astype(np.float32))
    x0 = rng.normal(0, 1, (rows, H)).astype(np.float32)
    logits = O.router_logits_rows(hn, L["router"], rows, 17, H)
    idx, wts, sg = O.moe_topk(logits, rows, 16, topk, 17)
    out = O.moe_prefill_layer(L, hn, rows, idx, wts, sg, x0, H, I, topk)
    sact, sh = O.shared_prefill(L, hn, rows, H, I)
    for r in range(rows):
        acc = x0[r].astype(np.float64) + 1 / (1 + np.exp(-float(sg[r]))) * sh[r]
        for k in range(topk):
            e = idx[r * topk + k]
            c = np.zeros(16, np.int32)
            c[e] = 1
            off = np.concatenate([[0], np.cumsum(c)[:-1]]).astype(np.int32)
            _, yp = O.moe_prefill_experts(L, hn[r:r + 1].copy(), off, c, 16, H, I)
            acc += float(wts[r * topk + k]) * yp[0]
        np.testing.assert_allclose(out[r], acc, rtol=1e-5, atol=1e-5)


def test_gemv_q4_and_q8_vs_numpy():
    rng = np.random.default_rng(19)
    q, sm = synth.q4_experts(rng, 1, 64, 2048, synth.BF16)
    x = rng.normal(0, 1, 2048).astype(np.float32)
    np.testing.assert_allclose(O.gemv_q4(q[0], sm[0], O.BF16, x, 64, 2048),
                               np_dequant_q4(q[0], sm[0], synth.BF16) @ x.astype(np.float64), rtol=1e-5, atol=1e-5)
    q8, s8, kind, group = synth.q8_dense(rng, 64, 2048, "ref")
    np.testing.assert_allclose(O.gemv_q8(q8, s8, kind, group, x, 64, 2048),
                               np_dequant_q8(q8, s8, kind, group) @ x.astype(np.float64), rtol=1e-5, atol=1e-5)


@pytest.mark.parametrize("fmt,E", [("cfg", 64), ("ref", 12)])
def test_cpu_baseline_layer_matches_oracle(fmt, E):
    """The fp32 host baseline bench.py times (or_cpu_layer_f32) computes the oracle's layer:
    the same experts and weights (its own fp32 router agrees on these seeded inputs) and y
    within 1e-3 + 1e-3 |ref| of or_moe_decode, on 1 and on several threads (same values)."""
    L = synth.make_layer(31, E=E, fmt=fmt)
    x = np.random.default_rng(32).normal(0, 1, H).astype(np.float32)
    res = np.random.default_rng(33).normal(0, 1, H).astype(np.float32)
    _, ri, rw, rs = O.router_topk(L["router"], x, L["nw"], 1e-6, E, 8)
    _, ry = O.moe_decode(L, x, ri, rw, rs, res, H, I, 8, nw=L["nw"], eps=1e-6)
    n0 = O.lib().or_num_threads()
    try:
        for th in (1, 4):
            O.lib().or_set_threads(th)
            idx, wts, y = O.cpu_layer_f32(L, x, res, H, I, 8)
            np.testing.assert_array_equal(idx, ri)
            np.testing.assert_allclose(wts, rw, rtol=1e-5, atol=1e-7)
            assert np.all(np.abs(y.astype(np.float64) - ry) <= 1e-3 + 1e-3 * np.abs(ry))
    finally:
        O.lib().or_set_threads(n0)
