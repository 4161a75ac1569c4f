"""GPU parity of the prefill path through the C ABI: grouping (exact), expert-grouped int4/fp8
MFMA GEMM, fused int8 shared expert, combine, and the whole layer chain of
Engine::moe_prefill (src/engine.rs:544-604) against the oracle.

act is bf16 (kernels/drama.cu:879): it must match the oracle within one bf16 ulp (a last-bit
rounding flip when the fp32 sums differ in their last bits).  fp32 outputs are checked with
|gpu - ref| <= 1e-3 + 1e-3 |ref|; the down projection is checked on the GPU's own act so both
sides multiply identical inputs."""
import numpy as np
import pytest

import dramamoe as D
import oracle as O
import synth
from helpers import assert_close, dev, host

pytestmark = pytest.mark.gpu
H, I = 2048, 512


def t_i32(n):
    import torch

    return torch.zeros(n, dtype=torch.int32, device="cuda")


def check_act(act, ract, what="act"):
    """bf16 act within one rounding flip: |a - r| <= 2^-7 |r| + 1e-3 (1e-3 covers u ~ 0
    cancellation, where fp32-vs-fp64 sums differ by ~1e-6 absolute)."""
    a, r = synth.bf16_to_f32(act).astype(np.float64), synth.bf16_to_f32(ract).astype(np.float64)
    bad = np.abs(a - r) > 2.0 ** -7 * np.abs(r) + 1e-3
    assert not bad.any(), f"{what}: {int(bad.sum())} elements beyond one bf16 rounding flip"
    return a, r


def assert_close_with_flips(y, ref, Dmat, a, r, what):
    """|y - ref| <= 1e-3 + 1e-3 |ref| + sum_j |D[n, j]| |a_j - r_j|: the tolerance plus exactly the
    propagation of the act rounding flips observed (bf16 act, kernels/drama.cu:879)."""
    extra = np.abs(a - r) @ np.abs(Dmat).T
    err = np.abs(np.asarray(y, np.float64) - ref)
    bad = err > 1e-3 + 1e-3 * np.abs(ref) + extra
    assert not bad.any(), f"{what}: {int(bad.sum())}/{bad.size} outside tolerance + flip propagation"


def bf16_ulp_diff(a, b):
    a = a.astype(np.int32)
    b = b.astype(np.int32)
    sa, sb = a >> 15, b >> 15
    # map sign-magnitude bf16 to a monotone integer line
    ia = np.where(sa == 1, -(a & 0x7FFF), a & 0x7FFF)
    ib = np.where(sb == 1, -(b & 0x7FFF), b & 0x7FFF)
    return np.abs(ia - ib)


@pytest.mark.parametrize("n,E,skew", [(2400, 256, False), (2400, 256, True), (1, 256, False), (8192, 256, False),
                                      (17, 4, False), (0, 8, False)])
def test_group_exact(n, E, skew):
    import torch

    rng = np.random.default_rng(n + E)
    if skew:  # 10% of experts receive 50% of the pairs
        hot = rng.choice(E, E // 10, replace=False)
        idx = np.where(rng.random(n) < 0.5, rng.choice(hot, n), rng.integers(0, E, n)).astype(np.int32)
    else:
        idx = rng.integers(0, E, n).astype(np.int32)
    rc, ro, rs = O.moe_group(idx, E)
    counts, offsets, slot_of = t_i32(E), t_i32(E), t_i32(max(n, 1))
    didx = dev(idx) if n else t_i32(1)
    D.lib().dr_moe_group(D.ptr(didx), n, E, D.ptr(counts), D.ptr(offsets), D.ptr(slot_of), D.stream_ptr())
    torch.cuda.synchronize()
    np.testing.assert_array_equal(host(counts), rc)
    np.testing.assert_array_equal(host(offsets), ro)
    if n:
        np.testing.assert_array_equal(host(slot_of)[:n], rs)


@pytest.mark.parametrize("rows", [300, 4, 8, 9])
def test_count_and_permute_reference_abi(rows):
    """dr_moe_count + host scan + dr_moe_permute, the reference's sequence (src/engine.rs:564-578),
    at prefill and decode-batch row counts."""
    import torch

    rng = np.random.default_rng(3 + rows)
    topk, E = 8, 256
    idx = rng.integers(0, E, rows * topk).astype(np.int32)
    x = synth.f32_to_bf16(rng.normal(0, 1, (rows, H)).astype(np.float32))
    rc, ro, rs = O.moe_group(idx, E)
    L = D.lib()
    didx, counts = dev(idx), t_i32(E)
    L.dr_moe_count(D.ptr(didx), rows * topk, D.ptr(counts), D.stream_ptr())
    torch.cuda.synchronize()
    np.testing.assert_array_equal(host(counts), rc)
    offsets, fill, slot_of = dev(ro), t_i32(E), t_i32(rows * topk)
    dx = dev(x)
    xp = torch.zeros(rows * topk * H, dtype=torch.int16, device="cuda")
    L.dr_moe_permute(D.ptr(didx), rows, topk, D.ptr(offsets), D.ptr(fill), D.ptr(slot_of), D.ptr(dx), D.ptr(xp), H,
                     D.stream_ptr())
    torch.cuda.synchronize()
    np.testing.assert_array_equal(host(slot_of), rs)
    np.testing.assert_array_equal(host(fill), rc)
    xph = host(xp).view(np.uint16).reshape(rows * topk, H)
    np.testing.assert_array_equal(xph[rs], x[np.arange(rows * topk) // topk])


@pytest.mark.parametrize("rows,E", [(5, 8), (37, 24), (1100, 64)])
def test_permute_touches_only_routed_experts(rows, E):
    """offsets/fill sized for E < 256 experts with guard words behind them: the permute must
    leave the guards alone (it reads and writes only experts that occur), and 1100 rows x 8
    (8800 pairs, beyond one 8192-pair segment) must still give the stable slots."""
    import torch

    rng = np.random.default_rng(40 + rows)
    topk = 8
    idx = rng.integers(0, E, rows * topk).astype(np.int32)
    if E > 8:
        idx[idx == 3] = 4  # one expert that never occurs
    x = synth.f32_to_bf16(rng.normal(0, 1, (rows, H)).astype(np.float32))
    rc, ro, rs = O.moe_group(idx, E)
    guard = np.int32(-0x3C3C3C3D)
    off_g = np.concatenate([ro, np.full(256, guard, np.int32)])
    offsets, fill = dev(off_g), dev(np.concatenate([np.zeros(E, np.int32), np.full(256, guard, np.int32)]))
    didx, slot_of, dx = dev(idx), t_i32(rows * topk), dev(x)
    xp = torch.zeros(rows * topk * H, dtype=torch.int16, device="cuda")
    D.lib().dr_moe_permute(D.ptr(didx), rows, topk, D.ptr(offsets), D.ptr(fill), D.ptr(slot_of), D.ptr(dx), D.ptr(xp),
                           H, D.stream_ptr())
    torch.cuda.synchronize()
    np.testing.assert_array_equal(host(slot_of), rs)
    f = host(fill)
    np.testing.assert_array_equal(f[:E], rc)
    assert (f[E:] == guard).all() and (host(offsets)[E:] == guard).all(), "guard words after E entries changed"
    xph = host(xp).view(np.uint16).reshape(rows * topk, H)
    np.testing.assert_array_equal(xph[rs], x[np.arange(rows * topk) // topk])


def grouped_inputs(seed, E, rows, topk, skew=False):
    rng = np.random.default_rng(seed)
    n = rows * topk
    if skew:
        hot = rng.choice(E, max(1, E // 10), replace=False)
        idx = np.where(rng.random(n) < 0.5, rng.choice(hot, n), rng.integers(0, E, n)).astype(np.int32)
    else:
        idx = np.stack([rng.choice(E, topk, replace=False) for _ in range(rows)]).ravel().astype(np.int32)
    counts, offsets, slot_of = O.moe_group(idx, E)
    x = synth.f32_to_bf16(rng.normal(0, 1, (rows, H)).astype(np.float32))
    xp = np.empty((n, H), np.uint16)
    xp[slot_of] = x[np.arange(n) // topk]
    return idx, counts, offsets, slot_of, x, xp


def run_prefill(Lh, xp, offsets, counts, fmt, kind):
    import torch

    E = Lh["E"]
    n = xp.shape[0]
    t = {k: dev(Lh[k]) for k in ("gu_q", "gu_s", "d_q", "d_s")}
    dxp, doff, dcnt = dev(xp), dev(offsets), dev(counts)
    act = torch.zeros(n * I, dtype=torch.int16, device="cuda")
    yp = torch.zeros(n * H, dtype=torch.float32, device="cuda")
    name = {("q4", "ref"): "dr_moe_prefill", ("q4", "cfg"): "dr_moe_prefill_bf16s",
            ("fp8", "ref"): "dr_moe_prefill_fp8", ("fp8", "cfg"): "dr_moe_prefill_fp8_bf16s"}[(kind, fmt)]
    getattr(D.lib(), name)(D.ptr(t["gu_q"]), D.ptr(t["gu_s"]), D.ptr(t["d_q"]), D.ptr(t["d_s"]), D.ptr(dxp), D.ptr(doff),
                           D.ptr(dcnt), D.ptr(act), D.ptr(yp), E, H, I, D.stream_ptr())
    torch.cuda.synchronize()
    return host(act).view(np.uint16).reshape(n, I), host(yp).reshape(n, H)


def expert_dense(Lh, which, e):
    """Dequantised [N, K] matrix of expert e via the oracle."""
    kind = Lh["kind"]
    q, s = Lh[which + "_q"][e], Lh[which + "_s"][e]
    N = q.shape[0]
    if kind == "q4":
        return O.dequant_q4(np.ascontiguousarray(q), np.ascontiguousarray(s), Lh["sc_kind"], N, q.shape[1] * 2)
    return O.dequant_fp8(np.ascontiguousarray(q), np.ascontiguousarray(s), Lh["sc_kind"], N, q.shape[1])


@pytest.mark.parametrize("fmt,kind,skew", [("cfg", "q4", False), ("ref", "q4", False), ("cfg", "q4", True),
                                           ("cfg", "fp8", False), ("ref", "fp8", False)])
def test_grouped_gemm(fmt, kind, skew):
    E, rows, topk = 24, 96, 8
    Lh = synth.make_layer(40 + (kind == "fp8"), E=E, fmt=fmt, kind=kind)
    idx, counts, offsets, slot_of, x, xp = grouped_inputs(41, E, rows, topk, skew)
    act, yp = run_prefill(Lh, xp, offsets, counts, fmt, kind)
    ract, ryp = O.moe_prefill_experts(Lh, xp, offsets, counts, E, H, I)
    af, rf = check_act(act, ract)
    print(f"counts min {counts.min()} max {counts.max()}; act rounding flips: {int((af != rf).sum())}/{af.size}")
    for e in range(E):
        if counts[e] == 0:
            continue
        sl = slice(offsets[e], offsets[e] + counts[e])
        Dm = expert_dense(Lh, "d", e).astype(np.float64)
        assert_close(yp[sl], af[sl] @ Dm.T, what=f"down expert {e} on the GPU's act")
        assert_close_with_flips(yp[sl], ryp[sl].astype(np.float64), Dm, af[sl], rf[sl], f"expert {e} end to end")


@pytest.mark.parametrize("rows,E,topk", [(300, 256, 8), (1, 8, 8), (4, 256, 8), (1024, 256, 8), (37, 64, 12),
                                         (5, 24, 2)])
def test_topk_group_matches_oracle(rows, E, topk):
    """dr_moe_topk_group: idx / wts / sgate bit for bit as the oracle's top-k, counts / offsets /
    slot_of as its stable grouping, row_of_slot the inverse map, counter reset; logits with ties."""
    import torch

    rng = np.random.default_rng(rows * 7 + E + topk)
    lg = rng.normal(0, 1, (rows, E + 1)).astype(np.float32)
    lg[:, 1::5] = lg[:, 0:1]  # ties: equal logits across experts of a row
    ri, rw, rs = O.moe_topk(lg.ravel(), rows, E, topk, E + 1)
    rc, ro, rso = O.moe_group(ri, E)
    n = rows * topk
    dl, idx, wts, sg = dev(lg.ravel()), t_i32(n), torch.zeros(n, device="cuda"), torch.zeros(rows, device="cuda")
    counts, offsets, slot_of, row_of_slot, counter = t_i32(E), t_i32(E), t_i32(n), t_i32(n + 16), t_i32(4)
    D.lib().dr_moe_topk_group(D.ptr(dl), rows, E, topk, E + 1, D.ptr(idx), D.ptr(wts), D.ptr(sg), D.ptr(counts),
                              D.ptr(offsets), D.ptr(slot_of), D.ptr(row_of_slot), D.ptr(counter), D.stream_ptr())
    torch.cuda.synchronize()
    np.testing.assert_array_equal(host(idx), ri)
    np.testing.assert_array_equal(host(wts).view(np.uint32), rw.view(np.uint32))
    np.testing.assert_array_equal(host(sg).view(np.uint32), rs.view(np.uint32))
    np.testing.assert_array_equal(host(counts), rc)
    np.testing.assert_array_equal(host(offsets), ro)
    np.testing.assert_array_equal(host(slot_of), rso)
    np.testing.assert_array_equal(host(row_of_slot)[rso], np.arange(n) // topk)
    assert int(host(counter)[0]) == 0, "counter not reset"


@pytest.mark.parametrize("fmt,kind,skew", [("cfg", "q4", False), ("ref", "q4", False), ("cfg", "q4", True),
                                           ("cfg", "fp8", False), ("ref", "fp8", False)])
def test_prefill_rows_matches_gathered(fmt, kind, skew):
    """dr_moe_prefill_rows*: the token rows read through row_of_slot give the same act and y bits
    as the gathered xp through dr_moe_prefill*."""
    import torch

    E, rows, topk = 24, 96, 8
    Lh = synth.make_layer(40 + (kind == "fp8"), E=E, fmt=fmt, kind=kind)
    idx, counts, offsets, slot_of, x, xp = grouped_inputs(43, E, rows, topk, skew)
    act_ref, y_ref = run_prefill(Lh, xp, offsets, counts, fmt, kind)
    n = rows * topk
    ros = np.zeros(n + 16, np.int32)
    ros[slot_of] = np.arange(n) // topk
    t = {k: dev(Lh[k]) for k in ("gu_q", "gu_s", "d_q", "d_s")}
    dx, dros, doff, dcnt = dev(x), dev(ros), dev(offsets), dev(counts)
    act = torch.zeros(n * I, dtype=torch.int16, device="cuda")
    yp = torch.zeros(n * H, dtype=torch.float32, device="cuda")
    name = {("q4", "ref"): "dr_moe_prefill_rows", ("q4", "cfg"): "dr_moe_prefill_rows_bf16s",
            ("fp8", "ref"): "dr_moe_prefill_rows_fp8", ("fp8", "cfg"): "dr_moe_prefill_rows_fp8_bf16s"}[(kind, fmt)]
    getattr(D.lib(), name)(D.ptr(t["gu_q"]), D.ptr(t["gu_s"]), D.ptr(t["d_q"]), D.ptr(t["d_s"]), D.ptr(dx), rows,
                           D.ptr(dros), D.ptr(doff), D.ptr(dcnt), D.ptr(act), D.ptr(yp), E, H, I, D.stream_ptr())
    torch.cuda.synchronize()
    np.testing.assert_array_equal(host(act).view(np.uint16).reshape(n, I), act_ref)
    np.testing.assert_array_equal(host(yp).reshape(n, H).view(np.uint32), y_ref.view(np.uint32))


@pytest.mark.parametrize("fmt", ["cfg", "ref"])
@pytest.mark.parametrize("rows", [300, 33, 5, 1])
def test_shared_prefill(fmt, rows):
    import torch

    Lh = synth.make_layer(50, E=8, fmt=fmt)
    rng = np.random.default_rng(51)
    hn = synth.f32_to_bf16(rng.normal(0, 1, (rows, H)).astype(np.float32))
    t = {k: dev(Lh[k]) for k in ("sgu_q", "sgu_s", "sd_q", "sd_s")}
    dhn = dev(hn)
    act = torch.zeros(rows * I, dtype=torch.int16, device="cuda")
    out = torch.zeros(rows * H, dtype=torch.float32, device="cuda")
    name = "dr_moe_shared_prefill_bf16s" if fmt == "cfg" else "dr_moe_shared_prefill"
    getattr(D.lib(), name)(D.ptr(t["sgu_q"]), D.ptr(t["sgu_s"]), D.ptr(t["sd_q"]), D.ptr(t["sd_s"]), D.ptr(dhn), rows,
                           D.ptr(act), D.ptr(out), H, I, D.stream_ptr())
    torch.cuda.synchronize()
    ract, rout = O.shared_prefill(Lh, hn, rows, H, I)
    a = host(act).view(np.uint16).reshape(rows, I)
    af, rf = check_act(a, ract, "shared act")
    sd = O.dequant_q8(Lh["sd_q"], Lh["sd_s"], Lh["sh_kind"], Lh["sh_group_d"], H, I).astype(np.float64)
    o = host(out).reshape(rows, H)
    assert_close(o, af @ sd.T, what="shared out on the GPU's act")
    assert_close_with_flips(o, rout.astype(np.float64), sd, af, rf, "shared out end to end")


def test_combine():
    import torch

    rng = np.random.default_rng(60)
    rows, topk = 37, 8
    n = rows * topk
    x = rng.normal(0, 1, (rows, H)).astype(np.float32)
    y = rng.normal(0, 1, (n, H)).astype(np.float32)
    slot_of = rng.permutation(n).astype(np.int32)
    wts = rng.random((rows, topk)).astype(np.float32)
    sg = rng.normal(0, 2, rows).astype(np.float32)
    sh = rng.normal(0, 1, (rows, H)).astype(np.float32)
    dx = dev(x)
    dy, dso, dw, dsg, dsh = dev(y), dev(slot_of), dev(wts), dev(sg), dev(sh)
    D.lib().dr_moe_combine(D.ptr(dx), D.ptr(dy), D.ptr(dso), D.ptr(dw), D.ptr(dsg), D.ptr(dsh), rows, topk, H,
                           D.stream_ptr())
    torch.cuda.synchronize()
    sig = 1 / (1 + np.exp(-sg.astype(np.float64)))
    ref = x.astype(np.float64) + sig[:, None] * sh + np.einsum("rk,rkc->rc", wts.astype(np.float64),
                                                               y[slot_of.reshape(rows, topk)].astype(np.float64))
    assert_close(host(dx).reshape(rows, H), ref, rtol=1e-5, atol=1e-5, what="combine")


@pytest.mark.parametrize("fmt,path", [("cfg", "gather"), ("ref", "gather"), ("cfg", "rows"), ("ref", "rows")])
def test_prefill_layer_chain(fmt, path):
    """router GEMM -> top-k -> shared -> group -> gather -> grouped GEMM -> combine (E = 256);
    path "rows": top-k with grouping in one launch, the grouped GEMM reading hn through the slot
    map (dr_moe_topk_group + dr_moe_prefill_rows*)."""
    import torch

    E, rows, topk = 256, 300, 8
    Lh = synth.make_layer(70, E=E, fmt=fmt)
    rng = np.random.default_rng(71)
    hn = synth.f32_to_bf16(rng.normal(0, 1, (rows, H)).astype(np.float32))
    x0 = rng.normal(0, 1, (rows, H)).astype(np.float32)
    L, sp = D.lib(), D.stream_ptr()
    t = {k: dev(Lh[k]) for k in ("router", "gu_q", "gu_s", "d_q", "d_s", "sgu_q", "sgu_s", "sd_q", "sd_s")}
    dhn, dx = dev(hn), dev(x0)
    logits = torch.zeros(rows * (E + 1), dtype=torch.float32, device="cuda")
    idx, wts, sg = t_i32(rows * topk), torch.zeros(rows * topk, device="cuda"), torch.zeros(rows, device="cuda")
    h = np.zeros(1, np.uint64)
    L.dr_cublas_create(h.ctypes.data, sp)
    L.dr_gemm(int(h[0]), D.ptr(dhn), D.ptr(t["router"]), D.ptr(logits), rows, E + 1, H, 0.0)
    counts, offsets, slot_of = t_i32(E), t_i32(E), t_i32(rows * topk)
    row_of_slot, counter = t_i32(rows * topk + 16), t_i32(4)
    if path == "rows":
        L.dr_moe_topk_group(D.ptr(logits), rows, E, topk, E + 1, D.ptr(idx), D.ptr(wts), D.ptr(sg), D.ptr(counts),
                            D.ptr(offsets), D.ptr(slot_of), D.ptr(row_of_slot), D.ptr(counter), sp)
    else:
        L.dr_moe_topk(D.ptr(logits), rows, E, topk, E + 1, D.ptr(idx), D.ptr(wts), D.ptr(sg), sp)
    sact = torch.zeros(rows * I, dtype=torch.int16, device="cuda")
    sh = torch.zeros(rows * H, device="cuda")
    shname = "dr_moe_shared_prefill_bf16s" if fmt == "cfg" else "dr_moe_shared_prefill"
    getattr(L, shname)(D.ptr(t["sgu_q"]), D.ptr(t["sgu_s"]), D.ptr(t["sd_q"]), D.ptr(t["sd_s"]), D.ptr(dhn), rows,
                       D.ptr(sact), D.ptr(sh), H, I, sp)
    act = torch.zeros(rows * topk * I, dtype=torch.int16, device="cuda")
    yp = torch.zeros(rows * topk * H, device="cuda")
    if path == "rows":
        pname = "dr_moe_prefill_rows_bf16s" if fmt == "cfg" else "dr_moe_prefill_rows"
        getattr(L, pname)(D.ptr(t["gu_q"]), D.ptr(t["gu_s"]), D.ptr(t["d_q"]), D.ptr(t["d_s"]), D.ptr(dhn), rows,
                          D.ptr(row_of_slot), D.ptr(offsets), D.ptr(counts), D.ptr(act), D.ptr(yp), E, H, I, sp)
    else:
        L.dr_moe_group(D.ptr(idx), rows * topk, E, D.ptr(counts), D.ptr(offsets), D.ptr(slot_of), sp)
        xp = torch.zeros(rows * topk * H, dtype=torch.int16, device="cuda")
        L.dr_moe_gather_rows(D.ptr(slot_of), rows, topk, D.ptr(dhn), D.ptr(xp), H, sp)
        pname = "dr_moe_prefill_bf16s" if fmt == "cfg" else "dr_moe_prefill"
        getattr(L, pname)(D.ptr(t["gu_q"]), D.ptr(t["gu_s"]), D.ptr(t["d_q"]), D.ptr(t["d_s"]), D.ptr(xp),
                          D.ptr(offsets), D.ptr(counts), D.ptr(act), D.ptr(yp), E, H, I, sp)
    L.dr_moe_combine(D.ptr(dx), D.ptr(yp), D.ptr(slot_of), D.ptr(wts), D.ptr(sg), D.ptr(sh), rows, topk, H, sp)
    torch.cuda.synchronize()
    # routing: bit-exact against the oracle's canonical GEMM + softmax/top-k
    rl = O.router_logits_rows(hn, Lh["router"], rows, E + 1, H)
    ri, rw, rs = O.moe_topk(rl, rows, E, topk, E + 1)
    np.testing.assert_array_equal(host(logits).reshape(rows, E + 1).view(np.uint32), rl.view(np.uint32))
    np.testing.assert_array_equal(host(idx), ri)
    np.testing.assert_array_equal(host(wts).view(np.uint32), rw.view(np.uint32))
    rc, ro, rso = O.moe_group(ri, E)
    np.testing.assert_array_equal(host(counts), rc)
    np.testing.assert_array_equal(host(slot_of), rso)
    if path == "rows":
        np.testing.assert_array_equal(host(offsets), ro)
        np.testing.assert_array_equal(host(row_of_slot)[rso], np.arange(rows * topk) // topk)
        assert int(host(counter)[0]) == 0, "counter not reset"
    ref = O.moe_prefill_layer(Lh, hn, rows, ri, rw, rs, x0, H, I, topk).astype(np.float64)
    # intermediates of the oracle, to bound the effect of bf16 act rounding flips
    n = rows * topk
    xpr = np.empty((n, H), np.uint16)
    xpr[rso] = hn[np.arange(n) // topk]
    ract, _ = O.moe_prefill_experts(Lh, xpr, ro, rc, E, H, I)
    rsact, _ = O.shared_prefill(Lh, hn, rows, H, I)
    af, rf = check_act(host(act).view(np.uint16).reshape(n, I), ract, "routed act")
    saf, srf = check_act(host(sact).view(np.uint16).reshape(rows, I), rsact, "shared act")
    extra_slot = np.zeros((n, H))
    for e in np.nonzero(rc)[0]:
        sl = slice(ro[e], ro[e] + rc[e])
        d = np.abs(af[sl] - rf[sl])
        if d.any():
            extra_slot[sl] = d @ np.abs(expert_dense(Lh, "d", e).astype(np.float64)).T
    sd = O.dequant_q8(Lh["sd_q"], Lh["sd_s"], Lh["sh_kind"], Lh["sh_group_d"], H, I).astype(np.float64)
    sig = 1 / (1 + np.exp(-rs.astype(np.float64)))
    extra = sig[:, None] * (np.abs(saf - srf) @ np.abs(sd).T)
    extra += np.einsum("rk,rkc->rc", rw.reshape(rows, topk).astype(np.float64), extra_slot[rso.reshape(rows, topk)])
    got = host(dx).reshape(rows, H).astype(np.float64)
    bad = np.abs(got - ref) > 1e-3 + 1e-3 * np.abs(ref) + extra
    print(f"act flips routed {int((af != rf).sum())}, shared {int((saf != srf).sum())}; "
          f"max |err| {np.abs(got - ref).max():.2e}")
    assert not bad.any(), f"prefill layer output: {int(bad.sum())} outside tolerance + flip propagation"


def test_reference_elementwise_entry_points():
    """dr_dequant_q8 and dr_f32_to_bf16 bit for bit (one fp32 product / one RNE rounding,
    kernels/drama.cu:1114-1164), dr_swiglu_rows within one bf16 rounding flip."""
    import torch

    rng = np.random.default_rng(90)
    L, sp = D.lib(), D.stream_ptr()
    q = rng.integers(-127, 128, (96, 512), dtype=np.int8)
    s = synth.f32_to_f16((np.abs(rng.normal(0, 0.02, (96, 4))) + 1e-4).astype(np.float32))
    out = torch.zeros(96 * 512, dtype=torch.int16, device="cuda")
    dq, ds = dev(q), dev(s)  # kept alive until the kernels have run
    L.dr_dequant_q8(D.ptr(dq), D.ptr(ds), D.ptr(out), 96, 512, sp)
    x = rng.normal(0, 3, 5000).astype(np.float32)
    x[:6] = [np.inf, -np.inf, np.nan, 0.0, -0.0, 3.4e38]
    xb = torch.zeros(5000, dtype=torch.int16, device="cuda")
    dxx = dev(x)
    L.dr_f32_to_bf16(D.ptr(dxx), D.ptr(xb), 5000, sp)
    rows, ii = 7, 512
    hh = rng.normal(0, 2, (rows, 2 * ii)).astype(np.float32)
    y = torch.zeros(rows * ii, dtype=torch.int16, device="cuda")
    dhh = dev(hh)
    L.dr_swiglu_rows(D.ptr(dhh), D.ptr(y), rows, ii, sp)
    torch.cuda.synchronize()
    sf = O.f16_to_f32(s)
    want = synth.f32_to_bf16(q.astype(np.float32) * np.repeat(sf, 128, axis=1))
    np.testing.assert_array_equal(host(out).view(np.uint16).reshape(96, 512), want)
    got = host(xb).view(np.uint16)
    np.testing.assert_array_equal(got[3:], synth.f32_to_bf16(x[3:]))
    assert got[0] == 0x7F80 and got[1] == 0xFF80 and (got[2] & 0x7F80) == 0x7F80 and (got[2] & 0x7F)
    g, u = hh[:, :ii].astype(np.float64), hh[:, ii:].astype(np.float64)
    ref = g / (1 + np.exp(-g)) * u
    check_act(host(y).view(np.uint16).reshape(rows, ii), synth.f32_to_bf16(ref.astype(np.float32)), "swiglu rows")


def test_reference_shared_expert_sequence_300_rows():
    """The unchanged engine's shared-expert prefill (src/engine.rs:351-355,560-562):
    dr_dequant_q8 -> dr_gemm (300 x 1024 x 2048) -> dr_swiglu_rows -> dr_dequant_q8 -> dr_gemm
    (300 x 2048 x 512).  Each GEMM equals the oracle's canonical-order GEMM bit for bit on the
    GPU's own operands; the output is within the tolerance (plus act rounding flips) of the
    float64 computation on the bf16-dequantised weights the reference multiplies."""
    import torch

    rows = 300
    Lh = synth.make_layer(95, E=8, fmt="ref")
    rng = np.random.default_rng(96)
    hn = synth.f32_to_bf16(rng.normal(0, 1, (rows, H)).astype(np.float32))
    L, sp, P = D.lib(), D.stream_ptr(), D.ptr
    h = np.zeros(1, np.uint64)
    L.dr_cublas_create(h.ctypes.data, sp)
    wbuf = torch.zeros(2 * I * H, dtype=torch.int16, device="cuda")
    shh = torch.zeros(rows * 2 * I, device="cuda")
    act = torch.zeros(rows * I, dtype=torch.int16, device="cuda")
    out = torch.zeros(rows * H, device="cuda")
    dhn = dev(hn)
    w = {k: dev(Lh[k]) for k in ("sgu_q", "sgu_s", "sd_q", "sd_s")}
    L.dr_dequant_q8(P(w["sgu_q"]), P(w["sgu_s"]), P(wbuf), 2 * I, H, sp)
    torch.cuda.synchronize()
    wgu = host(wbuf).view(np.uint16).reshape(2 * I, H).copy()
    L.dr_gemm(int(h[0]), P(dhn), P(wbuf), P(shh), rows, 2 * I, H, 0.0)
    L.dr_swiglu_rows(P(shh), P(act), rows, I, sp)
    torch.cuda.synchronize()
    g_shh = host(shh).reshape(rows, 2 * I)
    g_act = host(act).view(np.uint16).reshape(rows, I)
    L.dr_dequant_q8(P(w["sd_q"]), P(w["sd_s"]), P(wbuf), H, I, sp)
    torch.cuda.synchronize()
    wd = host(wbuf).view(np.uint16)[:H * I].reshape(H, I).copy()
    L.dr_gemm(int(h[0]), P(act), P(wbuf), P(out), rows, H, I, 0.0)
    torch.cuda.synchronize()
    g_out = host(out).reshape(rows, H)
    # each GEMM: canonical order, bit for bit
    np.testing.assert_array_equal(g_shh.view(np.uint32), O.router_logits_rows(hn, wgu, rows, 2 * I, H).view(np.uint32))
    np.testing.assert_array_equal(g_out.view(np.uint32), O.router_logits_rows(g_act, wd, rows, H, I).view(np.uint32))
    # end to end against float64 on the reference's bf16 weights
    wguf = synth.bf16_to_f32(wgu).astype(np.float64)
    wdf = synth.bf16_to_f32(wd).astype(np.float64)
    hh = synth.bf16_to_f32(hn).astype(np.float64) @ wguf.T
    ref_act = hh[:, :I] / (1 + np.exp(-hh[:, :I])) * hh[:, I:]
    af, rf = check_act(g_act, synth.f32_to_bf16(ref_act.astype(np.float32)), "shared act (reference sequence)")
    assert_close_with_flips(g_out, rf @ wdf.T, wdf, af, rf, "shared out (reference sequence)")


@pytest.mark.parametrize("rows,E,skew", [(300, 256, False), (300, 256, True), (1024, 256, True), (4, 256, False),
                                         (1, 8, False), (37, 64, True)])
def test_group_rows_matches_oracle(rows, E, skew):
    """dr_moe_group_rows (grouping of a routing given from outside, as bench.py's skewed
    configuration 4 uses): counts, offsets and slot_of equal to the oracle's stable grouping of
    the rows * 8 pairs, row_of_slot the inverse map; skewed: 10% of the experts take about half
    of the pairs (the reference's semantics: kernels/drama.cu:744-778, src/engine.rs:564-575)."""
    topk = 8
    rng = np.random.default_rng(rows + E + 17 * skew)
    idx = np.empty((rows, topk), np.int32)
    hot = rng.choice(E, max(1, E // 10), replace=False)
    for r in range(rows):  # distinct experts per row, as a router produces
        nh = int(rng.binomial(topk, 0.5)) if skew else 0
        nh = min(nh, hot.size)
        hsel = rng.choice(hot, nh, replace=False)
        rest = rng.choice(np.setdiff1d(np.arange(E), hsel), topk - nh, replace=False)
        idx[r] = rng.permutation(np.concatenate([hsel, rest]))
    idx = idx.ravel()
    n = rows * topk
    rc, ro, rso = O.moe_group(idx, E)
    if skew and E == 256:
        assert rc[hot].sum() >= 0.4 * n, "routing is not skewed as intended"
    counts, offsets, slot_of, row_of_slot = t_i32(E), t_i32(E), t_i32(n), t_i32(n + 16)
    for rep in range(2):  # outputs are fully rewritten by every call
        counts.fill_(-7)
        slot_of.fill_(-7)
        D.lib().dr_moe_group_rows(D.ptr(dev(idx)), rows, topk, E, D.ptr(counts), D.ptr(offsets), D.ptr(slot_of),
                                  D.ptr(row_of_slot), D.stream_ptr())
        np.testing.assert_array_equal(host(counts), rc)
        np.testing.assert_array_equal(host(offsets), ro)
        np.testing.assert_array_equal(host(slot_of), rso)
        np.testing.assert_array_equal(host(row_of_slot)[rso], np.arange(n) // topk)


def _pack_ref(q, sm, n, k):
    """Host restatement of the tile-step layout of dr_moe_pack_q4 (include/drama_moe.h)."""
    e = q.shape[0]
    spt = k // 256
    qv = q.reshape(e, n // 16, 16, spt, 2, 4, 16)      # [e][tile][row][step][p][g][b]
    qo = qv.transpose(0, 1, 3, 4, 5, 2, 6)              # [e][tile][step][p][g][row][b]: lane l = 16 g + row
    sv = sm.reshape(e, n // 16, 16, spt, 4, 2)          # [e][tile][row][step][word][half]
    so = sv.transpose(0, 1, 3, 2, 4, 5)                 # [e][tile][step][row][word][half]
    return np.ascontiguousarray(qo).reshape(e, n * k // 2), np.ascontiguousarray(so).reshape(e, n * k // 32)


@pytest.mark.parametrize("e,n,k", [(3, 1024, 2048), (2, 2048, 512), (1, 16, 256)])
def test_pack_q4_layout(e, n, k):
    """dr_moe_pack_q4 against a numpy restatement of the layout, byte for byte."""
    import torch

    rng = np.random.default_rng(n + k + e)
    q = rng.integers(0, 256, (e, n, k // 2), dtype=np.uint8)
    sm = rng.integers(0, 65536, (e, n, k // 64, 2), dtype=np.uint16)
    dq, ds = dev(q), dev(sm)
    qo = torch.zeros(q.size, dtype=torch.uint8, device="cuda")
    so = torch.zeros(sm.size, dtype=torch.int16, device="cuda")
    D.lib().dr_moe_pack_q4(D.ptr(dq), D.ptr(ds), e, n, k, D.ptr(qo), D.ptr(so), D.stream_ptr())
    torch.cuda.synchronize()
    rq, rs = _pack_ref(q, sm, n, k)
    np.testing.assert_array_equal(host(qo).reshape(e, -1), rq)
    np.testing.assert_array_equal(host(so).view(np.uint16).reshape(e, -1), rs)
    assert D.lib().raw("dr_moe_pack_q4")(D.ptr(dq), D.ptr(ds), e, 24, k, D.ptr(qo), D.ptr(so), None) == -1


@pytest.mark.parametrize("fmt,skew,E,rows", [("cfg", False, 24, 96), ("ref", False, 24, 96), ("cfg", True, 24, 96),
                                             ("cfg", False, 256, 300), ("cfg", True, 256, 300), ("cfg", False, 256, 1)])
def test_prefill_rows_packed_matches(fmt, skew, E, rows):
    """dr_moe_prefill_rows_packed*: weights packed by dr_moe_pack_q4 give the act and y bits of
    dr_moe_prefill_rows* on the reference layout."""
    import torch

    topk = 8
    Lh = synth.make_layer(40, E=E, fmt=fmt, kind="q4")
    idx, counts, offsets, slot_of, x, xp = grouped_inputs(45 + rows, E, rows, topk, skew)
    n = rows * topk
    ros = np.zeros(n + 16, np.int32)
    ros[slot_of] = np.arange(n) // topk
    t = {k: dev(Lh[k]) for k in ("gu_q", "gu_s", "d_q", "d_s")}
    pk = {k: torch.zeros_like(v) for k, v in t.items()}
    lib = D.lib()
    lib.dr_moe_pack_q4(D.ptr(t["gu_q"]), D.ptr(t["gu_s"]), E, 2 * I, H, D.ptr(pk["gu_q"]), D.ptr(pk["gu_s"]),
                       D.stream_ptr())
    lib.dr_moe_pack_q4(D.ptr(t["d_q"]), D.ptr(t["d_s"]), E, H, I, D.ptr(pk["d_q"]), D.ptr(pk["d_s"]), D.stream_ptr())
    dx, dros, doff, dcnt = dev(x), dev(ros), dev(offsets), dev(counts)
    outs = []
    for packed, w in ((False, t), (True, pk)):
        act = torch.zeros(n * I, dtype=torch.int16, device="cuda")
        yp = torch.zeros(n * H, dtype=torch.float32, device="cuda")
        name = "dr_moe_prefill_rows" + ("_packed" if packed else "") + ("_bf16s" if fmt == "cfg" else "")
        getattr(lib, name)(D.ptr(w["gu_q"]), D.ptr(w["gu_s"]), D.ptr(w["d_q"]), D.ptr(w["d_s"]), D.ptr(dx), rows,
                           D.ptr(dros), D.ptr(doff), D.ptr(dcnt), D.ptr(act), D.ptr(yp), E, H, I, D.stream_ptr())
        torch.cuda.synchronize()
        outs.append((host(act), host(yp)))
    np.testing.assert_array_equal(outs[1][0], outs[0][0])
    np.testing.assert_array_equal(outs[1][1].view(np.uint32), outs[0][1].view(np.uint32))


def _pack_fp8_ref(q, n, k):
    """Host restatement of the tile-step layout of dr_moe_pack_fp8 (include/drama_moe.h)."""
    e = q.shape[0]
    qv = q.reshape(e, n // 16, 16, k // 256, 4, 4, 16)   # [e][tile][row][step][p][g][b]
    return np.ascontiguousarray(qv.transpose(0, 1, 3, 4, 5, 2, 6)).reshape(e, n * k)


@pytest.mark.parametrize("e,n,k", [(2, 1024, 2048), (1, 16, 256)])
def test_pack_fp8_layout(e, n, k):
    """dr_moe_pack_fp8 against a numpy restatement of the layout, byte for byte."""
    import torch

    q = np.random.default_rng(n + k).integers(0, 256, (e, n, k), dtype=np.uint8)
    dq = dev(q)
    qo = torch.zeros(q.size, dtype=torch.uint8, device="cuda")
    assert D.lib().raw("dr_moe_pack_fp8")(D.ptr(dq), e, n, k, D.ptr(qo), D.stream_ptr()) == 0
    torch.cuda.synchronize()
    np.testing.assert_array_equal(host(qo).reshape(e, -1), _pack_fp8_ref(q, n, k))
    assert D.lib().raw("dr_moe_pack_fp8")(D.ptr(dq), e, n, 200, D.ptr(qo), None) == -1


@pytest.mark.parametrize("fmt,skew,E,rows", [("cfg", False, 24, 96), ("ref", False, 24, 96), ("cfg", True, 256, 300),
                                             ("cfg", False, 256, 1)])
def test_prefill_rows_packed_fp8_matches(fmt, skew, E, rows):
    """dr_moe_prefill_rows_packed_fp8*: weights packed by dr_moe_pack_fp8 give the act and y bits
    of dr_moe_prefill_rows_fp8* on the reference layout."""
    import torch

    topk = 8
    Lh = synth.make_layer(41, E=E, fmt=fmt, kind="fp8")
    idx, counts, offsets, slot_of, x, xp = grouped_inputs(46 + rows, E, rows, topk, skew)
    n = rows * topk
    ros = np.zeros(n + 16, np.int32)
    ros[slot_of] = np.arange(n) // topk
    t = {k: dev(Lh[k]) for k in ("gu_q", "gu_s", "d_q", "d_s")}
    pk = dict(t)
    lib = D.lib()
    for q, nn, kk in (("gu_q", 2 * I, H), ("d_q", H, I)):
        pk[q] = torch.zeros_like(t[q])
        assert lib.raw("dr_moe_pack_fp8")(D.ptr(t[q]), E, nn, kk, D.ptr(pk[q]), D.stream_ptr()) == 0
    dx, dros, doff, dcnt = dev(x), dev(ros), dev(offsets), dev(counts)
    outs = []
    for packed, w in ((False, t), (True, pk)):
        act = torch.zeros(n * I, dtype=torch.int16, device="cuda")
        yp = torch.zeros(n * H, dtype=torch.float32, device="cuda")
        name = "dr_moe_prefill_rows" + ("_packed" if packed else "") + "_fp8" + ("_bf16s" if fmt == "cfg" else "")
        rc = lib.raw(name)(D.ptr(w["gu_q"]), D.ptr(w["gu_s"]), D.ptr(w["d_q"]), D.ptr(w["d_s"]), D.ptr(dx), rows,
                           D.ptr(dros), D.ptr(doff), D.ptr(dcnt), D.ptr(act), D.ptr(yp), E, H, I, D.stream_ptr())
        assert rc == 0, f"{name} returned {rc}"
        torch.cuda.synchronize()
        outs.append((host(act), host(yp)))
    np.testing.assert_array_equal(outs[1][0], outs[0][0])
    np.testing.assert_array_equal(outs[1][1].view(np.uint32), outs[0][1].view(np.uint32))
