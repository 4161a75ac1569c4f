"""GPU parity of the small-batch decode path (dr_router_topk_rows, dr_moe_decode_rows*): a few
tokens decoded together through the batch-1 chain's kernels, each row checked against the
oracle on that row alone.  Routing (logits, picks, weights, shared gate) bit for bit with the
oracle's canonical router; outputs within |gpu - ref| <= 1e-3 + 1e-3 |ref|."""
import numpy as np
import pytest

import dramamoe as D
import oracle as O
import synth
from helpers import assert_close, bits, dev, host

pytestmark = pytest.mark.gpu
H, I, TOPK = 2048, 512, 8


@pytest.mark.parametrize("rows,E,norm", [(1, 256, True), (4, 256, True), (8, 64, True), (3, 16, False)])
def test_router_rows_bit_exact_per_row(rows, E, norm):
    import torch

    L = synth.make_layer(200 + rows, E=E, fmt="cfg", with_norm=norm, quick=True)
    rng = np.random.default_rng(rows + E)
    x = rng.normal(0, 1 if norm else 0.05, (rows, H)).astype(np.float32)
    dw, dx = dev(L["router"]), dev(x)
    dnw = dev(L["nw"]) if norm else None
    logits = torch.zeros(rows * (E + 1), device="cuda")
    idx = torch.full((rows * TOPK,), -1, dtype=torch.int32, device="cuda")
    wts = torch.zeros(rows * TOPK, device="cuda")
    sg = torch.zeros(rows, device="cuda")
    counter = torch.zeros(4, dtype=torch.int32, device="cuda")
    for rep in range(2):  # the counter is back at zero after a call
        D.lib().dr_router_topk_rows(D.ptr(dw), D.ptr(dx), D.ptr(dnw), 1e-6, D.ptr(logits), E, TOPK, H, rows,
                                    D.ptr(idx), D.ptr(wts), D.ptr(sg), D.ptr(counter), D.stream_ptr())
        torch.cuda.synchronize()
        assert int(host(counter)[0]) == 0
        gl = host(logits).reshape(rows, E + 1)
        for r in range(rows):
            rl, ri, rw, rs = O.router_topk(L["router"], x[r], L["nw"] if norm else None, 1e-6, E, TOPK)
            np.testing.assert_array_equal(bits(gl[r]), bits(rl), err_msg=f"row {r} logits")
            np.testing.assert_array_equal(host(idx)[r * TOPK:(r + 1) * TOPK], ri, err_msg=f"row {r} experts")
            np.testing.assert_array_equal(bits(host(wts)[r * TOPK:(r + 1) * TOPK]), bits(rw), err_msg=f"row {r} weights")
            assert bits(host(sg)[r:r + 1])[0] == bits(np.float32(rs))


def _routing(rng, rows, E):
    """Distinct experts per row, with rows sharing some experts (as real routing does)."""
    common = rng.choice(E, 4, replace=False)
    idx = np.empty((rows, TOPK), np.int32)
    for r in range(rows):
        own = rng.choice(np.setdiff1d(np.arange(E), common), TOPK - 2, replace=False)
        idx[r] = rng.permutation(np.concatenate([rng.choice(common, 2, replace=False), own]))
    w = rng.random((rows, TOPK)).astype(np.float32) + 0.1
    return idx, (w / w.sum(1, keepdims=True)).astype(np.float32), rng.normal(0, 1, rows).astype(np.float32)


@pytest.mark.parametrize("kind,fmt,rows", [("q4", "cfg", 4), ("q4", "ref", 3), ("q4", "cfg", 6), ("q4", "cfg", 1),
                                           ("fp8", "cfg", 4), ("fp8", "ref", 2), ("fp8", "cfg", 5)])
def test_decode_rows_matches_oracle_per_row(kind, fmt, rows):
    import torch

    E = 32
    print(f"decode rows kind={kind} fmt={fmt} rows={rows}", flush=True)
    L = synth.make_layer(210 + rows, E=E, fmt=fmt, kind=kind, quick=True)
    rng = np.random.default_rng(211 + rows)
    x = rng.normal(0, 1, (rows, H)).astype(np.float32)
    res = rng.normal(0, 1, (rows, H)).astype(np.float32)
    idx, wts, sg = _routing(rng, rows, E)
    t = {k: dev(L[k]) for k in ("gu_q", "gu_s", "d_q", "d_s", "sgu_q", "sgu_s", "sd_q", "sd_s", "nw")}
    dx, dres, didx, dwts, dsg = dev(x), dev(res), dev(idx), dev(wts), dev(sg)
    act = torch.zeros(rows * (TOPK + 1) * I, device="cuda")
    y = torch.zeros(rows * H, device="cuda")
    P = D.ptr
    args = [P(t["gu_q"]), P(t["gu_s"]), P(t["d_q"]), P(t["d_s"]), P(t["sgu_q"]), P(t["sgu_s"]), P(t["sd_q"]),
            P(t["sd_s"]), P(dx), P(didx), P(dwts), P(dsg), P(dres), P(act), P(y)]
    name = "dr_moe_decode_rows" + ("_fp8" if kind == "fp8" else "") + ("_bf16s" if fmt == "cfg" else "")
    if fmt == "cfg":
        args.append(None)  # yb
    getattr(D.lib(), name)(*args, rows, H, I, TOPK, P(t["nw"]), 1e-6, D.stream_ptr())
    torch.cuda.synchronize()
    gy = host(y).reshape(rows, H)
    for r in range(rows):
        _, ry = O.moe_decode(L, x[r], idx[r], wts[r], sg[r], res[r], H, I, TOPK, nw=L["nw"], eps=1e-6)
        assert_close(gy[r], ry, what=f"row {r}")


def test_decode_rows_alias_and_shape_gates():
    """x == res == y (the engine's aliasing) gives the same bits as separate buffers; bad
    shapes return -1 before any launch."""
    import torch

    E, rows = 16, 4
    L = synth.make_layer(230, E=E, fmt="cfg", quick=True)
    rng = np.random.default_rng(231)
    x = rng.normal(0, 1, (rows, H)).astype(np.float32)
    idx, wts, sg = _routing(rng, rows, E)
    t = {k: dev(L[k]) for k in ("gu_q", "gu_s", "d_q", "d_s", "sgu_q", "sgu_s", "sd_q", "sd_s", "nw")}
    didx, dwts, dsg = dev(idx), dev(wts), dev(sg)
    act = torch.zeros(rows * (TOPK + 1) * I, device="cuda")
    P = D.ptr
    f = D.lib().raw("dr_moe_decode_rows_bf16s")
    w8 = [P(t[k]) for k in ("gu_q", "gu_s", "d_q", "d_s", "sgu_q", "sgu_s", "sd_q", "sd_s")]
    xa, xb, ya = dev(x), dev(x), torch.zeros(rows * H, device="cuda")
    assert f(*w8, P(xa), P(didx), P(dwts), P(dsg), P(xa), P(act), P(ya), None, rows, H, I, TOPK, P(t["nw"]), 1e-6,
             D.stream_ptr()) == 0
    assert f(*w8, P(xb), P(didx), P(dwts), P(dsg), P(xb), P(act), P(xb), None, rows, H, I, TOPK, P(t["nw"]), 1e-6,
             D.stream_ptr()) == 0
    torch.cuda.synchronize()
    np.testing.assert_array_equal(bits(host(xb).ravel()), bits(host(ya).ravel()))
    for pos, bad in ((16, 0), (16, 65), (17, 1024), (18, 256), (19, 4)):
        a = [*w8, P(xa), P(didx), P(dwts), P(dsg), P(xa), P(act), P(ya), None, rows, H, I, TOPK, P(t["nw"]), 1e-6,
             D.stream_ptr()]
        a[pos] = bad
        assert f(*a) == -1
    g = D.lib().raw("dr_router_topk_rows")
    assert g(None, None, None, 1e-6, None, 256, 8, 2048, 9, None, None, None, None, D.stream_ptr()) == -1
    assert g(None, None, None, 1e-6, None, 257, 8, 2048, 4, None, None, None, None, D.stream_ptr()) == -1


@pytest.mark.parametrize("fmt", ["cfg", "ref"])
def test_cfg5_fp8_batch4_rows_path_full_size(fmt):
    """Configuration 5 batch 4 through the small-batch path at E = 256: router rows, then the
    decode rows kernels, checked per row against the oracle (the routed experts handed to the
    oracle are gathered to the host, as in tests/test_gpu_configs.py)."""
    import torch

    from test_gpu_configs import compact, fp8_layer_gpu, host_layer

    E, rows = 256, 4
    Ld = fp8_layer_gpu(61 if fmt == "cfg" else 62, fmt)
    rng = np.random.default_rng(63)
    x = rng.normal(0, 1, (rows, H)).astype(np.float32)
    dx = dev(x)
    logits = torch.zeros(rows * (E + 1), device="cuda")
    idx = torch.zeros(rows * TOPK, dtype=torch.int32, device="cuda")
    wts = torch.zeros(rows * TOPK, device="cuda")
    sg = torch.zeros(rows, device="cuda")
    counter = torch.zeros(4, dtype=torch.int32, device="cuda")
    act = torch.zeros(rows * (TOPK + 1) * I, device="cuda")
    L, P, sp = D.lib(), D.ptr, D.stream_ptr()
    L.dr_router_topk_rows(P(Ld["router"]), P(dx), P(Ld["nw"]), 1e-6, P(logits), E, TOPK, H, rows, P(idx), P(wts),
                          P(sg), P(counter), sp)
    args = [P(Ld[k]) for k in ("gu_q", "gu_s", "d_q", "d_s", "sgu_q", "sgu_s", "sd_q", "sd_s")]
    args += [P(dx), P(idx), P(wts), P(sg), P(dx), P(act), P(dx)]
    if fmt == "cfg":
        L.dr_moe_decode_rows_fp8_bf16s(*args, None, rows, H, I, TOPK, P(Ld["nw"]), 1e-6, sp)
    else:
        L.dr_moe_decode_rows_fp8(*args, rows, H, I, TOPK, P(Ld["nw"]), 1e-6, sp)
    torch.cuda.synchronize()
    gi, gw, gs, gy = host(idx).reshape(rows, TOPK), host(wts).reshape(rows, TOPK), host(sg), host(dx).reshape(rows, H)
    router = Ld["router"].cpu().numpy().view(np.uint16)
    nw = Ld["nw"].cpu().numpy()
    for r in range(rows):
        _, ri, rw, rs = O.router_topk(router, x[r], nw, 1e-6, E, TOPK)
        np.testing.assert_array_equal(gi[r], ri)
        np.testing.assert_array_equal(bits(gw[r]), bits(rw))
        used, ric = compact(ri)
        hl = host_layer(Ld, "fp8", fmt, used)
        _, ry = O.moe_decode(hl, x[r], ric, rw, rs, x[r], H, I, TOPK, nw=nw, eps=1e-6)
        assert_close(gy[r], ry, what=f"batch-4 row {r}")
    del Ld
    torch.cuda.empty_cache()


def _check_rows_vs_oracle(Ld, fmt, E, x, out):
    """Routed launch outputs of one call against the oracle, row by row: logits, picks, weights
    and shared gate bit for bit with O.router_topk on that row, y (x + layer, res aliasing x)
    within 1e-3 + 1e-3 |ref| of O.moe_decode over the experts the row picked."""
    from test_gpu_configs import compact, host_layer

    lg, idx, wts, sg, _, y, _ = out
    rows = x.shape[0]
    router = Ld["router"].cpu().numpy().view(np.uint16)
    nw = Ld["nw"].cpu().numpy()
    gl, gi, gw, gy = lg.reshape(rows, E + 1), idx.reshape(rows, TOPK), wts.reshape(rows, TOPK), y.reshape(rows, H)
    for r in range(rows):
        rl, ri, rw, rs = O.router_topk(router, x[r], nw, 1e-6, E, TOPK)
        np.testing.assert_array_equal(bits(gl[r]), bits(rl), err_msg=f"row {r} logits")
        np.testing.assert_array_equal(gi[r], ri, err_msg=f"row {r} experts")
        np.testing.assert_array_equal(bits(gw[r]), bits(rw), err_msg=f"row {r} weights")
        assert bits(sg[r:r + 1])[0] == bits(np.float32(rs)), f"row {r} shared gate"
        used, ric = compact(ri)
        hl = host_layer(Ld, "fp8", fmt, used)
        _, ry = O.moe_decode(hl, x[r], ric, rw, rs, x[r], H, I, TOPK, nw=nw, eps=1e-6)
        assert_close(gy[r], ry, what=f"routed launch row {r}")


@pytest.mark.parametrize("fmt,rows,E", [("cfg", 4, 256), ("ref", 4, 256), ("cfg", 5, 256), ("cfg", 1, 256),
                                         ("cfg", 3, 256), ("cfg", 4, 64), ("cfg", 2, 9)])
def test_routed_fp8_rows_equal_three_launch_path(fmt, rows, E):
    """dr_moe_decode_rows_routed_fp8(_bf16s) (router + top-k in the gate_up launch, then down)
    against
    dr_router_topk_rows + dr_moe_decode_rows_fp8(_bf16s) on the same inputs: logits, picks,
    weights, shared gates, activations and outputs bit for bit (both run the same arithmetic),
    over three calls in a row with different x on one counter and tag buffer (each launch tags
    its picks afresh), the last with y aliasing x and res.  The routed launch's first and last
    calls are also checked against the oracle row by row (routing bit-exact, y in tolerance)."""
    import torch

    from test_gpu_configs import fp8_layer_gpu

    # E < 256: the same weights, the router over the first E experts (rows 0 .. E of its matrix)
    Ld = fp8_layer_gpu(71 if fmt == "cfg" else 72, fmt)
    L, P, sp = D.lib(), D.ptr, D.stream_ptr()
    wargs = [P(Ld[k]) for k in ("gu_q", "gu_s", "d_q", "d_s", "sgu_q", "sgu_s", "sd_q", "sd_s")]
    z = lambda n, dt=torch.float32: torch.zeros(n, dtype=dt, device="cuda")
    counter, tags = z(4, torch.int32), z(896, torch.int64)
    c3 = z(4, torch.int32)
    rng = np.random.default_rng(70 + rows)
    for call in range(3):
        x = rng.normal(0, 1, (rows, H)).astype(np.float32)
        outs = []
        for fused in (False, True):
            dx = dev(x)
            lg, idx, wts, sg = z(rows * (E + 1)), z(rows * TOPK, torch.int32), z(rows * TOPK), z(rows)
            act = z(rows * (TOPK + 1) * I)
            y = dx if call == 2 else z(rows * H)
            yb = z(rows * H, torch.int16)
            if fused:
                if fmt == "cfg":
                    rc = L.dr_moe_decode_rows_routed_fp8_bf16s(P(Ld["router"]), P(Ld["nw"]), 1e-6, E, *wargs, P(dx),
                                                               P(lg), P(idx), P(wts), P(sg), P(counter), P(tags), P(dx),
                                                               P(act), P(y), P(yb), rows, H, I, TOPK, sp)
                else:
                    rc = L.dr_moe_decode_rows_routed_fp8(P(Ld["router"]), P(Ld["nw"]), 1e-6, E, *wargs, P(dx), P(lg),
                                                         P(idx), P(wts), P(sg), P(counter), P(tags), P(dx), P(act),
                                                         P(y), rows, H, I, TOPK, sp)
                assert rc == 0
            else:
                assert L.dr_router_topk_rows(P(Ld["router"]), P(dx), P(Ld["nw"]), 1e-6, P(lg), E, TOPK, H, rows,
                                             P(idx), P(wts), P(sg), P(c3), sp) == 0
                args = [*wargs, P(dx), P(idx), P(wts), P(sg), P(dx), P(act), P(y)]
                if fmt == "cfg":
                    rc = L.dr_moe_decode_rows_fp8_bf16s(*args, P(yb), rows, H, I, TOPK, P(Ld["nw"]), 1e-6, sp)
                else:
                    rc = L.dr_moe_decode_rows_fp8(*args, rows, H, I, TOPK, P(Ld["nw"]), 1e-6, sp)
                assert rc == 0
            torch.cuda.synchronize()
            assert L.dr_last_error() == 0
            outs.append([host(t) for t in (lg, idx, wts, sg, act, y, yb)])
            if fused and call != 1:
                _check_rows_vs_oracle(Ld, fmt, E, x, outs[-1])
        for name, a, b in zip(("logits", "idx", "wts", "sgate", "act", "y", "yb"), *outs):
            np.testing.assert_array_equal(bits(a) if a.dtype == np.float32 else a,
                                          bits(b) if b.dtype == np.float32 else b, err_msg=f"call {call}: {name}")
        assert int(host(counter)[0]) == 0 and int(host(counter)[2]) == 0
    # one tag per chunk of four rows
    assert int(host(counter)[1]) == 3 * ((rows + 3) // 4)
    assert not host(tags)[640:].any()  # the launch's block counters are back at zero
    del Ld
    torch.cuda.empty_cache()

