"""GPU parity at the benchmark configurations' full sizes, through the C ABI.

- configuration 3: the 40-layer, 256-expert int4 decode step (dr_moe_decode_step_bf16s) with
  ~17 GiB of weights resident: routing of every layer bit-exact against the oracle's router on
  the step's own layer input, layer outputs within 1e-3 + 1e-3 |ref| on layers 0, 19 and 39,
  and graph replays equal to the eager call bit for bit;
- configuration 5, batch 4: four decode rows through the reference engine's grouped path
  (router GEMM, top-k, shared expert, grouping, gather, FP8 grouped GEMM, combine) with 256
  block-FP8 experts, in both scale formats;
- configuration 4, skewed: 300 rows where 10% of the 256 experts receive half of the 2400
  pairs, through grouping, gather, the int4 grouped GEMM and the combine.

Weights are generated on the device (torch RNG).  The oracle is handed only the experts a
check routes to (gathered to the host, indices renumbered): an expert's result does not
depend on where it is stored, which tests/test_oracle_moe.py pins for the oracle."""
import ctypes

import numpy as np
import pytest

import dramamoe as D
import oracle as O
import synth
from helpers import assert_close, bits, dev, host
from test_gpu_prefill import check_act, expert_dense, t_i32

pytestmark = pytest.mark.gpu
H, I, E, TOPK = 2048, 512, 256, 8
KEYS = ("router", "nw", "gu_q", "gu_s", "d_q", "d_s", "sgu_q", "sgu_s", "sd_q", "sd_s")


def _bf16(t):
    import torch

    return t.to(torch.bfloat16).view(torch.int16)


def _f16(t):
    import torch

    return t.to(torch.float16).view(torch.int16)


def fp8_layer_gpu(seed, fmt):
    """256 e4m3 experts quantised from N(0, 0.02) with 128 x 128 block scales: bf16 (fmt
    "cfg") or the reference's f32 scale_inv (fmt "ref"); int8 shared expert with per-row bf16
    scales ("cfg") or f16 scales per 128 inputs ("ref")."""
    import torch

    g = torch.Generator(device="cuda").manual_seed(seed)
    L = {"router": _bf16(torch.randn(E + 1, H, generator=g, device="cuda") * 0.02),
         "nw": 1.0 + 0.1 * torch.randn(H, generator=g, device="cuda")}

    def fp8(n, k):
        q = torch.empty(E, n, k, dtype=torch.uint8, device="cuda")
        s = torch.empty(E, n // 128, k // 128, dtype=torch.int16 if fmt == "cfg" else torch.float32, device="cuda")
        for e0 in range(0, E, 16):
            w = torch.randn(16, n, k, generator=g, device="cuda") * 0.02
            blk = w.view(16, n // 128, 128, k // 128, 128)
            amax = blk.abs().amax(dim=(2, 4)).clamp_min(1e-12)
            sb = (amax / 448.0).to(torch.bfloat16).float() if fmt == "cfg" else amax / 448.0
            qv = (blk / sb[:, :, None, :, None]).clamp(-448, 448).to(torch.float8_e4m3fn)
            q[e0:e0 + 16] = qv.view(torch.uint8).view(16, n, k)
            s[e0:e0 + 16] = _bf16(sb) if fmt == "cfg" else sb
        return q, s

    L["gu_q"], L["gu_s"] = fp8(2 * I, H)
    L["d_q"], L["d_s"] = fp8(H, I)

    def q8(n, k):
        q = torch.randint(-127, 128, (n, k), generator=g, device="cuda", dtype=torch.int8)
        if fmt == "cfg":
            return q, _bf16((torch.randn(n, generator=g, device="cuda").abs() * 0.02 + 1e-4) / 73.0)
        return q, _f16((torch.randn(n, k // 128, generator=g, device="cuda").abs() * 0.02 + 1e-4) / 73.0)

    L["sgu_q"], L["sgu_s"] = q8(2 * I, H)
    L["sd_q"], L["sd_s"] = q8(H, I)
    return L


def host_layer(Ld, kind, fmt, used):
    """Oracle layer dict holding only experts `used` (in that order) of a device layer."""
    import torch

    u = torch.as_tensor(np.asarray(used, np.int64), device="cuda")
    h = {k: Ld[k][u].cpu().numpy() for k in ("gu_q", "gu_s", "d_q", "d_s")}
    for k in ("gu_s", "d_s"):
        if h[k].dtype == np.int16:
            h[k] = h[k].view(np.uint16)
    for k in ("sgu_q", "sd_q"):
        h[k] = Ld[k].cpu().numpy()
    for k in ("sgu_s", "sd_s"):
        h[k] = Ld[k].cpu().numpy().view(np.uint16)
    h["router"] = Ld["router"].cpu().numpy().view(np.uint16)
    h["nw"] = Ld["nw"].cpu().numpy()
    if kind == "q4":
        h["sc_kind"] = O.BF16 if fmt == "cfg" else O.F16
    else:
        h["sc_kind"] = O.BF16 if fmt == "cfg" else O.F32
    h["sh_kind"] = O.BF16 if fmt == "cfg" else O.F16
    h["sh_group_gu"], h["sh_group_d"] = (H, I) if fmt == "cfg" else (128, 128)
    h.update({"kind": kind, "E": len(used), "H": H, "I": I, "fmt": fmt})
    return h


def compact(idx):
    """Sorted distinct experts of idx and idx renumbered into them."""
    used = np.unique(idx)
    remap = np.full(E, -1, np.int32)
    remap[used] = np.arange(used.size, dtype=np.int32)
    return used, remap[idx]


# ---------------------------------------------------------------------------------------------
# configuration 3
# ---------------------------------------------------------------------------------------------


def test_cfg3_forty_layer_step_full_size():
    import torch

    import bench

    nl = 40
    print("cfg3: generating 40 layers x 256 int4 experts on the device", flush=True)
    layers = [bench.make_layer_gpu(None, l) for l in range(nl)]
    table = torch.tensor([[Lr[k].data_ptr() for k in KEYS] for Lr in layers], dtype=torch.int64, device="cuda")
    ll = torch.zeros(D.STEP_LL_WORDS, dtype=torch.int64, device="cuda")
    sync = torch.zeros(4, dtype=torch.int32, device="cuda")
    idx = torch.full((nl * TOPK,), -1, dtype=torch.int32, device="cuda")
    wts = torch.zeros(nl * TOPK, device="cuda")
    sg = torch.zeros(nl, device="cuda")
    xs = torch.zeros(nl * H, device="cuda")
    x0 = np.random.default_rng(33).normal(0, 1, H).astype(np.float32)
    xd = dev(x0)
    lib, P = D.lib(), D.ptr
    torch.cuda.synchronize()
    print("cfg3: step launch", flush=True)
    lib.dr_moe_decode_step_bf16s(P(table), nl, P(xd), E, H, I, TOPK, 1e-6, P(ll), P(sync), P(idx), P(wts), P(sg),
                                 P(xs), None, 0, D.stream_ptr())
    torch.cuda.synchronize()
    assert int(host(sync)[1]) == 0
    gi, gw, gs = host(idx).reshape(nl, TOPK), host(wts).reshape(nl, TOPK), host(sg)
    xsh = host(xs).reshape(nl, H)
    assert np.isfinite(xsh).all()
    np.testing.assert_array_equal(bits(host(xd)), bits(xsh[-1]))
    for l in range(nl):
        xin = x0 if l == 0 else xsh[l - 1]
        rh, nwh = layers[l]["router"].cpu().numpy().view(np.uint16), layers[l]["nw"].cpu().numpy()
        _, ri, rw, rs = O.router_topk(rh, xin, nwh, 1e-6, E, TOPK)
        np.testing.assert_array_equal(gi[l], ri, err_msg=f"layer {l} experts")
        np.testing.assert_array_equal(bits(gw[l]), bits(rw), err_msg=f"layer {l} weights")
        assert bits(gs[l:l + 1])[0] == bits(np.float32(rs)), f"layer {l} shared gate"
        if l in (0, 19, 39):
            used, ric = compact(ri)
            hl = host_layer(layers[l], "q4", "cfg", used)
            _, ry = O.moe_decode(hl, xin, ric, rw, rs, xin, H, I, TOPK, nw=nwh, eps=1e-6)
            assert_close(xsh[l], ry, what=f"layer {l} output")
    # graph replays of the whole 40-layer step: the eager call's bits every time
    want = host(xd).copy()
    st = torch.cuda.Stream()
    sp = st.cuda_stream
    xg = torch.zeros(H, device="cuda")
    g = ctypes.c_void_p()
    lib.dr_graph_begin(sp)
    lib.dr_moe_decode_step_bf16s(P(table), nl, P(xg), E, H, I, TOPK, 1e-6, P(ll), P(sync), None, None, None, None, None, 0, sp)
    lib.dr_graph_end(sp, ctypes.byref(g))
    try:
        for rep in range(3):
            xg.copy_(torch.from_numpy(x0).cuda())
            torch.cuda.synchronize()
            lib.dr_graph_launch(g, sp)
            st.synchronize()
            np.testing.assert_array_equal(bits(host(xg)), bits(want), err_msg=f"replay {rep}")
        assert int(host(sync)[1]) == 0
    finally:
        lib.dr_graph_destroy(g)
    del layers, table
    torch.cuda.empty_cache()


@pytest.mark.parametrize("fmt,act_bits", [("cfg", 30), ("ref", 32)])
def test_cfg5_fp8_fused_step_full_size(fmt, act_bits):
    """Configuration 5 batch 1 through the fused step (dr_moe_decode_step_fp8*): three layers of
    256 block-FP8 experts, routing of every layer bit-exact against the oracle's router on the
    step's own layer input, every layer output within 1e-3 + 1e-3 |ref|; act_bits is the routed
    activations' transport between workgroups (30: the default, two fp32 per exchange word;
    32: full fp32 as the reference's act buffer)."""
    import torch

    nl = 3
    print(f"cfg5 fused fp8 step fmt={fmt} act exchange {act_bits}: generating {nl} layers", flush=True)
    layers = [fp8_layer_gpu(90 + l + 10 * (fmt == "ref"), fmt) for l in range(nl)]
    table = torch.tensor([[Lr[k].data_ptr() for k in KEYS] for Lr in layers], dtype=torch.int64, device="cuda")
    ll = torch.zeros(D.STEP_LL_WORDS, dtype=torch.int64, device="cuda")
    sync = torch.zeros(4, dtype=torch.int32, device="cuda")
    idx = torch.full((nl * TOPK,), -1, dtype=torch.int32, device="cuda")
    wts = torch.zeros(nl * TOPK, device="cuda")
    sg = torch.zeros(nl, device="cuda")
    xs = torch.zeros(nl * H, device="cuda")
    x0 = np.random.default_rng(93).normal(0, 1, H).astype(np.float32)
    xd = dev(x0)
    lib, P = D.lib(), D.ptr
    torch.cuda.synchronize()
    fn = lib.dr_moe_decode_step_fp8_bf16s if fmt == "cfg" else lib.dr_moe_decode_step_fp8
    lib.dr_step_set_act_exchange(act_bits)
    try:
        fn(P(table), nl, P(xd), E, H, I, TOPK, 1e-6, P(ll), P(sync), P(idx), P(wts), P(sg), P(xs), None, 0, D.stream_ptr())
        torch.cuda.synchronize()
    finally:
        lib.dr_step_set_act_exchange(0)
    assert int(host(sync)[1]) == 0
    gi, gw, gs = host(idx).reshape(nl, TOPK), host(wts).reshape(nl, TOPK), host(sg)
    xsh = host(xs).reshape(nl, H)
    np.testing.assert_array_equal(bits(host(xd)), bits(xsh[-1]))
    for l in range(nl):
        xin = x0 if l == 0 else xsh[l - 1]
        rh, nwh = layers[l]["router"].cpu().numpy().view(np.uint16), layers[l]["nw"].cpu().numpy()
        _, ri, rw, rs = O.router_topk(rh, xin, nwh, 1e-6, E, TOPK)
        np.testing.assert_array_equal(gi[l], ri, err_msg=f"layer {l} experts")
        np.testing.assert_array_equal(bits(gw[l]), bits(rw), err_msg=f"layer {l} weights")
        assert bits(gs[l:l + 1])[0] == bits(np.float32(rs)), f"layer {l} shared gate"
        used, ric = compact(ri)
        hl = host_layer(layers[l], "fp8", fmt, used)
        _, ry = O.moe_decode(hl, xin, ric, rw, rs, xin, H, I, TOPK, nw=nwh, eps=1e-6)
        assert_close(xsh[l], ry, what=f"layer {l} output")
    del layers, table
    torch.cuda.empty_cache()


# ---------------------------------------------------------------------------------------------
# prefill-path layer chains (configuration 5 batch 4, configuration 4 skewed)
# ---------------------------------------------------------------------------------------------


def run_chain(Ld, kind, fmt, hn, x0, routing=None):
    """Engine::moe_prefill's sequence on the device layer Ld; routing=None runs the router GEMM
    and top-k, else (idx, wts, sgate) are given.  Returns host copies of everything checked."""
    import torch

    rows = hn.shape[0]
    n = rows * TOPK
    L, sp, P = D.lib(), D.stream_ptr(), D.ptr
    dhn, dx = dev(hn), dev(x0)
    logits = torch.zeros(rows * (E + 1), device="cuda")
    if routing is None:
        idx, wts, sg = t_i32(n), torch.zeros(n, device="cuda"), torch.zeros(rows, device="cuda")
        h = ctypes.c_void_p()
        L.dr_cublas_create(ctypes.byref(h), sp)
        L.dr_gemm(h.value, P(dhn), P(Ld["router"]), P(logits), rows, E + 1, H, 0.0)
        L.dr_moe_topk(P(logits), rows, E, TOPK, E + 1, P(idx), P(wts), P(sg), sp)
    else:
        idx, wts, sg = dev(routing[0]), dev(routing[1]), dev(routing[2])
    sact, sh = torch.zeros(rows * I, dtype=torch.int16, device="cuda"), torch.zeros(rows * H, device="cuda")
    getattr(L, "dr_moe_shared_prefill" + ("_bf16s" if fmt == "cfg" else ""))(
        P(Ld["sgu_q"]), P(Ld["sgu_s"]), P(Ld["sd_q"]), P(Ld["sd_s"]), P(dhn), rows, P(sact), P(sh), H, I, sp)
    counts, offsets, slot_of = t_i32(E), t_i32(E), t_i32(n)
    L.dr_moe_group(P(idx), n, E, P(counts), P(offsets), P(slot_of), sp)
    xp = torch.zeros(n * H, dtype=torch.int16, device="cuda")
    L.dr_moe_gather_rows(P(slot_of), rows, TOPK, P(dhn), P(xp), H, sp)
    act, yp = torch.zeros(n * I, dtype=torch.int16, device="cuda"), torch.zeros(n * H, device="cuda")
    name = "dr_moe_prefill" + ("_fp8" if kind == "fp8" else "") + ("_bf16s" if fmt == "cfg" else "")
    getattr(L, name)(P(Ld["gu_q"]), P(Ld["gu_s"]), P(Ld["d_q"]), P(Ld["d_s"]), P(xp), P(offsets), P(counts), P(act),
                     P(yp), E, H, I, sp)
    L.dr_moe_combine(P(dx), P(yp), P(slot_of), P(wts), P(sg), P(sh), rows, TOPK, H, sp)
    torch.cuda.synchronize()
    return {"logits": host(logits).reshape(rows, E + 1), "idx": host(idx), "wts": host(wts), "sg": host(sg),
            "counts": host(counts), "slot_of": host(slot_of), "act": host(act).view(np.uint16).reshape(n, I),
            "sact": host(sact).view(np.uint16).reshape(rows, I), "x": host(dx).reshape(rows, H)}


def check_chain(Ld, kind, fmt, hn, x0, g, ri, rw, rs):
    """Grouping exact; layer output within 1e-3 + 1e-3 |ref| plus the propagation of the bf16
    act rounding flips observed (the bar of the 300-row layer test in test_gpu_prefill.py)."""
    rc, ro, rso = O.moe_group(ri, E)
    np.testing.assert_array_equal(g["counts"], rc)
    np.testing.assert_array_equal(g["slot_of"], rso)
    used, ric = compact(ri)
    np.testing.assert_array_equal(O.moe_group(ric, used.size)[2], rso)  # renumbering keeps the slot order
    Lh = host_layer(Ld, kind, fmt, used)
    check_layer_with_flips(Lh, hn, x0, g["act"], g["sact"], g["x"], ric, rw, rs)


def check_layer_with_flips(Lh, hn, x0, act, sact, xgot, ric, rw, rs):
    """Prefill layer output xgot against O.moe_prefill_layer: |gpu - ref| <= 1e-3 + 1e-3 |ref|
    plus exactly the propagation of the bf16 act rounding flips observed between the GPU's
    routed / shared activations (act, sact: bf16 bits in grouped-slot / row order) and the
    oracle's.  Lh holds only the experts the routing uses, ric the routing renumbered into them."""
    rows = hn.shape[0]
    n = rows * TOPK
    ne = Lh["gu_q"].shape[0]
    Hh, Ih = Lh["H"], Lh["I"]
    ref = O.moe_prefill_layer(Lh, hn, rows, ric, rw, rs, x0, Hh, Ih, TOPK).astype(np.float64)
    cc, co, cso = O.moe_group(ric, ne)
    xpr = np.empty((n, Hh), np.uint16)
    xpr[cso] = hn[np.arange(n) // TOPK]
    ract, _ = O.moe_prefill_experts(Lh, xpr, co, cc, ne, Hh, Ih)
    rsact, _ = O.shared_prefill(Lh, hn, rows, Hh, Ih)
    af, rf = check_act(act, ract, "routed act")
    saf, srf = check_act(sact, rsact, "shared act")
    extra_slot = np.zeros((n, Hh))
    for e in range(ne):
        sl = slice(co[e], co[e] + cc[e])
        d = np.abs(af[sl] - rf[sl])
        if d.any():
            extra_slot[sl] = d @ np.abs(expert_dense(Lh, "d", e).astype(np.float64)).T
    sd = O.dequant_q8(Lh["sd_q"], Lh["sd_s"], Lh["sh_kind"], Lh["sh_group_d"], Hh, Ih).astype(np.float64)
    sig = 1 / (1 + np.exp(-np.asarray(rs, np.float64)))
    extra = sig[:, None] * (np.abs(saf - srf) @ np.abs(sd).T)
    extra += np.einsum("rk,rkc->rc", np.asarray(rw, np.float64).reshape(rows, TOPK), extra_slot[cso.reshape(rows, TOPK)])
    got = np.asarray(xgot, np.float64).reshape(rows, Hh)
    bad = np.abs(got - ref) > 1e-3 + 1e-3 * np.abs(ref) + extra
    print(f"experts hit {ne}, act flips routed {int((af != rf).sum())}, shared {int((saf != srf).sum())}, "
          f"max |err| {np.abs(got - ref).max():.2e}", flush=True)
    assert not bad.any(), f"layer output: {int(bad.sum())} outside tolerance + flip propagation"


@pytest.mark.parametrize("fmt", ["cfg", "ref"])
def test_cfg5_fp8_batch4_decode_chain(fmt):
    import torch

    print(f"cfg5 batch 4 fp8 fmt={fmt}", flush=True)
    Ld = fp8_layer_gpu(41 if fmt == "cfg" else 42, fmt)
    rng = np.random.default_rng(44)
    rows = 4
    hn = synth.f32_to_bf16(rng.normal(0, 1, (rows, H)).astype(np.float32))
    x0 = rng.normal(0, 1, (rows, H)).astype(np.float32)
    g = run_chain(Ld, "fp8", fmt, hn, x0)
    router = Ld["router"].cpu().numpy().view(np.uint16)
    rl = O.router_logits_rows(hn, router, rows, E + 1, H)
    ri, rw, rs = O.moe_topk(rl, rows, E, TOPK, E + 1)
    np.testing.assert_array_equal(g["logits"].view(np.uint32), rl.view(np.uint32))
    np.testing.assert_array_equal(g["idx"], ri)
    np.testing.assert_array_equal(bits(g["wts"]), bits(rw))
    np.testing.assert_array_equal(bits(g["sg"]), bits(rs))
    check_chain(Ld, "fp8", fmt, hn, x0, g, ri, rw, rs)
    del Ld
    torch.cuda.empty_cache()


def test_cfg4_skewed_prefill_chain_full_size():
    import torch

    import bench

    print("cfg4 skewed: 300 rows, 10% of 256 experts get half the pairs", flush=True)
    Ld = bench.make_layer_gpu(None, 7)
    rng = np.random.default_rng(45)
    rows = 300
    n = rows * TOPK
    hot = rng.choice(E, E // 10, replace=False)
    idx = np.empty((rows, TOPK), np.int32)
    for r in range(rows):  # distinct experts per row, half of the picks from the hot set
        nh = int(rng.binomial(TOPK, 0.5))
        hsel = rng.choice(hot, nh, replace=False)
        rest = rng.choice(np.setdiff1d(np.arange(E), hsel), TOPK - nh, replace=False)
        idx[r] = rng.permutation(np.concatenate([hsel, rest]))
    idx = idx.ravel()
    w = rng.random((rows, TOPK)).astype(np.float32) + 0.1
    wts = (w / w.sum(1, keepdims=True)).astype(np.float32).ravel()
    sg = rng.normal(0, 1, rows).astype(np.float32)
    hn = synth.f32_to_bf16(rng.normal(0, 1, (rows, H)).astype(np.float32))
    x0 = rng.normal(0, 1, (rows, H)).astype(np.float32)
    g = run_chain(Ld, "q4", "cfg", hn, x0, routing=(idx, wts, sg))
    cnt = np.bincount(idx, minlength=E)
    assert cnt[hot].sum() >= 0.4 * n and cnt.max() >= 30, "routing is not skewed as intended"
    check_chain(Ld, "q4", "cfg", hn, x0, g, idx, wts, sg)
    del Ld
    torch.cuda.empty_cache()
