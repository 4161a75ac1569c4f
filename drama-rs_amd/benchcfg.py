"""Measurements of the benchmark configurations other than the headline 40-layer decode step
(configurations 1, 4 and 5), used by bench.py.  Every timing is HIP events on the stream the
kernels run on; weights are rotated over distinct copies wherever one launch would otherwise
re-read data that fits in the 256 MB memory-side cache."""
from __future__ import annotations

import ctypes

import torch

import dramamoe as D

HBM = 8000.0  # GB/s
H, I, E, TOPK = 2048, 512, 256, 8


def bf16_bits(t):
    return t.to(torch.bfloat16).view(torch.int16)


def timed(fn, iters, st, warmup=3):
    # inputs are generated on torch's default stream; the kernels run on st
    torch.cuda.synchronize()
    for i in range(warmup):
        fn(i)
    st.synchronize()
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    a.record(st)
    for i in range(iters):
        fn(i)
    b.record(st)
    torch.cuda.synchronize()
    return a.elapsed_time(b) / iters  # ms


def timed_graph(fn, iters, st, period):
    """fn(0) .. fn(period - 1) captured once into a HIP graph (dr_graph_*), replayed: the
    per-call time without host launch gaps, as a caller that records its step in a graph sees it."""
    lib = D.lib()
    sp = st.cuda_stream
    torch.cuda.synchronize()
    g = ctypes.c_void_p()
    lib.dr_graph_begin(sp)
    for i in range(period):
        fn(i)
    lib.dr_graph_end(sp, ctypes.byref(g))
    try:
        for _ in range(2):
            lib.dr_graph_launch(g, sp)
        st.synchronize()
        reps = max(1, iters // period)
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record(st)
        for _ in range(reps):
            lib.dr_graph_launch(g, sp)
        b.record(st)
        torch.cuda.synchronize()
        return a.elapsed_time(b) / (reps * period)  # ms
    finally:
        lib.dr_graph_destroy(g)


def rec(us, nbytes, **kw):
    gbs = nbytes / (us * 1e-6) / 1e9
    out = {"us": round(us, 2), "bytes": int(nbytes), "GBps": round(gbs, 1), "frac_hbm": round(gbs / HBM, 4)}
    out.update(kw)
    return out


def config1_gemv(lib, st, iters=200):
    """Single int4 GEMV 1024 x 2048, group 64, bf16 scale/min, bf16 x, bf16 + f32 out."""
    N, K, R = 1024, 2048, 256
    g = torch.Generator(device="cuda").manual_seed(11)
    q = torch.randint(0, 256, (R, N, K // 2), generator=g, device="cuda", dtype=torch.uint8)
    sc = torch.randn(R, N, K // 64, generator=g, device="cuda").abs() * 0.02 + 1e-4
    mn = torch.randn(R, N, K // 64, generator=g, device="cuda") * 0.02
    sm = torch.stack([bf16_bits(sc), bf16_bits(mn)], -1).contiguous()
    del sc, mn
    x = bf16_bits(torch.randn(K, generator=g, device="cuda"))
    y = torch.empty(N, device="cuda")
    yb = torch.empty(N, dtype=torch.int16, device="cuda")
    sp = st.cuda_stream
    P = D.ptr
    qs, ss = q.stride(0), sm.stride(0) * 2

    def f(i):
        r = i % R
        lib.dr_gemv_q4_bf16s(q.data_ptr() + r * qs, sm.data_ptr() + r * ss, P(x), P(y), P(yb), N, K, sp)

    ms = timed(f, iters, st)
    msg = timed_graph(f, iters, st, 64)
    nbytes = N * K // 2 + N * (K // 64) * 4 + K * 2 + N * 6
    return rec(ms * 1000, nbytes, shape=f"{N}x{K}", us_graph=round(msg * 1000, 2),
               note="rotated over 256 distinct matrices; per call with launch gaps (eager) and replayed from a "
                    "HIP graph of 64 calls (us_graph); the kernel's own duration is in the rocprof summary")


class Prefill:
    """Buffers of one prefill layer call for `rows` rows (Engine::moe_prefill, src/engine.rs:544-604)."""

    def __init__(self, rows, st, overlap=True):
        z = lambda n, dt=torch.float32: torch.zeros(n, dtype=dt, device="cuda")
        n = rows * TOPK
        self.rows, self.n, self.st, self.sp = rows, n, st, st.cuda_stream
        self.overlap = overlap and rows >= 64  # for a few rows the cross-stream events cost more than they save
        g = torch.Generator(device="cuda").manual_seed(21)
        self.hn = bf16_bits(torch.randn(rows, H, generator=g, device="cuda"))
        self.x = torch.randn(rows, H, generator=g, device="cuda")
        self.logits = z(rows * (E + 1))
        self.idx, self.wts, self.sg = z(n, torch.int32), z(n), z(rows)
        self.sact, self.sh = z(rows * I, torch.int16), z(rows * H)
        self.counts, self.offsets, self.slot_of = z(E, torch.int32), z(E, torch.int32), z(n, torch.int32)
        self.row_of_slot, self.counter = z(n + 16, torch.int32), z(4, torch.int32)
        self.act, self.yp = z(n * I, torch.int16), z(n * H)
        self.grouped = False  # set by router(): top-k came with its grouping
        h = ctypes.c_void_p()
        D.lib().dr_cublas_create(ctypes.byref(h), self.sp)
        self.h = h.value
        # the shared expert needs only hn: it runs on a second stream beside the routing,
        # grouping and gather (the grouping kernel is a single workgroup)
        self.st2 = torch.cuda.Stream()
        self.ev_fork, self.ev_join = torch.cuda.Event(), torch.cuda.Event()

    def shared_begin(self, lib, L):
        P = D.ptr
        if not self.overlap:
            lib.dr_moe_shared_prefill_bf16s(P(L["sgu_q"]), P(L["sgu_s"]), P(L["sd_q"]), P(L["sd_s"]), P(self.hn),
                                            self.rows, P(self.sact), P(self.sh), H, I, self.sp)
            return
        self.ev_fork.record(self.st)
        self.st2.wait_event(self.ev_fork)
        lib.dr_moe_shared_prefill_bf16s(P(L["sgu_q"]), P(L["sgu_s"]), P(L["sd_q"]), P(L["sd_s"]), P(self.hn), self.rows,
                                        P(self.sact), P(self.sh), H, I, self.st2.cuda_stream)
        self.ev_join.record(self.st2)

    def router(self, lib, L):
        P = D.ptr
        lib.dr_gemm(self.h, P(self.hn), P(L["router"]), P(self.logits), self.rows, E + 1, H, 0.0)
        lib.dr_moe_topk_group(P(self.logits), self.rows, E, TOPK, E + 1, P(self.idx), P(self.wts), P(self.sg),
                              P(self.counts), P(self.offsets), P(self.slot_of), P(self.row_of_slot), P(self.counter),
                              self.sp)
        self.grouped = True

    def experts(self, lib, L, fp8=False, shared_started=False, packed=False):
        """packed: L's routed experts are in the tile-step layout (packed_q4)."""
        P, sp = D.ptr, self.sp
        if not shared_started:
            self.shared_begin(lib, L)
        if not self.grouped:  # a routing given from outside (the skewed variant)
            lib.dr_moe_group_rows(P(self.idx), self.rows, TOPK, E, P(self.counts), P(self.offsets), P(self.slot_of),
                                  P(self.row_of_slot), sp)
        self.grouped = False
        if fp8:
            f = lib.dr_moe_prefill_rows_packed_fp8_bf16s if packed else lib.dr_moe_prefill_rows_fp8_bf16s
        else:
            f = lib.dr_moe_prefill_rows_packed_bf16s if packed else lib.dr_moe_prefill_rows_bf16s
        f(P(L["gu_q"]), P(L["gu_s"]), P(L["d_q"]), P(L["d_s"]), P(self.hn), self.rows, P(self.row_of_slot),
          P(self.offsets), P(self.counts), P(self.act), P(self.yp), E, H, I, sp)
        if self.overlap:
            self.st.wait_event(self.ev_join)
        lib.dr_moe_combine(P(self.x), P(self.yp), P(self.slot_of), P(self.wts), P(self.sg), P(self.sh), self.rows, TOPK,
                           H, sp)

    def layer_bytes(self, L, include_router=True):
        hit = int((self.counts > 0).sum().item())
        per_expert = sum(L[k].numel() * L[k].element_size() for k in ("gu_q", "gu_s", "d_q", "d_s")) // E
        shared = sum(L[k].numel() * L[k].element_size() for k in ("sgu_q", "sgu_s", "sd_q", "sd_s"))
        r, n = self.rows, self.n
        acts = (r * H * 2 * 3          # hn read by router, shared expert and gate_up
                + n * I * 2 * 2        # act written and read
                + n * H * 4 * 2        # yp written and read
                + r * I * 2 * 2 + r * H * 4 * 2  # shared act / out
                + r * H * 4 * 2)       # x read and written
        return hit * per_expert + shared + (L["router"].numel() * 2 if include_router else 0) + acts, hit


def packed_q4(lib, L, st):
    """L with its routed experts in the tile-step layout of dr_moe_pack_q4 (a second copy, made
    once and kept in L)."""
    if "pk" not in L:
        P = D.ptr
        pk = dict(L)
        for q, sc, n, k in (("gu_q", "gu_s", 2 * I, H), ("d_q", "d_s", H, I)):
            pk[q], pk[sc] = torch.empty_like(L[q]), torch.empty_like(L[sc])
            lib.dr_moe_pack_q4(P(L[q]), P(L[sc]), E, n, k, P(pk[q]), P(pk[sc]), st.cuda_stream)
        st.synchronize()
        L["pk"] = pk
    return L["pk"]


def packed_fp8(lib, L, st):
    """L with its routed e4m3 experts in the tile-step layout of dr_moe_pack_fp8 (scales shared)."""
    if "pk" not in L:
        pk = dict(L)
        for q, n, k in (("gu_q", 2 * I, H), ("d_q", H, I)):
            pk[q] = torch.empty_like(L[q])
            if lib.dr_moe_pack_fp8(D.ptr(L[q]), E, n, k, D.ptr(pk[q]), st.cuda_stream) != 0:
                raise RuntimeError("dr_moe_pack_fp8 rejected the layer")
        st.synchronize()
        L["pk"] = pk
    return L["pk"]


def config4_prefill(lib, layers, st, iters=40, overlap=True):
    """300 token rows, top-8 of 256 (2400 pairs), rotated over the 40 resident layers; the
    routed experts read from their tile-step copy (packed_q4), the reference layout beside it."""
    pf = Prefill(300, st, overlap)
    nl = len(layers)
    pl = [packed_q4(lib, L, st) for L in layers]

    def full(i, packed=True):
        L = (pl if packed else layers)[i % nl]
        pf.shared_begin(lib, L)
        pf.router(lib, L)
        pf.experts(lib, L, shared_started=True, packed=packed)

    ms_ref = timed(lambda i: full(i, False), iters, st)
    ms = timed(full, iters, st)
    msg = timed_graph(full, iters, st, min(nl, 8))
    nbytes, hit = pf.layer_bytes(layers[0])
    cnt = pf.counts.cpu()
    uniform = rec(ms * 1000, nbytes, experts_hit=hit, rows_per_expert_max=int(cnt.max()), pairs=pf.n,
                  us_graph=round(msg * 1000, 2), us_reference_layout=round(ms_ref * 1000, 2),
                  note="router GEMM + top-k with grouping + grouped GEMM (token rows read through the slot map, "
                       "experts in the tile-step layout) + combine" + (
                      ", the shared expert on a second stream beside them" if pf.overlap else " + shared, one stream")
                       + "; us_graph: replayed from a HIP graph; us_reference_layout: the experts read in the "
                         "reference layout (dr_moe_prefill_rows_bf16s)")
    # the same 300 rows' experts (routing of the last uniform call) two ways: the grouped MFMA
    # path (grouping, gate_up, down, combine, shared expert) and the small-batch GEMV kernels
    # (dr_moe_decode_rows_bf16s: each weight row read once per 60-row call and multiplied by
    # every row routed to it with VALU FMAs), 5 calls of 60 rows
    pf.grouped = False
    ms_mfma = timed(lambda i: pf.experts(lib, pl[i % nl], packed=True), iters, st)
    P = D.ptr
    rows_c = 60
    xg = pf.x.clone()
    act_g = torch.zeros(rows_c * (TOPK + 1) * I, device="cuda")

    def gemv_path(i):
        L = layers[i % nl]
        for r0 in range(0, pf.rows, rows_c):
            xr = xg[r0:r0 + rows_c]
            lib.dr_moe_decode_rows_bf16s(P(L["gu_q"]), P(L["gu_s"]), P(L["d_q"]), P(L["d_s"]), P(L["sgu_q"]),
                                         P(L["sgu_s"]), P(L["sd_q"]), P(L["sd_s"]), P(xr), P(pf.idx[r0 * TOPK:]),
                                         P(pf.wts[r0 * TOPK:]), P(pf.sg[r0:]), P(xr), P(act_g), P(xr), None, rows_c,
                                         H, I, TOPK, None, 1e-6, pf.sp)

    ms_gemv = timed(gemv_path, max(4, iters // 4), st)
    mfma_vs_gemv = {"mfma_grouped_us": round(ms_mfma * 1000, 2), "gemv_rows_us": round(ms_gemv * 1000, 2),
                    "rows_per_expert_mean": round(pf.n / max(1, hit), 2),
                    "note": "experts of one 300-row layer (routing given): grouped MFMA kernels on the tile-step copy (grouping, gate_up, "
                            "down, combine, shared expert) against the small-batch GEMV kernels "
                            "(dr_moe_decode_rows_bf16s, 5 calls of 60 rows, shared expert and residual included)"}
    # skewed routing: 10% of experts receive 50% of the pairs (synthetic indices)
    g = torch.Generator(device="cuda").manual_seed(31)
    hot = torch.randperm(E, generator=g, device="cuda")[: E // 10]
    pick_hot = torch.rand(pf.n, generator=g, device="cuda") < 0.5
    idx = torch.where(pick_hot, hot[torch.randint(0, hot.numel(), (pf.n,), generator=g, device="cuda")],
                      torch.randint(0, E, (pf.n,), generator=g, device="cuda")).to(torch.int32)
    pf.idx.copy_(idx)
    pf.wts.fill_(1.0 / TOPK)

    def skewed(i):
        pf.experts(lib, pl[i % nl], packed=True)

    ms2 = timed(skewed, iters, st)
    nbytes2, hit2 = pf.layer_bytes(layers[0], include_router=False)
    cnt2 = pf.counts.cpu()
    skew = rec(ms2 * 1000, nbytes2, experts_hit=hit2, rows_per_expert_max=int(cnt2.max()),
               note="skewed: 10% of experts get 50% of the pairs; routing given, no router GEMM")
    return {"uniform": uniform, "skewed": skew, "mfma_vs_gemv": mfma_vs_gemv,
            "shared_expert": shared_prefill_compare(lib, st, pf.rows)}


def shared_prefill_compare(lib, st, rows, iters=40, copies=8):
    """The shared expert of a prefill layer two ways, on the reference's weight format (int8,
    f16 scale per 128 inputs): the sequence the reference engine issues (src/engine.rs:351-355,
    560-562: dr_dequant_q8 -> dr_gemm [rows x 1024 x 2048] -> dr_swiglu_rows -> dr_dequant_q8
    -> dr_gemm [rows x 2048 x 512]) and the fused dr_moe_shared_prefill.  dr_gemm keeps the
    router's canonical fp32 summation order (one symbol serves both), so it is not a fast GEMM."""
    g = torch.Generator(device="cuda").manual_seed(61)
    sp, P = st.cuda_stream, D.ptr
    z = lambda n, dt=torch.float32: torch.zeros(n, dtype=dt, device="cuda")
    Ws = []
    for _ in range(copies):
        Ws.append({"sgu_q": torch.randint(-127, 128, (2 * I, H), generator=g, device="cuda", dtype=torch.int8),
                   "sgu_s": (torch.rand(2 * I, H // 128, generator=g, device="cuda") * 1e-3 + 1e-4).half(),
                   "sd_q": torch.randint(-127, 128, (H, I), generator=g, device="cuda", dtype=torch.int8),
                   "sd_s": (torch.rand(H, I // 128, generator=g, device="cuda") * 1e-3 + 1e-4).half()})
    hn = bf16_bits(torch.randn(rows, H, generator=g, device="cuda"))
    wbuf, hh, act, out = z(2 * I * H, torch.int16), z(rows * 2 * I), z(rows * I, torch.int16), z(rows * H)
    h = ctypes.c_void_p()
    lib.dr_cublas_create(ctypes.byref(h), sp)

    def ref_seq(i):
        w = Ws[i % copies]
        lib.dr_dequant_q8(P(w["sgu_q"]), P(w["sgu_s"]), P(wbuf), 2 * I, H, sp)
        lib.dr_gemm(h.value, P(hn), P(wbuf), P(hh), rows, 2 * I, H, 0.0)
        lib.dr_swiglu_rows(P(hh), P(act), rows, I, sp)
        lib.dr_dequant_q8(P(w["sd_q"]), P(w["sd_s"]), P(wbuf), H, I, sp)
        lib.dr_gemm(h.value, P(act), P(wbuf), P(out), rows, H, I, 0.0)

    def fused(i):
        w = Ws[i % copies]
        lib.dr_moe_shared_prefill(P(w["sgu_q"]), P(w["sgu_s"]), P(w["sd_q"]), P(w["sd_s"]), P(hn), rows, P(act), P(out),
                                  H, I, sp)

    ms_ref, ms_fused = timed(ref_seq, iters, st), timed(fused, iters, st)
    wbytes = 2 * I * H + 2 * I * (H // 128) * 2 + H * I + H * (I // 128) * 2
    nbytes = wbytes + rows * H * 2 + rows * H * 4
    return {"reference_sequence": rec(ms_ref * 1000, nbytes, launches=5,
                                      note="dr_dequant_q8 -> dr_gemm -> dr_swiglu_rows -> dr_dequant_q8 -> dr_gemm "
                                           "(the reference engine's calls); bytes = int8 weights + scales + hn + out"),
            "fused": rec(ms_fused * 1000, nbytes, launches=1, note="dr_moe_shared_prefill, same weights and rows")}


def make_fp8_layer(seed):
    """256 e4m3 experts quantised from N(0, 0.02) with bf16 128 x 128 block scales."""
    g = torch.Generator(device="cuda").manual_seed(seed)
    L = {"router": bf16_bits(torch.randn(E + 1, H, generator=g, device="cuda") * 0.02),
         "nw": 1.0 + 0.1 * torch.randn(H, generator=g, device="cuda")}

    def fp8(n, k):
        q = torch.empty(E, n, k, dtype=torch.uint8, device="cuda")
        s = torch.empty(E, n // 128, k // 128, dtype=torch.int16, device="cuda")
        for e0 in range(0, E, 16):
            w = torch.randn(16, n, k, generator=g, device="cuda") * 0.02
            blk = w.view(16, n // 128, 128, k // 128, 128)
            amax = blk.abs().amax(dim=(2, 4)).clamp_min(1e-12)
            sb = (amax / 448.0).to(torch.bfloat16)
            qv = (blk / sb.float()[:, :, None, :, None]).clamp(-448, 448).to(torch.float8_e4m3fn)
            q[e0:e0 + 16] = qv.view(torch.uint8).view(16, n, k)
            s[e0:e0 + 16] = sb.view(torch.int16)
        return q, s

    L["gu_q"], L["gu_s"] = fp8(2 * I, H)
    L["d_q"], L["d_s"] = fp8(H, I)

    def q8(n, k):
        return (torch.randint(-127, 128, (n, k), generator=g, device="cuda", dtype=torch.int8),
                bf16_bits((torch.randn(n, generator=g, device="cuda").abs() * 0.02 + 1e-4) / 73.0))

    L["sgu_q"], L["sgu_s"] = q8(2 * I, H)
    L["sd_q"], L["sd_s"] = q8(H, I)
    return L


def config5_fp8(lib, st, iters=100, copies=4):
    out = {}
    L = make_fp8_layer(41)
    # the calls rotate over `copies` copies of the layer at distinct addresses (3.2 GB), so no
    # call finds its weights in the 256 MB MALL
    Ls = [L] + [{k: v.clone() for k, v in L.items()} for _ in range(copies - 1)]
    sp, P = st.cuda_stream, D.ptr
    z = lambda n, dt=torch.float32: torch.zeros(n, dtype=dt, device="cuda")
    x = torch.randn(H, device="cuda")
    logits, idx, wts, sg, counter, act = z(E + 1), z(TOPK, torch.int32), z(TOPK), z(1), z(4, torch.int32), z(9 * I)

    def dec(i):
        L = Ls[i % copies]
        lib.dr_router_topk(P(L["router"]), P(x), P(L["nw"]), 1e-6, P(logits), E, TOPK, H, P(idx), P(wts), P(sg),
                           P(counter), None, None, None, None, 0, 0, 0, 0, sp)
        lib.dr_moe_decode_fp8_bf16s(P(L["gu_q"]), P(L["gu_s"]), P(L["d_q"]), P(L["d_s"]), P(L["sgu_q"]), P(L["sgu_s"]),
                                    P(L["sd_q"]), P(L["sd_s"]), P(x), P(idx), P(wts), P(sg), P(x), P(act), P(x), None,
                                    H, I, TOPK, P(L["nw"]), 1e-6, None, 0, sp)

    ms = timed(dec, iters, st)
    per_expert = sum(L[k].numel() * L[k].element_size() for k in ("gu_q", "gu_s", "d_q", "d_s")) // E
    shared = sum(L[k].numel() * L[k].element_size() for k in ("sgu_q", "sgu_s", "sd_q", "sd_s"))
    b1 = L["router"].numel() * 2 + TOPK * per_expert + shared + 6 * H * 4 + 2 * 9 * I * 4
    msg = timed_graph(dec, iters, st, copies)
    out["decode_batch1"] = rec(ms * 1000, b1, us_graph=round(msg * 1000, 2),
                               note="router + fp8 gate_up + down + int8 shared; x evolves per call; 4 layer copies "
                                    "rotated; us_graph: the same calls replayed from a HIP graph")
    # batch 1 with the router in the gate_up launch (2 launches)
    c1, tags1 = z(4, torch.int32), z(896, torch.int64)

    def dec_r(i):
        L = Ls[i % copies]
        lib.dr_moe_decode_rows_routed_fp8_bf16s(P(L["router"]), P(L["nw"]), 1e-6, E, P(L["gu_q"]), P(L["gu_s"]),
                                                P(L["d_q"]), P(L["d_s"]), P(L["sgu_q"]), P(L["sgu_s"]), P(L["sd_q"]),
                                                P(L["sd_s"]), P(x), P(logits), P(idx), P(wts), P(sg), P(c1), P(tags1),
                                                P(x), P(act), P(x), None, 1, H, I, TOPK, sp)

    msr = timed(dec_r, iters, st)
    out["decode_batch1_routed"] = rec(msr * 1000, b1, note="router + top-k in the gate_up launch, then down "
                                                           "(dr_moe_decode_rows_routed_fp8_bf16s, 1 row)")
    # the fused persistent step over 40 layers: layer l has its own router (so the routing
    # differs from layer to layer) and the experts of copy l % copies (a layer's 8 experts are
    # one of 4 x 256 3-MiB blocks, so few are still in the MALL from an earlier layer)
    keys = ("router", "nw", "gu_q", "gu_s", "d_q", "d_s", "sgu_q", "sgu_s", "sd_q", "sd_s")
    nl = 40
    gr = torch.Generator(device="cuda").manual_seed(43)
    routers = [bf16_bits(torch.randn(E + 1, H, generator=gr, device="cuda") * 0.02) for _ in range(nl)]
    table = torch.tensor([[(routers[l] if k == "router" else Ls[l % copies][k]).data_ptr() for k in keys]
                          for l in range(nl)], dtype=torch.int64, device="cuda")
    ll, sync = z(D.STEP_LL_WORDS, torch.int64), z(4, torch.int32)

    def fused(i):
        lib.dr_moe_decode_step_fp8_bf16s(P(table), nl, P(x), E, H, I, TOPK, 1e-6, P(ll), P(sync), None, None, None,
                                         None, None, 0, sp)

    msf = timed(fused, max(1, iters // 10), st)
    if int(sync[1].item()) != 0:
        raise RuntimeError("dr_moe_decode_step_fp8_bf16s timed out")
    out["decode_batch1_fused"] = rec(msf * 1000 / nl, b1,
                                     note=f"{nl} layers (own router each, experts of copy l % {copies}) in one "
                                          "dr_moe_decode_step_fp8_bf16s launch; us per layer")
    # batch 4 through the grouped (prefill) path: union of up to 32 experts
    pf = Prefill(4, st)

    def b4(i):
        pf.router(lib, Ls[i % copies])
        pf.experts(lib, Ls[i % copies], fp8=True)

    ms4 = timed(b4, iters, st)
    ms4g = timed_graph(b4, iters, st, copies)
    nb4, hit = pf.layer_bytes(L)
    out["decode_batch4_grouped"] = rec(ms4 * 1000, nb4, experts_hit=hit, us_graph=round(ms4g * 1000, 2),
                                       note="4 rows via the prefill path (router GEMM, top-k with grouping, "
                                            "grouped MFMA GEMMs, combine: 7 launches); us_graph: from a HIP graph")
    # the small-batch decode path: router + top-k for the 4 rows in one launch, then the batch-1
    # chain's expert kernels over the 4 rows (3 launches)
    x4 = torch.randn(4, H, device="cuda")
    lg4, idx4, wts4, sg4 = z(4 * (E + 1)), z(4 * TOPK, torch.int32), z(4 * TOPK), z(4)
    act4 = z(4 * 9 * I)

    def b4r(i):
        Lc = Ls[i % copies]
        lib.dr_router_topk_rows(P(Lc["router"]), P(x4), P(Lc["nw"]), 1e-6, P(lg4), E, TOPK, H, 4, P(idx4), P(wts4),
                                P(sg4), P(counter), sp)
        lib.dr_moe_decode_rows_fp8_bf16s(P(Lc["gu_q"]), P(Lc["gu_s"]), P(Lc["d_q"]), P(Lc["d_s"]), P(Lc["sgu_q"]),
                                         P(Lc["sgu_s"]), P(Lc["sd_q"]), P(Lc["sd_s"]), P(x4), P(idx4), P(wts4), P(sg4),
                                         P(x4), P(act4), P(x4), None, 4, H, I, TOPK, P(Lc["nw"]), 1e-6, sp)

    ms4r = timed(b4r, iters, st)
    ms4rg = timed_graph(b4r, iters, st, copies)
    hit4 = int(torch.unique(idx4).numel())
    nb4r = (L["router"].numel() * 2 + hit4 * per_expert + shared + 4 * 6 * H * 4 + 4 * 2 * 9 * I * 4)
    out["decode_batch4"] = rec(ms4r * 1000, nb4r, experts_hit=hit4, us_graph=round(ms4rg * 1000, 2),
                               note="4 rows via the small-batch decode path (dr_router_topk_rows + "
                                    "dr_moe_decode_rows_fp8_bf16s, 3 launches); bytes = router + distinct "
                                    "experts + shared + vectors; us_graph: replayed from a HIP graph")
    # the same with the router in the gate_up launch (2 launches)
    c4, tags4 = z(4, torch.int32), z(896, torch.int64)

    def b4f(i):
        Lc = Ls[i % copies]
        lib.dr_moe_decode_rows_routed_fp8_bf16s(P(Lc["router"]), P(Lc["nw"]), 1e-6, E, P(Lc["gu_q"]), P(Lc["gu_s"]),
                                                P(Lc["d_q"]), P(Lc["d_s"]), P(Lc["sgu_q"]), P(Lc["sgu_s"]),
                                                P(Lc["sd_q"]), P(Lc["sd_s"]), P(x4), P(lg4), P(idx4), P(wts4), P(sg4),
                                                P(c4), P(tags4), P(x4), P(act4), P(x4), None, 4, H, I, TOPK, sp)

    ms4f = timed(b4f, iters, st)
    ms4fg = timed_graph(b4f, iters, st, copies)
    if lib.dr_last_error() != 0:
        raise RuntimeError("dr_moe_decode_rows_routed_fp8_bf16s reported an error")
    out["decode_batch4_routed"] = rec(ms4f * 1000, nb4r, experts_hit=hit4, us_graph=round(ms4fg * 1000, 2),
                                      note="4 rows, router + top-k in the gate_up launch, then down "
                                           "(dr_moe_decode_rows_routed_fp8_bf16s, 2 launches); bytes as decode_batch4")
    # 300-row prefill of the fp8 layer copies (configuration 4's shape), reference layout and
    # tile-step copy (dr_moe_pack_fp8)
    pf3 = Prefill(300, st)
    pks = [packed_fp8(lib, Lc, st) for Lc in Ls]

    def p300(i, packed):
        Lc = (pks if packed else Ls)[i % copies]
        pf3.router(lib, Lc)
        pf3.experts(lib, Lc, fp8=True, packed=packed)

    ms3 = timed(lambda i: p300(i, False), iters // 2, st)
    ms3p = timed(lambda i: p300(i, True), iters // 2, st)
    nb3, hit3 = pf3.layer_bytes(L)
    out["prefill_fp8_300"] = rec(ms3p * 1000, nb3, experts_hit=hit3, us_reference_layout=round(ms3 * 1000, 2),
                                 note="300 rows x top-8 of 256, fp8 experts read from their tile-step copy "
                                      "(dr_moe_prefill_rows_packed_fp8_bf16s); us_reference_layout: "
                                      "dr_moe_prefill_rows_fp8_bf16s on the [e][n][k] layout")
    del L, Ls, routers, pks, pf3
    torch.cuda.empty_cache()
    # int8 lm_head 2048 x 151936 with per-row bf16 scales, and 2048 x 2048 projections
    g = torch.Generator(device="cuda").manual_seed(51)
    V = 151936
    W = torch.randint(-127, 128, (V, H), generator=g, device="cuda", dtype=torch.int8)
    S = bf16_bits(torch.rand(V, generator=g, device="cuda") * 1e-3 + 1e-5)
    y = z(V)
    xs = torch.randn(H, device="cuda")
    msl = timed(lambda i: lib.dr_gemv_q8_bf16s(P(W), P(S), P(xs), None, P(y), V, H, None, 0.0, sp), 20, st)
    out["lm_head_int8"] = rec(msl * 1000, V * H + V * 2 + H * 4 + V * 4, shape=f"{V}x{H}")
    del W, S, y
    R = 64
    Wp = torch.randint(-127, 128, (R, H, H), generator=g, device="cuda", dtype=torch.int8)
    Sp = bf16_bits(torch.rand(R, H, generator=g, device="cuda") * 1e-3 + 1e-5)
    yp = z(H)
    mp = timed(lambda i: lib.dr_gemv_q8_bf16s(Wp.data_ptr() + (i % R) * H * H, Sp.data_ptr() + (i % R) * H * 2, P(xs),
                                               None, P(yp), H, H, None, 0.0, sp), 200, st)
    out["proj_int8_2048"] = rec(mp * 1000, H * H + H * 2 + H * 8, shape="2048x2048",
                                note="rotated over 64 matrices; launch-bound")
    return out
