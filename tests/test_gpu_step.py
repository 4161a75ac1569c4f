"""GPU parity of the fused multi-layer decode step (dr_moe_decode_step*) through the C ABI.

Layer by layer, the routing of the step (experts, weights and shared gate) must equal the
oracle's router on the step's own layer input bit for bit, and every layer output must match
the oracle's dequant-then-fp64 layer (router -> experts -> shared -> combine, x = res = y)
within |gpu - ref| <= 1e-3 + 1e-3 |ref|."""
import numpy as np
import pytest

import dramamoe as D
import oracle as O
import synth
from helpers import assert_close, bits, dev, host

pytestmark = pytest.mark.gpu

H, I, TOPK = 2048, 512, 8
LL_WORDS = D.STEP_LL_WORDS
KEYS = ("router", "nw", "gu_q", "gu_s", "d_q", "d_s", "sgu_q", "sgu_s", "sd_q", "sd_s")


class Stack:
    """n_layers host layers, their device copies and the device table of dr_decode_layer."""

    def __init__(self, seeds, E, fmt, with_norm=True, kind="q4"):
        import torch

        self.E, self.fmt, self.kind = E, fmt, kind
        self.h = [synth.make_layer(s, E=E, fmt=fmt, with_norm=with_norm, kind=kind, quick=True) for s in seeds]
        self.d = [{k: (dev(L[k]) if L[k] is not None else None) for k in KEYS} for L in self.h]
        tab = np.array([[D.ptr(t[k]) if t[k] is not None else 0 for k in KEYS] for t in self.d], np.uint64)
        self.table = torch.from_numpy(tab.view(np.int64)).to("cuda:0")
        self.ll = torch.zeros(LL_WORDS, dtype=torch.int64, device="cuda")
        self.sync = torch.zeros(4, dtype=torch.int32, device="cuda")

    def run(self, x_dev, want_outputs=True):
        import torch

        n = len(self.h)
        idx = torch.full((n * TOPK,), -1, dtype=torch.int32, device="cuda")
        wts = torch.zeros(n * TOPK, device="cuda")
        sg = torch.zeros(n, device="cuda")
        xs = torch.zeros(n * H, device="cuda")
        name = "dr_moe_decode_step" + ("_fp8" if self.kind == "fp8" else "") + ("" if self.fmt == "ref" else "_bf16s")
        fn = getattr(D.lib(), name)
        fn(D.ptr(self.table), n, D.ptr(x_dev), self.E, H, I, TOPK, 1e-6, D.ptr(self.ll), D.ptr(self.sync),
           D.ptr(idx) if want_outputs else None, D.ptr(wts) if want_outputs else None,
           D.ptr(sg) if want_outputs else None, D.ptr(xs) if want_outputs else None, None, 0, D.stream_ptr())
        torch.cuda.synchronize()
        return host(idx).reshape(n, TOPK), host(wts).reshape(n, TOPK), host(sg), host(xs).reshape(n, H)


def check_stack(st, x0, idx, wts, sg, xs, x_final):
    xin = x0
    for l, L in enumerate(st.h):
        nw = L["nw"]
        _, ri, rw, rs = O.router_topk(L["router"], xin, nw, 1e-6, st.E, TOPK)
        np.testing.assert_array_equal(idx[l], ri, err_msg=f"layer {l} experts")
        np.testing.assert_array_equal(bits(wts[l]), bits(rw), err_msg=f"layer {l} weights")
        assert bits(sg[l:l + 1])[0] == bits(np.float32(rs)), f"layer {l} shared gate"
        _, ry = O.moe_decode(L, xin, ri, rw, rs, xin, H, I, TOPK, nw=nw, eps=1e-6)
        assert_close(xs[l], ry, what=f"layer {l} output")
        xin = xs[l].copy()  # the next layer's input is the step's own output (as the engine's)
    np.testing.assert_array_equal(bits(x_final), bits(xs[-1]))


@pytest.mark.parametrize("fmt,E,n,bits", [("cfg", 256, 3, 32), ("ref", 256, 2, 32), ("cfg", 64, 4, 32), ("cfg", 8, 2, 32),
                                          ("cfg", 256, 3, 30), ("ref", 64, 2, 30)])
def test_step_matches_oracle_layer_by_layer(fmt, E, n, bits):
    """bits: transport of the routed activations between workgroups (fp32 with a 32-bit tag, or
    fp32 with the phase in the two low mantissa bits)."""
    print(f"step parity fmt={fmt} E={E} layers={n} act exchange {bits} bit", flush=True)
    st = Stack([300 + 7 * i for i in range(n)], E, fmt)
    x0 = np.random.default_rng(5).normal(0, 1, H).astype(np.float32)
    xd = dev(x0)
    L = D.lib()
    L.dr_step_set_act_exchange(bits)
    try:
        idx, wts, sg, xs = st.run(xd)
    finally:
        L.dr_step_set_act_exchange(0)
    assert int(host(st.sync)[1]) == 0, "step reported a timeout"
    check_stack(st, x0, idx, wts, sg, xs, host(xd))


def test_step_in_band_phase_over_launches_of_any_length():
    """The in-band phase (act exchange 30) counts layers over launches of different lengths on
    one ll / sync pair: one-layer launches (the engine's), then 3, 1, 2 layers; every launch's
    routing and outputs against the oracle on its own input."""
    import torch

    st = Stack([700 + i for i in range(3)], 64, "cfg")
    L = D.lib()
    x0 = np.random.default_rng(9).normal(0, 1, H).astype(np.float32)
    xd = dev(x0)
    L.dr_step_set_act_exchange(30)
    try:
        for call, (first, n) in enumerate([(0, 1), (1, 1), (2, 1), (0, 1), (0, 3), (1, 1), (1, 2), (0, 1)]):
            print(f"in-band phase launch {call}: layers {first}..{first + n - 1}", flush=True)
            xin = host(xd).copy()
            idx = torch.full((n * TOPK,), -1, dtype=torch.int32, device="cuda")
            wts = torch.zeros(n * TOPK, device="cuda")
            sg = torch.zeros(n, device="cuda")
            xs = torch.zeros(n * H, device="cuda")
            L.dr_moe_decode_step_bf16s(D.ptr(st.table) + 80 * first, n, D.ptr(xd), st.E, H, I, TOPK, 1e-6,
                                       D.ptr(st.ll), D.ptr(st.sync), D.ptr(idx), D.ptr(wts), D.ptr(sg), D.ptr(xs),
                                       None, 0, D.stream_ptr())
            torch.cuda.synchronize()
            assert int(host(st.sync)[1]) == 0, "step reported a timeout"

            class Sub:
                h, E = st.h[first:first + n], st.E

            check_stack(Sub, xin, host(idx).reshape(n, TOPK), host(wts).reshape(n, TOPK), host(sg),
                        host(xs).reshape(n, H), host(xd))
        assert int(host(st.sync)[2]) == 11, "running layer count"
    finally:
        L.dr_step_set_act_exchange(0)


def test_step_transport_switch_on_one_ll():
    """Launches on one ll / sync pair that switch the activation transport (fp32 with tags ->
    packed -> fp32 -> packed).  Before each packed launch the packed routed slots are filled with
    junk (1e30) carrying the phase the launch would expect without the transport record in
    sync[3]: the launch must clear them, so every launch still matches the oracle."""
    import torch

    st = Stack([720, 721], 64, "cfg")
    L = D.lib()
    x0 = np.random.default_rng(19).normal(0, 1, H).astype(np.float32)
    xd = dev(x0)
    act_words = slice(264, 264 + 2048)  # LL_ACT: the packed routed slots
    try:
        for call, bits_ in enumerate([32, 30, 32, 30, 30]):
            print(f"transport switch launch {call}: {bits_} bit", flush=True)
            L.dr_step_set_act_exchange(bits_)
            if bits_ == 30 and call in (1, 3):
                t2 = (int(host(st.sync)[2]) + 1) & 3
                half = (np.float32(1e30).view(np.uint32) & ~np.uint32(3)) | np.uint32(t2)
                junk = (np.uint64(half) << np.uint64(32)) | np.uint64(half)
                st.ll[act_words] = torch.tensor(np.full(2048, junk, np.uint64).view(np.int64), device="cuda")
                torch.cuda.synchronize()
            xin = host(xd).copy()
            idx, wts, sg, xs = st.run(xd)
            assert int(host(st.sync)[1]) == 0, "step reported a timeout"
            assert int(host(st.sync)[3]) == (2 if bits_ == 32 else 1), "transport record"
            check_stack(st, xin, idx, wts, sg, xs, host(xd))
    finally:
        L.dr_step_set_act_exchange(0)


@pytest.mark.parametrize("fmt,E,n,bits", [("cfg", 32, 3, 32), ("ref", 16, 2, 32), ("cfg", 8, 2, 32), ("cfg", 16, 1, 32),
                                          ("cfg", 32, 2, 30)])
def test_step_fp8_matches_oracle_layer_by_layer(fmt, E, n, bits):
    """Block-FP8 routed experts (dr_moe_decode_step_fp8*): the same routing and layer bar."""
    print(f"fp8 step parity fmt={fmt} E={E} layers={n} act exchange {bits} bit", flush=True)
    st = Stack([500 + 3 * i for i in range(n)], E, fmt, kind="fp8")
    x0 = np.random.default_rng(15).normal(0, 1, H).astype(np.float32)
    xd = dev(x0)
    L = D.lib()
    L.dr_step_set_act_exchange(bits)
    try:
        idx, wts, sg, xs = st.run(xd)
    finally:
        L.dr_step_set_act_exchange(0)
    assert int(host(st.sync)[1]) == 0, "step reported a timeout"
    check_stack(st, x0, idx, wts, sg, xs, host(xd))


def test_step_tied_logits_pick_lowest_experts_first():
    """Copies of the top expert's router row in other 64-expert groups and next to it give
    exactly equal logits: the picks must come in (logit desc, expert asc) order, as the oracle's."""
    st = Stack([91, 92], 256, "cfg")
    x0 = np.random.default_rng(9).normal(0, 1, H).astype(np.float32)
    L0 = st.h[0]
    lg, ri, _, _ = O.router_topk(L0["router"], x0, L0["nw"], 1e-6, 256, TOPK)
    top, second = int(ri[0]), int(ri[1])
    for L, d in zip(st.h, st.d):
        for dst in {(top + 1) % 256, (top + 64) % 256, (top + 130) % 256, (second + 200) % 256} - {top, second}:
            L["router"][dst] = L["router"][top]
        d["router"].copy_(dev(L["router"]))
    _, ri2, _, _ = O.router_topk(L0["router"], x0, L0["nw"], 1e-6, 256, TOPK)
    assert len(set(ri2[:4].tolist())) == 4 and top in ri2[:4].tolist()
    xd = dev(x0)
    r = st.run(xd)
    check_stack(st, x0, *r, host(xd))


def test_step_repeats_and_matches_first_call_bits():
    """Consecutive calls reuse ll/sync (the epoch advances); the same input gives the same
    bits, and a call continuing from the previous output is again oracle-exact in routing."""
    st = Stack([41, 42], 64, "cfg")
    x0 = np.random.default_rng(6).normal(0, 1, H).astype(np.float32)
    xa, xb = dev(x0), dev(x0)
    r1 = st.run(xa)
    r2 = st.run(xb)
    for a, b in zip(r1, r2):
        np.testing.assert_array_equal(np.ascontiguousarray(a).view(np.uint8), np.ascontiguousarray(b).view(np.uint8))
    x1 = host(xa).copy()
    r3 = st.run(xa)
    check_stack(st, x1, *r3, host(xa))
    s = host(st.sync)
    assert s[0] == 3 and s[1] == 0


@pytest.mark.parametrize("kind", ["q4", "fp8"])
def test_step_without_norm_and_without_outputs(kind):
    # without the norm the activations grow with |x| (N(0,1) inputs give layer outputs of
    # 1e4 whose small elements are differences of 1e4-sized sums, beyond any fp32 tolerance
    # relative to the element); inputs of scale 0.05 keep the comparison meaningful
    st = Stack([77, 78], 32, "cfg", with_norm=False, kind=kind)
    x0 = (0.05 * np.random.default_rng(8).normal(0, 1, H)).astype(np.float32)
    xa, xb = dev(x0), dev(x0)
    r = st.run(xa)
    check_stack(st, x0, *r, host(xa))
    st.run(xb, want_outputs=False)  # optional outputs off: same final bits
    np.testing.assert_array_equal(bits(host(xb)), bits(host(xa)))


def test_step_rejects_bad_shapes():
    assert D.lib().raw("dr_step_set_act_exchange")(16) == -1
    assert D.lib().raw("dr_step_set_act_exchange")(24) == -1
    st = Stack([1], 16, "cfg")
    x = dev(np.zeros(H, np.float32))
    L = D.lib()
    base = [D.ptr(st.table), 1, D.ptr(x), 16, H, I, TOPK, 1e-6, D.ptr(st.ll), D.ptr(st.sync), None, None, None, None,
            None, 0, D.stream_ptr()]
    for pos, bad in ((4, 1024), (5, 256), (6, 4), (3, 257), (3, 4), (1, 0), (1, 2000)):
        a = list(base)
        a[pos] = bad
        assert L.raw("dr_moe_decode_step_bf16s")(*a) == -1


def test_step_graph_replays_match_eager():
    """One captured launch replayed several times, with eager work and synchronisations in
    between: every replay must give the eager call's bits (the step only reads its own slots'
    tags, so replays need no reset)."""
    import ctypes

    import torch

    st = Stack([61, 62], 64, "cfg")
    x0 = np.random.default_rng(9).normal(0, 1, H).astype(np.float32)
    ref = dev(x0)
    st.run(ref)
    want = host(ref).copy()
    L = D.lib()
    s = torch.cuda.Stream()
    xg = torch.zeros(H, device="cuda")
    sp = s.cuda_stream
    g = ctypes.c_void_p()
    L.dr_graph_begin(sp)
    L.dr_moe_decode_step_bf16s(D.ptr(st.table), 2, D.ptr(xg), 64, H, I, TOPK, 1e-6, D.ptr(st.ll), D.ptr(st.sync),
                               None, None, None, None, None, 0, sp)
    L.dr_graph_end(sp, ctypes.byref(g))
    try:
        for rep in range(4):
            xg.copy_(torch.from_numpy(x0).cuda())
            torch.cuda.synchronize()
            L.dr_graph_launch(g, sp)
            s.synchronize()
            np.testing.assert_array_equal(bits(host(xg)), bits(want), err_msg=f"replay {rep}")
            st.run(dev(x0))  # eager call in between advances the same epoch counter
        assert int(host(st.sync)[1]) == 0
    finally:
        L.dr_graph_destroy(g)


def _clear_library_error():
    L = D.lib()
    L.raw("dr_last_error")()


def test_step_gives_up_loudly_when_a_previous_call_timed_out():
    """sync[1] set (what a timed-out call leaves behind) and not reset: the call must poison x
    with NaN and raise DR_ERR_STEP_TIMEOUT; dr_stream_sync reports it, the launchers refuse to
    start until dr_last_error has returned and cleared it, and after the caller zeroes sync and
    ll the step is oracle-exact again."""
    import torch

    L = D.lib()
    st = Stack([81, 82], 64, "cfg")
    x0 = np.random.default_rng(12).normal(0, 1, H).astype(np.float32)
    _clear_library_error()
    try:
        st.sync[1] = 1
        xd = dev(x0)
        args = [D.ptr(st.table), 2, D.ptr(xd), 64, H, I, TOPK, 1e-6, D.ptr(st.ll), D.ptr(st.sync), None, None, None,
                None, None, 0, D.stream_ptr()]
        assert L.raw("dr_moe_decode_step_bf16s")(*args) == 0
        assert L.raw("dr_stream_sync")(D.stream_ptr()) == 9001
        assert np.isnan(host(xd)).all(), "a call that gave up must leave x all NaN"
        assert L.raw("dr_moe_decode_step_bf16s")(*args) == 9001, "launcher must refuse while the error is pending"
        assert L.raw("dr_last_error")() == 9001
        assert L.raw("dr_last_error")() == 0, "dr_last_error clears the library error"
        st.sync.zero_()
        st.ll.zero_()
        torch.cuda.synchronize()
        xd = dev(x0)
        r = st.run(xd)
        assert L.raw("dr_stream_sync")(D.stream_ptr()) == 0
        check_stack(st, x0, *r, host(xd))
    finally:
        _clear_library_error()


def _busy_stream_step(limit_us):
    """The fused step launched while 40 4096^3 bf16 matrix products queued on a second stream
    hold CUs, so the step's 256 workgroups may not all be resident at once.  Returns the
    dr_stream_sync code, the stack, x0 and the step's outputs."""
    import torch

    L = D.lib()
    st = Stack([83, 84], 64, "cfg")
    x0 = np.random.default_rng(13).normal(0, 1, H).astype(np.float32)
    a = torch.randn(4096, 4096, device="cuda", dtype=torch.bfloat16)
    xd = dev(x0)
    torch.cuda.synchronize()
    _clear_library_error()
    side = torch.cuda.Stream()
    try:
        if limit_us:
            L.dr_step_set_wait_limit(limit_us)
        with torch.cuda.stream(side):
            for _ in range(40):
                a = (a @ a) * 1e-3
        idx = torch.full((2 * TOPK,), -1, dtype=torch.int32, device="cuda")
        wts = torch.zeros(2 * TOPK, device="cuda")
        sg = torch.zeros(2, device="cuda")
        xs = torch.zeros(2 * H, device="cuda")
        main = torch.cuda.current_stream()
        rc = L.raw("dr_moe_decode_step_bf16s")(D.ptr(st.table), 2, D.ptr(xd), 64, H, I, TOPK, 1e-6, D.ptr(st.ll),
                                               D.ptr(st.sync), D.ptr(idx), D.ptr(wts), D.ptr(sg), D.ptr(xs),
                                               None, 0, main.cuda_stream)
        assert rc == 0
        code = L.raw("dr_stream_sync")(main.cuda_stream)
        side.synchronize()
        out = (host(idx).reshape(2, TOPK), host(wts).reshape(2, TOPK), host(sg), host(xs).reshape(2, H), host(xd))
        return code, st, x0, out
    finally:
        L.dr_step_set_wait_limit(0)
        torch.cuda.synchronize()
        _clear_library_error()


def test_step_beside_a_busy_stream_completes_within_the_default_limit():
    """With the default wait limit (0.2 s) the step's workgroups that could not start beside the
    matrix products start as those drain (a few ms of work), so the step completes and gives the
    oracle's bits: a concurrent workload that finishes within the limit only delays it."""
    code, st, x0, (idx, wts, sg, xs, xf) = _busy_stream_step(0)
    assert code == 0, f"step gave up beside a finite concurrent workload (code {code})"
    assert int(host(st.sync)[1]) == 0
    check_stack(st, x0, idx, wts, sg, xs, xf)


def test_step_beside_a_busy_stream_is_correct_or_reports(record_property):
    """With a 2 ms wait limit, shorter than the concurrent work, the step either completed (its
    workgroups happened to be resident together) and gives the oracle's bits, or it reports
    DR_ERR_STEP_TIMEOUT with sync[1] set and x holding NaN; which of the two happened is recorded
    (the test property "outcome" and a warning on give-up).  Every kernel exits by itself."""
    import warnings

    code, st, x0, (idx, wts, sg, xs, xf) = _busy_stream_step(2000)
    if code == 0:
        record_property("outcome", "completed")
        print("step ran beside the busy stream and completed", flush=True)
        check_stack(st, x0, idx, wts, sg, xs, xf)
    else:
        record_property("outcome", "gave up (DR_ERR_STEP_TIMEOUT)")
        warnings.warn("fused step beside a busy stream with a 2 ms wait limit gave up and reported "
                      "DR_ERR_STEP_TIMEOUT (x poisoned with NaN)")
        assert code == 9001
        assert int(host(st.sync)[1]) == 1 and np.isnan(xf).any()


def test_step_prefetch_range_changes_nothing():
    """pf / pf_bytes (the next op's weights, warmed after the last layer) leave every result bit
    unchanged, for ranges of odd sizes and one larger than the grid's share per thread."""
    import torch

    st = Stack([61, 62], 64, "cfg")
    x0 = np.random.default_rng(21).normal(0, 1, H).astype(np.float32)
    want = host(dev(x0))
    xa = dev(x0)
    st.run(xa)
    want = host(xa)
    for nbytes in (1, 1000, 4 << 20, (40 << 20) + 12345):
        buf = torch.randint(0, 255, (nbytes,), dtype=torch.uint8, device="cuda")
        st.sync.zero_()
        st.ll.zero_()
        xb = dev(x0)
        torch.cuda.synchronize()
        assert D.lib().raw("dr_moe_decode_step_bf16s")(D.ptr(st.table), 2, D.ptr(xb), 64, H, I, TOPK, 1e-6,
                                                       D.ptr(st.ll), D.ptr(st.sync), None, None, None, None,
                                                       D.ptr(buf), nbytes, D.stream_ptr()) == 0
        torch.cuda.synchronize()
        assert int(host(st.sync)[1]) == 0
        np.testing.assert_array_equal(bits(host(xb)), bits(want), err_msg=f"pf_bytes {nbytes}")
