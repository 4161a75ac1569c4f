"""A synthetic drama-rs-v1 checkpoint loaded by checkpoint.MoeStack and run through the fused
step and the per-layer chain: routing bit-exact with the oracle on each layer's input, outputs
within 1e-3 + 1e-3 |ref|, and the two paths route identically."""
import numpy as np
import pytest

import checkpoint as C
import oracle as O
from ckpt_helpers import write_checkpoint
from helpers import assert_close, bits, dev, host

pytestmark = pytest.mark.gpu


def test_checkpoint_stack_step_and_chain(tmp_path):
    import torch

    E, H, I = 64, 2048, 512
    layers = write_checkpoint(tmp_path, [90, 91, 92], E=E)
    st = C.MoeStack(str(tmp_path))
    x0 = np.random.default_rng(3).normal(0, 1, H).astype(np.float32)
    n = len(layers)
    idx = torch.zeros(n * 8, dtype=torch.int32, device="cuda")
    wts = torch.zeros(n * 8, device="cuda")
    xs = torch.zeros(n * H, device="cuda")
    xd = dev(x0)
    st.step(xd, idx_out=idx, wts_out=wts, xs_out=xs)
    torch.cuda.synchronize()
    gi, gw, gx = host(idx).reshape(n, 8), host(wts).reshape(n, 8), host(xs).reshape(n, H)
    xin = x0
    for l, L in enumerate(layers):
        _, ri, rw, rs = O.router_topk(L["router"], xin, L["nw"], 1e-6, E, 8)
        np.testing.assert_array_equal(gi[l], ri)
        np.testing.assert_array_equal(bits(gw[l]), bits(rw))
        _, ry = O.moe_decode(L, xin, ri, rw, rs, xin, H, I, 8, nw=L["nw"], eps=1e-6)
        assert_close(gx[l], ry, what=f"layer {l}")
        xin = gx[l].copy()
    xc = dev(x0)
    st.chain(xc)
    torch.cuda.synchronize()
    assert_close(host(xc), gx[-1], what="chain vs fused step")


def test_checkpoint_prefill_chunked(tmp_path):
    """MoeStack.prefill over 300 rows: routing bit-exact with the oracle, and chunking (3 chunks
    of 128 rows) gives the same bits as one 300-row call (rows are independent), also with the
    shared expert overlapped on a second stream."""
    import torch

    import synth

    E, H, rows = 256, 2048, 300
    layers = write_checkpoint(tmp_path, [95], E=E)
    st = C.MoeStack(str(tmp_path))
    rng = np.random.default_rng(4)
    hn = synth.f32_to_bf16(rng.normal(0, 1, (rows, H)).astype(np.float32))
    x0 = rng.normal(0, 1, (rows, H)).astype(np.float32)
    dhn = dev(hn)
    xa, xb = dev(x0), dev(x0)
    kept = {}
    st.prefill(0, xa.view(rows, H), dhn.view(rows, H), keep=kept)
    st.prefill(0, xb.view(rows, H), dhn.view(rows, H), chunk=128)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(bits(host(xa)), bits(host(xb)))
    # from a created stream the shared expert runs on a second stream beside the routed path
    xc = dev(x0)
    torch.cuda.synchronize()
    s = torch.cuda.Stream()
    with torch.cuda.stream(s):
        st.prefill(0, xc.view(rows, H), dhn.view(rows, H), chunk=128)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(bits(host(xa)), bits(host(xc)))
    # the tile-step copy of the experts (pack_prefill): the same bits
    sp = C.MoeStack(str(tmp_path), pack_prefill=True)
    xd = dev(x0)
    sp.prefill(0, xd.view(rows, H), dhn.view(rows, H), chunk=128)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(bits(host(xa)), bits(host(xd)))
    L = layers[0]
    rl = O.router_logits_rows(hn, L["router"], rows, E + 1, H)
    ri, rw, rs = O.moe_topk(rl, rows, E, 8, E + 1)
    _check_prefill(L, hn, x0, host(xa), kept, ri, rw, rs)


def _check_prefill(L, hn, x0, got, kept, ri, rw, rs):
    """Routing of the stack's prefill bit for bit with the oracle's, the layer output within
    1e-3 + 1e-3 |ref| plus the propagation of the bf16 act rounding flips observed (the bar
    of the other prefill layer tests)."""
    from test_gpu_configs import check_layer_with_flips

    np.testing.assert_array_equal(host(kept["idx"]), ri)
    np.testing.assert_array_equal(bits(host(kept["wts"])), bits(rw))
    np.testing.assert_array_equal(bits(host(kept["sgate"])), bits(rs))
    E = L["gu_q"].shape[0]
    np.testing.assert_array_equal(host(kept["slot_of"]), O.moe_group(ri, E)[2])
    rows = hn.shape[0]
    act = host(kept["act"]).view(np.uint16).reshape(-1, L["I"])
    sact = host(kept["sact"]).view(np.uint16).reshape(rows, L["I"])
    check_layer_with_flips(L, hn, x0, act, sact, got, ri, rw, rs)


def test_checkpoint_fp8_source_step_chain_prefill(tmp_path):
    """Routed experts from the original block-FP8 checkpoint (Fp8Source) beside the converted
    router/shared tensors: layer 0 on the GPU, layer 1 in pinned host memory read over PCIe
    (vram_layers=1).  Fused step: routing bit-exact with the oracle per layer, outputs within
    1e-3 + 1e-3 |ref|; the per-layer chain agrees with the step; prefill runs the FP8
    grouped kernels."""
    import torch

    import synth
    from ckpt_helpers import write_fp8_source

    E, H, I = 16, 2048, 512
    conv = tmp_path / "conv"
    src = tmp_path / "fp8"
    conv.mkdir()
    src.mkdir()
    layers = write_checkpoint(conv, [70, 71], E=E)
    fp8 = [synth.make_layer(80 + i, E=E, fmt="ref", kind="fp8", quick=True) for i in range(2)]
    write_fp8_source(str(src), fp8, E)
    st = C.MoeStack(str(conv), fp8_dir=str(src), vram_layers=1)
    assert st.layers[0]["gu_q"].is_cuda and not st.layers[1]["gu_q"].is_cuda and st.layers[1]["gu_q"].is_pinned()
    oracle_layers = []
    for L, F in zip(layers, fp8):
        M = dict(L)
        M.update({k: F[k] for k in ("kind", "gu_q", "gu_s", "d_q", "d_s", "sc_kind")})
        oracle_layers.append(M)
    n = 2
    x0 = np.random.default_rng(7).normal(0, 1, H).astype(np.float32)
    idx = torch.zeros(n * 8, dtype=torch.int32, device="cuda")
    wts = torch.zeros(n * 8, device="cuda")
    xs = torch.zeros(n * H, device="cuda")
    xd = dev(x0)
    st.step(xd, idx_out=idx, wts_out=wts, xs_out=xs)
    torch.cuda.synchronize()
    gi, gw, gx = host(idx).reshape(n, 8), host(wts).reshape(n, 8), host(xs).reshape(n, H)
    xin = x0
    for l, L in enumerate(oracle_layers):
        _, ri, rw, rs = O.router_topk(L["router"], xin, L["nw"], 1e-6, E, 8)
        np.testing.assert_array_equal(gi[l], ri)
        np.testing.assert_array_equal(bits(gw[l]), bits(rw))
        _, ry = O.moe_decode(L, xin, ri, rw, rs, xin, H, I, 8, nw=L["nw"], eps=1e-6)
        assert_close(gx[l], ry, what=f"fp8 layer {l}")
        xin = gx[l].copy()
    xc = dev(x0)
    st.chain(xc)
    torch.cuda.synchronize()
    assert_close(host(xc), gx[-1], what="fp8 chain vs fused step")
    rows = 24
    rng = np.random.default_rng(8)
    hn = synth.f32_to_bf16(rng.normal(0, 1, (rows, H)).astype(np.float32))
    xp0 = rng.normal(0, 1, (rows, H)).astype(np.float32)
    xa, dhn = dev(xp0), dev(hn)
    kept = {}
    st.prefill(0, xa.view(rows, H), dhn.view(rows, H), keep=kept)
    torch.cuda.synchronize()
    L = oracle_layers[0]
    rl = O.router_logits_rows(hn, L["router"], rows, E + 1, H)
    ri, rw, rs = O.moe_topk(rl, rows, E, 8, E + 1)
    _check_prefill(L, hn, xp0, host(xa), kept, ri, rw, rs)
    # pack_prefill: layer 0 (on the GPU) prefills from its tile-step copy, bit for bit the same;
    # layer 1 (host memory) is left unpacked and runs on the reference layout
    sp = C.MoeStack(str(conv), fp8_dir=str(src), vram_layers=1, pack_prefill=True)
    assert sp.packed[0] is not None and sp.packed[1] is None
    for l in (0, 1):
        xr, xq = dev(xp0), dev(xp0)
        st.prefill(l, xr.view(rows, H), dhn.view(rows, H))
        sp.prefill(l, xq.view(rows, H), dhn.view(rows, H))
        torch.cuda.synchronize()
        np.testing.assert_array_equal(bits(host(xq)), bits(host(xr)), err_msg=f"layer {l}")
