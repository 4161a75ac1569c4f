"""GPU parity of the router path through the C ABI: logits, softmax probabilities, selected
experts, weights and the shared gate must equal the oracle bit for bit."""
import numpy as np
import pytest

import dramamoe as D
import oracle as O
import synth
from helpers import bits, dev, host

pytestmark = pytest.mark.gpu


def _router_case(seed, E, nw_on, K=2048, scale=0.02):
    rng = np.random.default_rng(seed)
    W = synth.f32_to_bf16(rng.normal(0, scale, (E + 1, K)).astype(np.float32))
    x = rng.normal(0, 1, K).astype(np.float32)
    nw = (1 + rng.normal(0, 0.1, K)).astype(np.float32) if nw_on else None
    return W, x, nw


@pytest.mark.parametrize("seed,E,nw_on", [(0, 256, True), (1, 256, False), (2, 64, True), (3, 8, True), (4, 255, True)])
def test_router_topk_bit_exact(seed, E, nw_on):
    import torch

    L = D.lib()
    W, x, nw = _router_case(seed, E, nw_on)
    rl, ri, rw, rs = O.router_topk(W, x, nw, 1e-6, E, 8)
    dW, dx = dev(W), dev(x)
    dnw = dev(nw) if nw is not None else None
    logits = torch.empty(E + 1, dtype=torch.float32, device="cuda")
    idx = torch.empty(8, dtype=torch.int32, device="cuda")
    wts = torch.empty(8, dtype=torch.float32, device="cuda")
    sg = torch.empty(1, dtype=torch.float32, device="cuda")
    counter = torch.zeros(4, dtype=torch.int32, device="cuda")
    for rep in range(3):  # the counter must return to zero so calls can repeat
        L.dr_router_topk(D.ptr(dW), D.ptr(dx), D.ptr(dnw), 1e-6, D.ptr(logits), E, 8, 2048, D.ptr(idx), D.ptr(wts),
                         D.ptr(sg), D.ptr(counter), None, None, None, None, 0, 0, 0, 0, D.stream_ptr())
        torch.cuda.synchronize()
        np.testing.assert_array_equal(bits(host(logits)), bits(rl), err_msg="logits")
        np.testing.assert_array_equal(host(idx), ri)
        np.testing.assert_array_equal(bits(host(wts)), bits(rw), err_msg="wts")
        assert bits(host(sg))[0] == bits(np.float32(rs))
        assert int(host(counter)[0]) == 0


def test_router_topk_many_seeds_and_margins():
    """40 seeds at the real shape; reports the 8th/9th probability margin of each."""
    import torch

    L = D.lib()
    E = 256
    logits = torch.empty(E + 1, dtype=torch.float32, device="cuda")
    idx = torch.empty(8, dtype=torch.int32, device="cuda")
    wts = torch.empty(8, dtype=torch.float32, device="cuda")
    sg = torch.empty(1, dtype=torch.float32, device="cuda")
    counter = torch.zeros(4, dtype=torch.int32, device="cuda")
    margins = []
    for seed in range(100, 140):
        W, x, nw = _router_case(seed, E, True)
        rl, ri, rw, rs = O.router_topk(W, x, nw, 1e-6, E, 8)
        dW, dx, dnw = dev(W), dev(x), dev(nw)
        L.dr_router_topk(D.ptr(dW), D.ptr(dx), D.ptr(dnw), 1e-6, D.ptr(logits), E, 8, 2048, D.ptr(idx),
                         D.ptr(wts), D.ptr(sg), D.ptr(counter), None, None, None, None, 0, 0, 0, 0, D.stream_ptr())
        torch.cuda.synchronize()
        np.testing.assert_array_equal(bits(host(logits)), bits(rl))
        np.testing.assert_array_equal(host(idx), ri)
        np.testing.assert_array_equal(bits(host(wts)), bits(rw))
        p = np.sort(rl[:E])[::-1]
        margins.append(float(p[7] - p[8]))
    print(f"min logit margin between 8th and 9th expert over 40 seeds: {min(margins):.3e}")


def test_router_rejects_bad_shapes():
    L = D.lib()
    rc = L.raw("dr_router_topk")(None, None, None, 0.0, None, 257, 8, 2048, None, None, None, None, None, None, None,
                                 None, 0, 0, 0, 0, None)
    assert rc == -1
    assert L.raw("dr_router_topk")(None, None, None, 0.0, None, 256, 8, 1024, None, None, None, None, None, None,
                                   None, None, 0, 0, 0, 0, None) == -1
    assert L.raw("dr_moe_topk")(None, 4, 300, 8, 301, None, None, None, None) == -1


@pytest.mark.parametrize("rows,E,stride,ties", [(300, 256, 257, False), (7, 16, 20, False), (64, 256, 257, True)])
def test_moe_topk_rows_bit_exact(rows, E, stride, ties):
    import torch

    rng = np.random.default_rng(rows + E)
    lg = rng.normal(0, 1, (rows, stride)).astype(np.float32)
    if ties:
        lg = (np.round(lg * 4) / 4).astype(np.float32)
    ri, rw, rs = O.moe_topk(lg, rows, E, 8, stride)
    idx = torch.empty(rows * 8, dtype=torch.int32, device="cuda")
    wts = torch.empty(rows * 8, dtype=torch.float32, device="cuda")
    sg = torch.empty(rows, dtype=torch.float32, device="cuda")
    dlg = dev(lg)
    D.lib().dr_moe_topk(D.ptr(dlg), rows, E, 8, stride, D.ptr(idx), D.ptr(wts), D.ptr(sg), D.stream_ptr())
    torch.cuda.synchronize()
    np.testing.assert_array_equal(host(idx), ri)
    np.testing.assert_array_equal(bits(host(wts)), bits(rw))
    np.testing.assert_array_equal(bits(host(sg)), bits(rs))


def test_moe_topk_special_values():
    """Prefill top-k on logits holding signed zeros, infinities and NaNs (-0 just below +0,
    NaN last, lowest index on ties): indices bit-exact with the oracle; weights and shared
    gates bit-exact where the oracle's are finite, NaN where its are NaN."""
    import torch

    rows, E, stride = 6, 64, 65
    rng = np.random.default_rng(11)
    lg = rng.normal(0, 1, (rows, stride)).astype(np.float32)
    lg[0, :] = -1.0
    lg[0, [3, 9, 17, 30]] = 0.0
    lg[0, [5, 12, 40, 41, 60]] = -0.0  # the 8th pick falls among the -0s: lowest indices win
    lg[1, [2, 7]] = np.inf
    lg[2, :E:3] = np.nan
    lg[3, :] = -np.inf
    lg[3, [4, 44]] = 1.0
    lg[4, : E - 4] = np.nan  # fewer than 8 ordered values
    lg[5, :] = 0.5  # all equal
    lg[:, E] = rng.normal(0, 1, rows).astype(np.float32)  # shared gate logit
    lg[1, E] = -np.inf
    ri, rw, rs = O.moe_topk(lg, rows, E, 8, stride)
    idx = torch.empty(rows * 8, dtype=torch.int32, device="cuda")
    wts = torch.empty(rows * 8, dtype=torch.float32, device="cuda")
    sg = torch.empty(rows, dtype=torch.float32, device="cuda")
    dlg = dev(lg)  # kept alive until the kernel has run
    D.lib().dr_moe_topk(D.ptr(dlg), rows, E, 8, stride, D.ptr(idx), D.ptr(wts), D.ptr(sg), D.stream_ptr())
    torch.cuda.synchronize()
    hi, hw, hs = host(idx), host(wts), host(sg)
    np.testing.assert_array_equal(hi, ri)
    assert ((hi >= 0) & (hi < E)).all()
    for got, ref in ((hw, rw), (hs, rs)):
        fin = np.isfinite(ref)
        np.testing.assert_array_equal(bits(got[fin]), bits(ref[fin]))
        np.testing.assert_array_equal(np.isnan(got[~fin]), np.isnan(ref[~fin]))


@pytest.mark.parametrize("M,N,K", [(300, 257, 2048), (5, 33, 512), (17, 64, 4096), (1, 1, 8), (4, 257, 2048), (16, 257, 2048),
                                   (8, 100, 4096)])
def test_gemm_canonical_bit_exact(M, N, K):
    import torch

    rng = np.random.default_rng(M * N)
    A = synth.f32_to_bf16(rng.normal(0, 1, (M, K)).astype(np.float32))
    Wt = synth.f32_to_bf16(rng.normal(0, 0.02, (N, K)).astype(np.float32))
    ref = O.router_logits_rows(A, Wt, M, N, K)
    C = torch.empty(M * N, dtype=torch.float32, device="cuda")
    h = np.zeros(1, np.uint64)
    L = D.lib()
    L.dr_cublas_create(h.ctypes.data, D.stream_ptr())
    dA, dWt = dev(A), dev(Wt)
    L.dr_gemm(int(h[0]), D.ptr(dA), D.ptr(dWt), D.ptr(C), M, N, K, 0.0)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(bits(host(C)).reshape(M, N), bits(ref))


def test_router_nan_input_selects_valid_experts():
    """A NaN in x makes every probability NaN; the selected experts must still be distinct
    and below E (the decode kernels index expert weights with them)."""
    import torch

    E = 256
    W, x, nw = _router_case(7, E, True)
    x[5] = np.nan
    rl, ri, rw, rs = O.router_topk(W, x, nw, 1e-6, E, 8)
    dW, dx, dnw = dev(W), dev(x), dev(nw)
    logits = torch.empty(E + 1, dtype=torch.float32, device="cuda")
    idx = torch.full((8,), -7, dtype=torch.int32, device="cuda")
    wts = torch.empty(8, dtype=torch.float32, device="cuda")
    sg = torch.empty(1, dtype=torch.float32, device="cuda")
    counter = torch.zeros(4, dtype=torch.int32, device="cuda")
    D.lib().dr_router_topk(D.ptr(dW), D.ptr(dx), D.ptr(dnw), 1e-6, D.ptr(logits), E, 8, 2048, D.ptr(idx), D.ptr(wts),
                           D.ptr(sg), D.ptr(counter), None, None, None, None, 0, 0, 0, 0, D.stream_ptr())
    torch.cuda.synchronize()
    gi = host(idx)
    assert len(set(gi.tolist())) == 8 and gi.min() >= 0 and gi.max() < E
    np.testing.assert_array_equal(gi, ri)
