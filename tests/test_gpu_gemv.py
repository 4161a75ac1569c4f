"""GPU parity of the dense decode GEMVs (kernels/drama.cu:216-315) and the int8 lm_head of
benchmark configuration 5, against the oracle's dequant-then-fp64 dot (tolerance
|gpu - ref| <= 1e-3 + 1e-3 |ref|)."""
import numpy as np
import pytest

import dramamoe as D
import oracle as O
import synth
from helpers import assert_close, dev, host

pytestmark = pytest.mark.gpu


def q8_case(seed, N, K, fmt):
    rng = np.random.default_rng(seed)
    q, s, kind, group = synth.q8_dense(rng, N, K, fmt)
    x = rng.normal(0, 1, K).astype(np.float32)
    nw = (1 + rng.normal(0, 0.1, K)).astype(np.float32)
    res = rng.normal(0, 1, N).astype(np.float32)
    return q, s, kind, group, x, nw, res


def xn_of(x, nw):
    return O.rmsnorm(x, nw, 1e-6) if nw is not None else x


@pytest.mark.parametrize("K,N", [(512, 1000), (2048, 1000), (4096, 1000), (6144, 1000), (1024, 17001), (2048, 20003)])
@pytest.mark.parametrize("with_norm", [True, False])
def test_gemv_q8(K, N, with_norm):
    """Above 16384 rows the K = 1024 / 2048 forms walk row tiles with a grid of 2 blocks per CU."""
    import torch

    q, s, kind, group, x, nw, res = q8_case(K, N, K, "ref")
    nw = nw if with_norm else None
    ref = O.gemv_q8(q, s, kind, group, xn_of(x, nw), N, K) + res
    dq, ds, dx, dnw, dres = dev(q), dev(s), dev(x), dev(nw) if nw is not None else None, dev(res)
    y = torch.empty(N, device="cuda")
    D.lib().dr_gemv_q8(D.ptr(dq), D.ptr(ds), D.ptr(dx), D.ptr(dres), D.ptr(y), N, K, D.ptr(dnw), 1e-6, None, 0,
                       D.stream_ptr())
    torch.cuda.synchronize()
    assert_close(host(y), ref, what=f"gemv_q8 K={K}")


def test_gemv_q8_alias_res_and_y():
    import torch

    N, K = 2048, 2048
    q, s, kind, group, x, nw, res = q8_case(9, N, K, "ref")
    ref = O.gemv_q8(q, s, kind, group, xn_of(x, nw), N, K) + res
    dq, ds, dx, dnw, buf = dev(q), dev(s), dev(x), dev(nw), dev(res)
    D.lib().dr_gemv_q8(D.ptr(dq), D.ptr(ds), D.ptr(dx), D.ptr(buf), D.ptr(buf), N, K, D.ptr(dnw), 1e-6, None, 0,
                       D.stream_ptr())
    torch.cuda.synchronize()
    assert_close(host(buf), ref, what="gemv_q8 y aliasing res")


@pytest.mark.parametrize("K", [2048, 4096])
def test_gemv_q8_swiglu(K):
    import torch

    Ih = 768
    q, s, kind, group, x, nw, _ = q8_case(K + 1, 2 * Ih, K, "ref")
    h = O.gemv_q8(q, s, kind, group, xn_of(x, nw), 2 * Ih, K).astype(np.float64)
    ref = h[:Ih] / (1 + np.exp(-h[:Ih])) * h[Ih:]
    dq, ds, dx, dnw = dev(q), dev(s), dev(x), dev(nw)
    y = torch.empty(Ih, device="cuda")
    D.lib().dr_gemv_q8_swiglu(D.ptr(dq), D.ptr(ds), D.ptr(dx), D.ptr(y), Ih, K, D.ptr(dnw), 1e-6, None, 0,
                              D.stream_ptr())
    torch.cuda.synchronize()
    assert_close(host(y), ref, what="gemv_q8_swiglu")


@pytest.mark.parametrize("N,K", [(151936, 2048), (2048, 2048), (37, 512)])
def test_gemv_q8_per_row_bf16(N, K):
    """int8 lm_head / projection with one bf16 scale per row (configuration 5)."""
    import torch

    q, s, kind, group, x, _, _ = q8_case(N, N, K, "cfg")
    ref = O.gemv_q8(q, s, kind, group, x, N, K)
    dq, ds, dx = dev(q), dev(s), dev(x)
    y = torch.empty(N, device="cuda")
    D.lib().dr_gemv_q8_bf16s(D.ptr(dq), D.ptr(ds), D.ptr(dx), None, D.ptr(y), N, K, None, 0.0, D.stream_ptr())
    torch.cuda.synchronize()
    assert_close(host(y), ref, what=f"gemv_q8_bf16s {N}x{K}")


@pytest.mark.parametrize("K", [2048, 4096])
def test_gemv_bf16(K):
    import torch

    N = 4097
    rng = np.random.default_rng(K)
    W = synth.f32_to_bf16(rng.normal(0, 0.02, (N, K)).astype(np.float32))
    x = rng.normal(0, 1, K).astype(np.float32)
    nw = (1 + rng.normal(0, 0.1, K)).astype(np.float32)
    ref = synth.bf16_to_f32(W).astype(np.float64) @ O.rmsnorm(x, nw, 1e-6).astype(np.float64)
    dW, dx, dnw = dev(W), dev(x), dev(nw)
    y = torch.empty(N, device="cuda")
    D.lib().dr_gemv_bf16(D.ptr(dW), D.ptr(dx), D.ptr(y), N, K, D.ptr(dnw), 1e-6, None, 0, D.stream_ptr())
    torch.cuda.synchronize()
    assert_close(host(y), ref, what="gemv_bf16")


def test_gemv_rejects_bad_shapes():
    L = D.lib()
    assert L.raw("dr_gemv_q8")(None, None, None, None, None, 10, 3000, None, 0.0, None, 0, None) == -1
    assert L.raw("dr_gemv_bf16")(None, None, None, 10, 1000, None, 0.0, None, 0, None) == -1
