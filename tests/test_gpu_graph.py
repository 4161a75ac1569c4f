"""The prefill layer (router GEMM, top-k, grouping, gather, grouped expert GEMMs, shared expert,
combine; at 300 rows the shared expert on a second stream joined by events) captured into one
HIP graph and replayed several times with eager work and synchronisations in between: every
replay must give the eager call's bits."""
import ctypes

import numpy as np
import pytest

import dramamoe as D
from helpers import bits, host

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("rows", [300, 4])
def test_prefill_graph_replays_match_eager(rows):
    import torch

    import bench
    import benchcfg

    lib = D.lib()
    st = torch.cuda.Stream()
    L = bench.make_layer_gpu(None, 3)
    pf = benchcfg.Prefill(rows, st)
    assert pf.overlap == (rows >= 64)

    def layer():
        pf.shared_begin(lib, L)
        pf.router(lib, L)
        pf.experts(lib, L, shared_started=True)

    x0 = pf.x.clone()
    torch.cuda.synchronize()
    layer()
    st.synchronize()
    want = host(pf.x).copy()
    assert np.isfinite(want).all() and not np.array_equal(want, host(x0))
    g = ctypes.c_void_p()
    torch.cuda.synchronize()
    lib.dr_graph_begin(st.cuda_stream)
    layer()
    assert lib.dr_graph_end(st.cuda_stream, ctypes.byref(g)) == 0
    try:
        for rep in range(3):
            pf.x.copy_(x0)
            torch.cuda.synchronize()
            lib.dr_graph_launch(g, st.cuda_stream)
            st.synchronize()
            np.testing.assert_array_equal(bits(host(pf.x)), bits(want), err_msg=f"replay {rep}")
            pf.x.copy_(x0)  # eager call in between on the same buffers
            torch.cuda.synchronize()
            layer()
            st.synchronize()
            np.testing.assert_array_equal(bits(host(pf.x)), bits(want), err_msg=f"eager after replay {rep}")
    finally:
        lib.dr_graph_destroy(g)
