"""GPU test of the reference's runtime ABI (src/ffi.rs:13-31, kernels/drama.cu:1995-2044) as
the engine uses it (src/gpu.rs:146-257): allocation, pinned host memory, the three copies, the
fill, streams, memory info, the graph calls and the GEMM handle, each return code checked and
every byte round-tripped."""
import ctypes as C

import numpy as np
import pytest

import dramamoe as D

pytestmark = pytest.mark.gpu


def _rc(rc, what):
    assert rc == 0, f"{what} returned {rc}"


def test_runtime_abi_round_trips():
    L = D.lib()
    raw = L.raw
    n = 1 << 20
    st = C.c_void_p()
    _rc(raw("dr_stream_create")(C.byref(st)), "dr_stream_create")
    assert st.value, "no stream"
    free_b, total_b = C.c_size_t(), C.c_size_t()
    _rc(raw("dr_mem_info")(C.byref(free_b), C.byref(total_b)), "dr_mem_info")
    assert 0 < free_b.value <= total_b.value
    assert total_b.value > 200 << 30, "an MI355X holds 288 GB"
    d1, d2 = C.c_void_p(), C.c_void_p()
    _rc(raw("dr_malloc")(C.byref(d1), C.c_size_t(n)), "dr_malloc")
    _rc(raw("dr_malloc")(C.byref(d2), C.c_size_t(n)), "dr_malloc")
    h1, h2 = C.c_void_p(), C.c_void_p()
    _rc(raw("dr_host_alloc")(C.byref(h1), C.c_size_t(n)), "dr_host_alloc")
    _rc(raw("dr_host_alloc")(C.byref(h2), C.c_size_t(n)), "dr_host_alloc")
    try:
        src = np.frombuffer(np.random.default_rng(1).bytes(n), np.uint8)
        C.memmove(h1.value, src.ctypes.data, n)
        _rc(raw("dr_h2d")(d1, h1, C.c_size_t(n), st), "dr_h2d")
        _rc(raw("dr_d2d")(d2, d1, C.c_size_t(n), st), "dr_d2d")
        _rc(raw("dr_d2h")(h2, d2, C.c_size_t(n), st), "dr_d2h")
        _rc(raw("dr_stream_sync")(st), "dr_stream_sync")
        got = np.ctypeslib.as_array(C.cast(h2, C.POINTER(C.c_uint8)), (n,)).copy()
        np.testing.assert_array_equal(got, src)
        # fill: an unaligned range inside the buffer, the bytes around it untouched
        off, cnt = 13, n - 13 - 29
        _rc(raw("dr_memset")(C.c_void_p(d2.value + off), 0xA5, C.c_size_t(cnt), st), "dr_memset")
        _rc(raw("dr_memset")(d1, 0, C.c_size_t(0), st), "dr_memset of 0 bytes")
        _rc(raw("dr_d2h")(h2, d2, C.c_size_t(n), st), "dr_d2h")
        _rc(raw("dr_stream_sync")(st), "dr_stream_sync")
        got = np.ctypeslib.as_array(C.cast(h2, C.POINTER(C.c_uint8)), (n,)).copy()
        want = src.copy()
        want[off:off + cnt] = 0xA5
        np.testing.assert_array_equal(got, want)
        # graph: capture a fill and a copy on the created stream, replay it three times with
        # other work between the replays, each replay's bytes checked
        g = C.c_void_p()
        _rc(raw("dr_graph_begin")(st), "dr_graph_begin")
        _rc(raw("dr_memset")(d2, 0x3C, C.c_size_t(4096 + 7), st), "dr_memset in capture")
        _rc(raw("dr_d2d")(C.c_void_p(d2.value + 8192), d1, C.c_size_t(4096), st), "dr_d2d in capture")
        _rc(raw("dr_graph_end")(st, C.byref(g)), "dr_graph_end")
        assert g.value
        try:
            for rep in range(3):
                _rc(raw("dr_memset")(d2, rep, C.c_size_t(n), st), "dr_memset")
                _rc(raw("dr_stream_sync")(st), "dr_stream_sync")
                _rc(raw("dr_graph_launch")(g, st), "dr_graph_launch")
                _rc(raw("dr_d2h")(h2, d2, C.c_size_t(n), st), "dr_d2h")
                _rc(raw("dr_stream_sync")(st), "dr_stream_sync")
                got = np.ctypeslib.as_array(C.cast(h2, C.POINTER(C.c_uint8)), (n,)).copy()
                assert (got[:4103] == 0x3C).all(), f"replay {rep}: captured fill"
                assert (got[4103:8192] == rep).all(), f"replay {rep}: bytes past the fill"
                np.testing.assert_array_equal(got[8192:12288], src[:4096], err_msg=f"replay {rep}: captured copy")
                assert (got[12288:] == rep).all(), f"replay {rep}: bytes past the copy"
        finally:
            _rc(raw("dr_graph_destroy")(g), "dr_graph_destroy")
        _rc(raw("dr_device_sync")(), "dr_device_sync")
        hnd = C.c_void_p()
        _rc(raw("dr_cublas_create")(C.byref(hnd), st), "dr_cublas_create")
        assert hnd.value
        assert raw("dr_last_error")() == 0
        assert raw("dr_error_string")(-1) == b"unsupported shape"
        assert raw("dr_error_string")(9001).startswith(b"fused decode step")
    finally:
        _rc(raw("dr_free")(d1), "dr_free")
        _rc(raw("dr_free")(d2), "dr_free")
        _rc(raw("dr_host_free")(h1), "dr_host_free")
        _rc(raw("dr_host_free")(h2), "dr_host_free")
