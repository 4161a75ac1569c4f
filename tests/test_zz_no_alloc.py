"""dr_moe_decode_step_bf16s_noalloc (the step with its exchange buffer in a file-scope device
array) against dr_moe_decode_step_bf16s with caller buffers: identical bits for routing,
per-layer outputs and the final x, on two calls in a row, the second one smaller (fewer
layers and experts), so the array's leftover contents from the first call must not matter."""
import numpy as np
import pytest

import dramamoe as D
from helpers import bits, dev, host
from test_gpu_step import H, I, TOPK, Stack

pytestmark = pytest.mark.gpu


def _run_noalloc(st, x_dev):
    import torch

    n = len(st.h)
    idx = torch.full((n * TOPK,), -1, dtype=torch.int32, device="cuda")
    wts = torch.zeros(n * TOPK, device="cuda")
    sg = torch.zeros(n, device="cuda")
    xs = torch.zeros(n * H, device="cuda")
    D.lib().dr_moe_decode_step_bf16s_noalloc(D.ptr(st.table), n, D.ptr(x_dev), st.E, H, I, TOPK, 1e-6, D.ptr(idx),
                                             D.ptr(wts), D.ptr(sg), D.ptr(xs), None, 0, D.stream_ptr())
    torch.cuda.synchronize()
    return host(idx), host(wts), host(sg), host(xs)


@pytest.mark.parametrize("first,second", [((256, 3), (64, 2)), ((64, 2), (16, 1))])
def test_noalloc_step_matches_buffered_step(first, second):
    for E, n in (first, second):
        print(f"noalloc step E={E} layers={n}", flush=True)
        st = Stack([900 + E + 5 * i for i in range(n)], E, "cfg")
        x0 = np.random.default_rng(E + n).normal(0, 1, H).astype(np.float32)
        xa, xb = dev(x0), dev(x0)
        want = st.run(xa)
        got = _run_noalloc(st, xb)
        for w, g, what in zip(want, got, ("experts", "weights", "shared gate", "layer outputs")):
            np.testing.assert_array_equal(np.ascontiguousarray(w).ravel().view(np.uint32),
                                          np.ascontiguousarray(g).ravel().view(np.uint32), err_msg=what)
        np.testing.assert_array_equal(bits(host(xb)), bits(host(xa)))
        assert np.isfinite(host(xb)).all()


def test_noalloc_step_rejects_bad_shapes():
    st = Stack([1], 16, "cfg")
    x = dev(np.zeros(H, np.float32))
    f = D.lib().raw("dr_moe_decode_step_bf16s_noalloc")
    base = [D.ptr(st.table), 1, D.ptr(x), 16, H, I, TOPK, 1e-6, None, None, None, None, None, 0, D.stream_ptr()]
    for pos, bad in ((1, 0), (1, 1366), (3, 257), (4, 1024), (5, 256), (6, 4)):
        a = list(base)
        a[pos] = bad
        assert f(*a) == -1


_CHILD = r'''
import ctypes, sys
import numpy as np, torch
sys.path[:0] = sys.argv[1:]
import dramamoe as D
from test_gpu_step import H, I, TOPK, Stack
st = Stack([41, 42], 16, "cfg")          # the caller's buffers, from torch
x0 = np.random.default_rng(3).normal(0, 1, H).astype(np.float32)
L = D.lib()
xa = torch.from_numpy(x0).cuda(); torch.cuda.synchronize()
sp = torch.cuda.current_stream().cuda_stream
# first call of the library in this process: the no-allocation entry point, then the same call
# captured into a graph and replayed
assert L.raw("dr_moe_decode_step_bf16s_noalloc")(D.ptr(st.table), 2, D.ptr(xa), 16, H, I, TOPK, 1e-6,
                                                  None, None, None, None, None, 0, sp) == 0
torch.cuda.synchronize()
s2 = torch.cuda.Stream(); p2 = s2.cuda_stream
xg = torch.from_numpy(x0).cuda(); torch.cuda.synchronize()
g = ctypes.c_void_p()
assert L.raw("dr_graph_begin")(p2) == 0
assert L.raw("dr_moe_decode_step_bf16s_noalloc")(D.ptr(st.table), 2, D.ptr(xg), 16, H, I, TOPK, 1e-6,
                                                  None, None, None, None, None, 0, p2) == 0
assert L.raw("dr_graph_end")(p2, ctypes.byref(g)) == 0
for rep in range(3):
    xg.copy_(torch.from_numpy(x0).cuda()); torch.cuda.synchronize()
    assert L.raw("dr_graph_launch")(g, p2) == 0
    s2.synchronize()
    assert np.array_equal(xg.cpu().numpy().view(np.uint32), xa.cpu().numpy().view(np.uint32)), rep
L.raw("dr_graph_destroy")(g)
xb = torch.from_numpy(x0).cuda()
st.run(xb)
assert np.array_equal(xb.cpu().numpy().view(np.uint32), xa.cpu().numpy().view(np.uint32))
assert L.raw("dr_last_error")() == 0
print("noalloc-first OK")
'''


def test_noalloc_step_first_call_in_a_fresh_process():
    """In a fresh process the no-allocation entry point as the library's first call (its error
    word is set up when the library loads, so the call only launches), then the same call
    captured into a HIP graph and replayed three times: every result equal to the buffered
    step's bits."""
    import os
    import subprocess
    import sys

    here = os.path.dirname(os.path.abspath(__file__))
    root = os.path.dirname(here)
    paths = [here, root, os.path.join(root, "drama-rs_amd"), os.path.join(root, "oracle")]
    r = subprocess.run([sys.executable, "-c", _CHILD, *paths], capture_output=True, text=True, timeout=300)
    assert r.returncode == 0 and "noalloc-first OK" in r.stdout, r.stdout[-2000:] + r.stderr[-3000:]
