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
