"""Shared test helpers: device upload, tolerance checks, format conversions."""
import numpy as np

RTOL = 1e-3
ATOL = 1e-3


def dev(a):
    """numpy -> torch tensor on cuda:0 with the same bytes."""
    import torch

    a = np.ascontiguousarray(a)
    if a.dtype == np.uint16:
        t = torch.from_numpy(a.view(np.int16))
    elif a.dtype == np.uint32:
        t = torch.from_numpy(a.view(np.int32))
    else:
        t = torch.from_numpy(a)
    return t.to("cuda:0")


def host(t, dtype=None):
    a = t.detach().cpu().numpy()
    if dtype is not None:
        a = a.view(dtype)
    return a


def assert_close(got, ref, rtol=RTOL, atol=ATOL, what=""):
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    err = np.abs(got - ref)
    bound = atol + rtol * np.abs(ref)
    bad = err > bound
    if bad.any():
        i = int(np.argmax(err - bound))
        raise AssertionError(
            f"{what}: {int(bad.sum())}/{bad.size} outside atol={atol} rtol={rtol}; worst at {i}: "
            f"got {got.flat[i]!r} ref {ref.flat[i]!r}")


def bits(a):
    return np.ascontiguousarray(a).view(np.uint32)
