"""ctypes view of the CPU oracle (liboracle.so).  TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg import this module; the
product library never does.  Arrays are numpy; half-precision values travel as uint16 bits.
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "liboracle.so")

F16, BF16, F32 = 0, 1, 2

_lib = None


def build() -> None:
    subprocess.run(["make", "-s", "-C", HERE], check=True)


def lib() -> C.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build()
        _lib = C.CDLL(LIB_PATH)
        _declare(_lib)
    return _lib


P = C.c_void_p


def _declare(L: C.CDLL) -> None:
    i, f, u16, u8 = C.c_int, C.c_float, C.c_uint16, C.c_uint8
    sig = {
        "or_bf16_to_f32": (f, [u16]),
        "or_f32_to_bf16": (u16, [f]),
        "or_f16_to_f32": (f, [u16]),
        "or_f32_to_f16": (u16, [f]),
        "or_fp8e4m3_to_f32": (f, [u8]),
        "or_f32_to_fp8e4m3": (u8, [f]),
        "or_exp": (f, [f]),
        "or_exp_array": (None, [P, P, C.c_size_t]),
        "or_rmsnorm_canon": (None, [P, P, f, i, P]),
        "or_dot_bf16_canon": (f, [P, P, i]),
        "or_router_logits": (None, [P, P, i, i, P]),
        "or_softmax_topk": (i, [P, i, i, P, P]),
        "or_router_topk": (i, [P, P, P, f, P, i, i, i, P, P, P]),
        "or_moe_topk": (i, [P, i, i, i, i, P, P, P]),
        "or_router_logits_rows": (i, [P, P, P, i, i, i]),
        "or_moe_group": (i, [P, i, i, P, P, P]),
        "or_dequant_q4": (None, [P, P, i, i, i, P]),
        "or_dequant_q8": (None, [P, P, i, i, i, i, P]),
        "or_dequant_fp8": (None, [P, P, i, i, i, P]),
        "or_quant_q8": (None, [P, i, i, P, P]),
        "or_gemv_q4": (None, [P, P, i, P, i, i, P]),
        "or_gemv_q8": (None, [P, P, i, i, P, i, i, P]),
        "or_moe_decode": (i, [P, P, P, P, P, P, P, P, i, i, i, P, f]),
        "or_moe_decode_rows": (i, [P, P, i, P, P, P, P, i, i, i]),
        "or_moe_prefill_layer": (i, [P, P, i, P, P, P, P, i, i, i]),
        "or_moe_prefill_experts": (i, [P, P, P, P, i, P, P, i, i]),
        "or_shared_prefill": (i, [P, P, i, P, P, i, i]),
        "or_cpu_layer_f32": (i, [P, P, P, f, P, P, P, i, i, i, i, P, P]),
        "or_num_threads": (i, []),
        "or_set_threads": (None, [i]),
    }
    for name, (res, args) in sig.items():
        fn = getattr(L, name)
        fn.restype = res
        fn.argtypes = args


def ptr(a):
    if a is None:
        return None
    assert a.flags["C_CONTIGUOUS"], "oracle arrays must be contiguous"
    return a.ctypes.data


class MoeWeights(C.Structure):
    _fields_ = [
        ("kind", C.c_int),
        ("gu_q", P), ("gu_s", P), ("d_q", P), ("d_s", P), ("sc_kind", C.c_int),
        ("sgu_q", P), ("sgu_s", P), ("sd_q", P), ("sd_s", P), ("sh_kind", C.c_int),
        ("sh_group_gu", C.c_int), ("sh_group_d", C.c_int),
    ]


def moe_weights(layer) -> tuple[MoeWeights, list]:
    """Builds the C struct from a dict-like synthetic layer (see tests/synth.py)."""
    keep = []

    def p(a):
        keep.append(a)
        return ptr(a)

    w = MoeWeights()
    w.kind = 0 if layer["kind"] == "q4" else 1
    w.gu_q, w.gu_s = p(layer["gu_q"]), p(layer["gu_s"])
    w.d_q, w.d_s = p(layer["d_q"]), p(layer["d_s"])
    w.sc_kind = layer["sc_kind"]
    w.sgu_q, w.sgu_s = p(layer["sgu_q"]), p(layer["sgu_s"])
    w.sd_q, w.sd_s = p(layer["sd_q"]), p(layer["sd_s"])
    w.sh_kind = layer["sh_kind"]
    w.sh_group_gu, w.sh_group_d = layer["sh_group_gu"], layer["sh_group_d"]
    return w, keep


# ---- numpy-level helpers ---------------------------------------------------------------------

def bf16_to_f32(h: np.ndarray) -> np.ndarray:
    return (h.astype(np.uint32) << 16).view(np.float32)


def f32_to_bf16(x: np.ndarray) -> np.ndarray:
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    nan = np.isnan(x)
    if nan.any():
        r[nan] = 0x7FC0
    return r


def f16_to_f32(h: np.ndarray) -> np.ndarray:
    return h.view(np.float16).astype(np.float32)


def f32_to_f16(x: np.ndarray) -> np.ndarray:
    return np.asarray(x, dtype=np.float32).astype(np.float16).view(np.uint16)


def scale_to_f32(s: np.ndarray, kind: int) -> np.ndarray:
    if kind == F32:
        return s.astype(np.float32)
    return bf16_to_f32(s) if kind == BF16 else f16_to_f32(s)


def exp(x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    y = np.empty_like(x)
    lib().or_exp_array(ptr(x), ptr(y), x.size)
    return y


def rmsnorm(x, nw, eps):
    x = np.ascontiguousarray(x, np.float32)
    out = np.empty_like(x)
    lib().or_rmsnorm_canon(ptr(x), ptr(nw) if nw is not None else None, eps, x.size, ptr(out))
    return out


def router_topk(W, x, nw, eps, E, topk):
    K = x.size
    logits = np.empty(E + 1, np.float32)
    idx = np.empty(topk, np.int32)
    wts = np.empty(topk, np.float32)
    sg = np.empty(1, np.float32)
    rc = lib().or_router_topk(ptr(W), ptr(x), ptr(nw) if nw is not None else None, eps, ptr(logits),
                              E, topk, K, ptr(idx), ptr(wts), ptr(sg))
    if rc:
        raise ValueError("or_router_topk: unsupported shape")
    return logits, idx, wts, sg[0]


def softmax_topk(logits, E, topk):
    logits = np.ascontiguousarray(logits, np.float32)
    idx = np.empty(topk, np.int32)
    wts = np.empty(topk, np.float32)
    rc = lib().or_softmax_topk(ptr(logits), E, topk, ptr(idx), ptr(wts))
    if rc:
        raise ValueError("or_softmax_topk: unsupported shape")
    return idx, wts


def moe_topk(logits, rows, E, topk, stride):
    idx = np.empty(rows * topk, np.int32)
    wts = np.empty(rows * topk, np.float32)
    sg = np.empty(rows, np.float32)
    rc = lib().or_moe_topk(ptr(logits), rows, E, topk, stride, ptr(idx), ptr(wts), ptr(sg))
    if rc:
        raise ValueError("or_moe_topk: unsupported shape")
    return idx, wts, sg


def router_logits_rows(A, W, M, N, K):
    out = np.empty(M * N, np.float32)
    rc = lib().or_router_logits_rows(ptr(A), ptr(W), ptr(out), M, N, K)
    if rc:
        raise ValueError("or_router_logits_rows: unsupported shape")
    return out.reshape(M, N)


def moe_group(idx, E):
    idx = np.ascontiguousarray(idx, np.int32)
    counts = np.empty(E, np.int32)
    offsets = np.empty(E, np.int32)
    slot_of = np.empty(idx.size, np.int32)
    rc = lib().or_moe_group(ptr(idx), idx.size, E, ptr(counts), ptr(offsets), ptr(slot_of))
    if rc:
        raise ValueError("or_moe_group: index out of range")
    return counts, offsets, slot_of


def dequant_q4(q, sm, kind, N, K):
    w = np.empty(N * K, np.float32)
    lib().or_dequant_q4(ptr(q), ptr(sm), kind, N, K, ptr(w))
    return w.reshape(N, K)


def dequant_q8(q, s, kind, group, N, K):
    w = np.empty(N * K, np.float32)
    lib().or_dequant_q8(ptr(q), ptr(s), kind, group, N, K, ptr(w))
    return w.reshape(N, K)


def dequant_fp8(w8, s, kind, N, K):
    w = np.empty(N * K, np.float32)
    lib().or_dequant_fp8(ptr(w8), ptr(s), kind, N, K, ptr(w))
    return w.reshape(N, K)


def quant_q8(w):
    N, K = w.shape
    w = np.ascontiguousarray(w, np.float32)
    q = np.empty((N, K), np.int8)
    s = np.empty((N, K // 128), np.uint16)
    lib().or_quant_q8(ptr(w), N, K, ptr(q), ptr(s))
    return q, s


def gemv_q4(q, sm, kind, x, N, K):
    y = np.empty(N, np.float32)
    lib().or_gemv_q4(ptr(q), ptr(sm), kind, ptr(np.ascontiguousarray(x, np.float32)), N, K, ptr(y))
    return y


def gemv_q8(q, s, kind, group, x, N, K):
    y = np.empty(N, np.float32)
    lib().or_gemv_q8(ptr(q), ptr(s), kind, group, ptr(np.ascontiguousarray(x, np.float32)), N, K, ptr(y))
    return y


def moe_decode(layer, x, idx, wts, sgate, res, H, I, topk, nw=None, eps=1e-6):
    w, keep = moe_weights(layer)
    act = np.empty((topk + 1) * I, np.float32)
    y = np.empty(H, np.float32)
    sg = np.asarray([sgate], np.float32)
    x = np.ascontiguousarray(x, np.float32)
    res = np.ascontiguousarray(res, np.float32)
    idx = np.ascontiguousarray(idx, np.int32)
    wts = np.ascontiguousarray(wts, np.float32)
    rc = lib().or_moe_decode(C.byref(w), ptr(x), ptr(idx), ptr(wts), ptr(sg), ptr(res), ptr(act), ptr(y),
                             H, I, topk, ptr(nw) if nw is not None else None, eps)
    if rc:
        raise ValueError("or_moe_decode failed")
    return act, y


def cpu_layer_f32(layer, x, res, H, I, topk, eps=1e-6):
    """fp32 host baseline of one int4 decode layer (router, top-k, experts, shared): returns
    (idx, wts, y).  Measurement infrastructure, checked against moe_decode by the tests."""
    w, keep = moe_weights(layer)
    E = layer["gu_q"].shape[0]
    x = np.ascontiguousarray(x, np.float32)
    res = np.ascontiguousarray(res, np.float32)
    y = np.empty(H, np.float32)
    idx = np.empty(topk, np.int32)
    wts = np.empty(topk, np.float32)
    nw = layer.get("nw")
    rc = lib().or_cpu_layer_f32(C.byref(w), ptr(np.ascontiguousarray(layer["router"])), ptr(nw) if nw is not None else None,
                                eps, ptr(x), ptr(res), ptr(y), E, H, I, topk, ptr(idx), ptr(wts))
    if rc:
        raise ValueError("or_cpu_layer_f32: unsupported shape")
    return idx, wts, y


def moe_prefill_experts(layer, xp, offsets, counts, E, H, I):
    w, keep = moe_weights(layer)
    n = xp.shape[0]
    act = np.empty((n, I), np.uint16)
    yp = np.empty((n, H), np.float32)
    lib().or_moe_prefill_experts(C.byref(w), ptr(xp), ptr(offsets), ptr(counts), E, ptr(act), ptr(yp), H, I)
    return act, yp


def shared_prefill(layer, hn_b, rows, H, I):
    w, keep = moe_weights(layer)
    act = np.empty((rows, I), np.uint16)
    out = np.empty((rows, H), np.float32)
    lib().or_shared_prefill(C.byref(w), ptr(hn_b), rows, ptr(act), ptr(out), H, I)
    return act, out


def moe_prefill_layer(layer, hn_b, rows, idx, wts, sgate, x, H, I, topk):
    w, keep = moe_weights(layer)
    x = np.array(x, np.float32, copy=True)
    rc = lib().or_moe_prefill_layer(C.byref(w), ptr(hn_b), rows, ptr(idx), ptr(wts), ptr(sgate), ptr(x), H, I, topk)
    if rc:
        raise ValueError("or_moe_prefill_layer failed")
    return x
