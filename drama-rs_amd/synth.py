"""Seeded synthetic MoE layers in the layouts of the C ABI (numpy, host side).

Distributions follow the benchmark configurations: int4 nibbles uniform 0..15, group-64
scale |N(0, 0.02)| + 1e-4 and min N(0, 0.02); int8 values uniform -127..127 with
per-output-channel scales; fp8 e4m3 weights quantised from N(0, 0.02) with one scale per
128x128 block; router bf16 N(0, 0.02).  Two scale encodings:
  fmt="ref": f16 (scale, min) pairs and f16 int8 scales per 128 inputs (the reference layout,
             src/model.rs:16-43, tools/convert.py:33-41,92-110)
  fmt="cfg": bf16 pairs and bf16 per-channel int8 scales (the benchmark configurations).
"""
from __future__ import annotations

import numpy as np

F16, BF16, F32 = 0, 1, 2


def f32_to_bf16(x: np.ndarray) -> np.ndarray:
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    return ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)


def bf16_to_f32(h: np.ndarray) -> np.ndarray:
    return (np.asarray(h).astype(np.uint32) << 16).view(np.float32)


def f32_to_f16(x: np.ndarray) -> np.ndarray:
    return np.asarray(x, dtype=np.float32).astype(np.float16).view(np.uint16)


def enc(x: np.ndarray, kind: int) -> np.ndarray:
    if kind == BF16:
        return f32_to_bf16(x)
    if kind == F16:
        return f32_to_f16(x)
    return np.ascontiguousarray(x, dtype=np.float32)


def dec(h: np.ndarray, kind: int) -> np.ndarray:
    if kind == BF16:
        return bf16_to_f32(h)
    if kind == F16:
        return np.asarray(h).view(np.float16).astype(np.float32)
    return np.asarray(h, dtype=np.float32)


# ---- fp8 e4m3 (OCP): codes 0..126 are the finite non-negative values in increasing order
def _e4m3_table() -> np.ndarray:
    c = np.arange(256)
    s, e, m = (c >> 7) & 1, (c >> 3) & 15, c & 7
    mag = np.where(e == 0, m / 8.0 * 2.0 ** -6, (1 + m / 8.0) * 2.0 ** (e - 7.0))
    mag = np.where((e == 15) & (m == 7), np.nan, mag)
    return np.where(s == 1, -mag, mag).astype(np.float32)


E4M3 = _e4m3_table()
_POS = E4M3[:127].astype(np.float64)


def f32_to_e4m3(x: np.ndarray) -> np.ndarray:
    """Round to nearest, ties to even code, saturating at +-448."""
    x = np.asarray(x, dtype=np.float64)
    a = np.minimum(np.abs(x), 448.0)
    hi = np.clip(np.searchsorted(_POS, a), 0, 126)
    lo = np.clip(hi - 1, 0, 126)
    dlo, dhi = a - _POS[lo], _POS[hi] - a
    pick = np.where(dlo < dhi, lo, np.where(dhi < dlo, hi, np.where(lo % 2 == 0, lo, hi)))
    return (pick | np.where(np.signbit(x), 0x80, 0)).astype(np.uint8)


def q4_experts(rng, E, N, K, kind):
    q = rng.integers(0, 256, size=(E, N, K // 2), dtype=np.uint8)
    sc = np.abs(rng.normal(0, 0.02, size=(E, N, K // 64))) + 1e-4
    mn = rng.normal(0, 0.02, size=(E, N, K // 64))
    sm = np.stack([enc(sc.astype(np.float32), kind), enc(mn.astype(np.float32), kind)], axis=-1)
    return q, np.ascontiguousarray(sm)


def q8_dense(rng, N, K, fmt):
    q = rng.integers(-127, 128, size=(N, K), dtype=np.int8)
    if fmt == "ref":
        s = (np.abs(rng.normal(0, 0.02, size=(N, K // 128))) + 1e-4) / 73.0
        return q, f32_to_f16(s.astype(np.float32)), F16, 128
    s = (np.abs(rng.normal(0, 0.02, size=(N,))) + 1e-4) / 73.0
    return q, f32_to_bf16(s.astype(np.float32)), BF16, K


def fp8_experts_quick(rng, E, N, K, kind):
    """Like fp8_experts at a fraction of the host time (for large multi-layer tests): codes
    drawn from a pool of e4m3-rounded N(0, 100) values, block scales |N(0, 0.02)| / 100."""
    pool = f32_to_e4m3(rng.normal(0, 100.0, size=1 << 16).astype(np.float32))
    q = pool[rng.integers(0, pool.size, size=(E, N, K), dtype=np.int64)]
    s = (np.abs(rng.normal(0, 0.02, size=(E, N // 128, K // 128))) + 1e-4).astype(np.float32) / 100.0
    return np.ascontiguousarray(q), enc(s, kind)


def fp8_experts(rng, E, N, K, kind):
    w = rng.normal(0, 0.02, size=(E, N, K)).astype(np.float32)
    blk = w.reshape(E, N // 128, 128, K // 128, 128)
    amax = np.maximum(np.abs(blk).max(axis=(2, 4)), 1e-12)
    s = dec(enc((amax / 448.0).astype(np.float32), kind), kind)
    q = f32_to_e4m3(blk / s[:, :, None, :, None]).reshape(E, N, K)
    return np.ascontiguousarray(q), enc(s, kind)


def make_layer(seed: int, E: int = 256, H: int = 2048, I: int = 512, fmt: str = "cfg", kind: str = "q4",
               with_norm: bool = True, quick: bool = False) -> dict:
    rng = np.random.default_rng(seed)
    L = {"E": E, "H": H, "I": I, "fmt": fmt, "kind": kind}
    L["router"] = f32_to_bf16(rng.normal(0, 0.02, size=(E + 1, H)).astype(np.float32))
    L["nw"] = (1.0 + rng.normal(0, 0.1, size=H)).astype(np.float32) if with_norm else None
    if kind == "q4":
        sk = BF16 if fmt == "cfg" else F16
        L["gu_q"], L["gu_s"] = q4_experts(rng, E, 2 * I, H, sk)
        L["d_q"], L["d_s"] = q4_experts(rng, E, H, I, sk)
    else:
        sk = BF16 if fmt == "cfg" else F32
        fx = fp8_experts_quick if quick else fp8_experts
        L["gu_q"], L["gu_s"] = fx(rng, E, 2 * I, H, sk)
        L["d_q"], L["d_s"] = fx(rng, E, H, I, sk)
    L["sc_kind"] = sk
    L["sgu_q"], L["sgu_s"], L["sh_kind"], L["sh_group_gu"] = q8_dense(rng, 2 * I, H, fmt)
    L["sd_q"], L["sd_s"], _, L["sh_group_d"] = q8_dense(rng, H, I, fmt)
    return L


def layer_bytes(L: dict) -> int:
    """Bytes of every weight tensor of the layer."""
    return sum(L[k].nbytes for k in ("router", "gu_q", "gu_s", "d_q", "d_s", "sgu_q", "sgu_s", "sd_q", "sd_s"))


def decode_bytes(L: dict, topk: int = 8) -> int:
    """Algorithmic HBM bytes of one decode token through the layer: router, topk experts'
    gate_up and down (values and scales), the shared expert, x/nw/act/y traffic."""
    E = L["E"]
    per_expert = (L["gu_q"].nbytes + L["gu_s"].nbytes + L["d_q"].nbytes + L["d_s"].nbytes) // E
    shared = L["sgu_q"].nbytes + L["sgu_s"].nbytes + L["sd_q"].nbytes + L["sd_s"].nbytes
    H, I = L["H"], L["I"]
    act = (topk + 1) * I * 4
    vec = H * 4 * 3 + (H * 4 if L["nw"] is not None else 0)  # x read, res read, y write (+ nw)
    return L["router"].nbytes + topk * per_expert + shared + 2 * act + vec
