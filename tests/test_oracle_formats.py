"""Pins the oracle's format functions against the reference's known-answer tests and closed forms.

KATs: src/apple.rs:185-229 (q4/q8 packed layout), src/convert/mod.rs:614-635 (fp8 e4m3 table,
q8 rounding).  Conversions are checked against independent implementations (numpy float16,
torch bfloat16), exp against float64 numpy.
"""
import numpy as np
import pytest

import oracle as O
import synth


def test_q4_kat_apple_rs():
    # src/apple.rs:206-227: bytes 0..127 as [E=1, N=2, K/2=64]; (scale, min) per 64-group
    packed = np.arange(128, dtype=np.uint8).reshape(2, 64)
    scales = [0.25, 0.5, 0.125, 0.375]
    biases = [-2.0, -3.0, 1.0, -1.0]
    expected = []
    for i, b in enumerate(packed.ravel()):
        for nib in (b & 15, b >> 4):
            g = i // 32
            expected.append(nib * scales[g] + biases[g])
    expected = np.array(expected, np.float32).reshape(2, 128)
    for kind in (O.F16, O.BF16):
        enc = synth.enc(np.array([[scales[0], biases[0], scales[1], biases[1]],
                                  [scales[2], biases[2], scales[3], biases[3]]], np.float32), kind)
        sm = np.ascontiguousarray(enc.reshape(2, 2, 2))
        w = O.dequant_q4(packed, sm, kind, 2, 128)
        np.testing.assert_array_equal(w, expected)


def test_q4_closed_forms():
    rng = np.random.default_rng(1)
    sc = (np.abs(rng.normal(0, 0.02, 4)) + 1e-4).astype(np.float32)
    mn = rng.normal(0, 0.02, 4).astype(np.float32)
    sm = synth.enc(np.stack([sc, mn], -1), O.BF16).reshape(1, 4, 2)
    s, m = synth.bf16_to_f32(sm[..., 0]).ravel(), synth.bf16_to_f32(sm[..., 1]).ravel()
    zeros = np.zeros((1, 128), np.uint8)
    np.testing.assert_array_equal(O.dequant_q4(zeros, sm, O.BF16, 1, 256)[0], np.repeat(m, 64))
    full = np.full((1, 128), 0xFF, np.uint8)
    np.testing.assert_array_equal(O.dequant_q4(full, sm, O.BF16, 1, 256)[0],
                                  np.repeat((np.float32(15) * s).astype(np.float32) + m, 64))
    lo_only = np.full((1, 128), 0x0F, np.uint8)  # even elements 15, odd 0
    w = O.dequant_q4(lo_only, sm, O.BF16, 1, 256)[0]
    np.testing.assert_array_equal(w[1::2], np.repeat(m, 32))


def test_q8_kat_apple_rs():
    # src/apple.rs:191-203: (i as i8).wrapping_mul(3), scales 0.125 / 0.25 per 128-row
    signed = ((np.arange(256) * 3) & 0xFF).astype(np.uint8).view(np.int8).reshape(2, 128)
    s = synth.f32_to_f16(np.array([[0.125], [0.25]], np.float32))
    w = O.dequant_q8(np.ascontiguousarray(signed), np.ascontiguousarray(s), O.F16, 128, 2, 128)
    expected = signed.astype(np.float32) * np.array([[0.125], [0.25]], np.float32)
    np.testing.assert_array_equal(w, expected)
    # per-channel bf16 encoding of the same scales
    sb = synth.f32_to_bf16(np.array([0.125, 0.25], np.float32))
    np.testing.assert_array_equal(O.dequant_q8(np.ascontiguousarray(signed), sb, O.BF16, 128, 2, 128), expected)


def test_q8_quant_kat_convert_rs():
    # src/convert/mod.rs:624-635
    d = np.zeros((1, 128), np.float32)
    d[0, 0], d[0, 1], d[0, 2] = 127.0, 0.5, 1.5
    q, s = O.quant_q8(d)
    assert (int(q[0, 0]), int(q[0, 1]), int(q[0, 2])) == (127, 0, 2)
    assert O.lib().or_f16_to_f32(int(s[0, 0])) == 1.0


def test_fp8_kat_convert_rs():
    L = O.lib()
    assert L.or_fp8e4m3_to_f32(0x38) == 1.0
    assert L.or_fp8e4m3_to_f32(0x7E) == 448.0
    assert L.or_fp8e4m3_to_f32(0xB8) == -1.0
    assert L.or_fp8e4m3_to_f32(0x01) == 2.0 ** -9
    assert np.isnan(L.or_fp8e4m3_to_f32(0x7F))


def test_fp8_table_structure():
    L = O.lib()
    vals = np.array([L.or_fp8e4m3_to_f32(c) for c in range(256)], np.float64)
    pos = vals[:127]
    assert np.all(np.diff(pos) > 0), "codes 0..126 strictly increasing"
    np.testing.assert_array_equal(vals[128:255], -pos)
    assert np.isnan(vals[127]) and np.isnan(vals[255])
    # subnormal spacing 2^-9, then each binade has 8 values
    np.testing.assert_array_equal(pos[:8], np.arange(8) * 2.0 ** -9)
    for e in range(1, 16):
        binade = pos[8 * e: 8 * e + 8]
        binade = binade[~np.isnan(binade)]
        np.testing.assert_array_equal(binade, (1 + np.arange(binade.size) / 8) * 2.0 ** (e - 7))
    np.testing.assert_array_equal(synth.E4M3[:256].astype(np.float64)[~np.isnan(vals)], vals[~np.isnan(vals)])


def test_fp8_encode_roundtrip_and_vectorised_encoder():
    L = O.lib()
    codes = [c for c in range(256) if c not in (0x7F, 0xFF)]
    for c in codes:
        v = L.or_fp8e4m3_to_f32(c)
        enc = L.or_f32_to_fp8e4m3(v)
        assert enc == c or (v == 0 and enc in (0, 0x80)), (c, v, enc)
    rng = np.random.default_rng(3)
    x = np.concatenate([rng.normal(0, 50, 2000), rng.normal(0, 0.01, 2000), [448.0, 500.0, -1e4, 0.0]]).astype(np.float32)
    ref = np.array([L.or_f32_to_fp8e4m3(float(v)) for v in x], np.uint8)
    np.testing.assert_array_equal(synth.f32_to_e4m3(x), ref)


def test_half_conversions_against_numpy_and_torch():
    import torch

    rng = np.random.default_rng(5)
    x = np.concatenate([rng.normal(0, 1, 5000), rng.normal(0, 1e-5, 1000), rng.normal(0, 3e4, 1000)]).astype(np.float32)
    L = O.lib()
    f16 = np.array([L.or_f32_to_f16(float(v)) for v in x], np.uint16)
    np.testing.assert_array_equal(f16, x.astype(np.float16).view(np.uint16))
    back = np.array([L.or_f16_to_f32(int(h)) for h in f16], np.float32)
    np.testing.assert_array_equal(back, f16.view(np.float16).astype(np.float32))
    bf = np.array([L.or_f32_to_bf16(float(v)) for v in x], np.uint16)
    tb = torch.from_numpy(x).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    np.testing.assert_array_equal(bf, tb)
    np.testing.assert_array_equal(synth.f32_to_bf16(x), tb)


def ulp_err(a, ref):
    a = np.asarray(a, np.float64)
    ref = np.asarray(ref, np.float64)
    spacing = np.spacing(np.abs(ref).astype(np.float32)).astype(np.float64)
    return np.abs(a - ref) / spacing


def test_exp_accuracy_and_special_values():
    x = np.concatenate([np.linspace(-86.4, 0, 200001), np.linspace(0, 87.9, 100001)]).astype(np.float32)
    y = O.exp(x)
    ref = np.exp(x.astype(np.float64))
    assert ulp_err(y, ref).max() <= 2.0
    L = O.lib()
    assert L.or_exp(0.0) == 1.0
    assert L.or_exp(-100.0) == 0.0
    assert L.or_exp(-float("inf")) == 0.0
    assert L.or_exp(100.0) == float("inf")
    assert np.isnan(L.or_exp(float("nan")))
    assert np.all(np.diff(O.exp(np.linspace(-20, 0, 100001).astype(np.float32))) >= 0), "monotone"
