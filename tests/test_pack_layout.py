"""The tile-step layouts of dr_moe_pack_q4 and dr_moe_pack_fp8 (include/drama_moe.h): the numpy
restatements the GPU tests compare against (tests/test_gpu_prefill.py::_pack_ref and
_pack_fp8_ref, reshape/transposes) checked
element by element against the header's per-byte definition, on the CPU."""
import numpy as np

from test_gpu_prefill import _pack_fp8_ref, _pack_ref


def test_pack_ref_matches_the_byte_definition():
    rng = np.random.default_rng(0)
    for e, n, k in ((2, 32, 512), (1, 16, 256), (1, 48, 768)):
        spt = k // 256
        q = rng.integers(0, 256, (e, n, k // 2), dtype=np.uint8)
        sm = rng.integers(0, 65536, (e, n, k // 64, 2), dtype=np.uint16)
        qo, so = _pack_ref(q, sm, n, k)
        for ee in range(e):
            for blk in range(n // 16 * spt):
                t, s = divmod(blk, spt)
                for p in range(2):
                    for lane in range(64):
                        src = q[ee, 16 * t + (lane & 15), 128 * s + 64 * p + 16 * (lane >> 4):][:16]
                        dst = qo[ee, blk * 2048 + p * 1024 + 16 * lane:][:16]
                        np.testing.assert_array_equal(dst, src)
                for r in range(16):
                    for w in range(4):
                        np.testing.assert_array_equal(so[ee, (blk * 64 + 4 * r + w) * 2:][:2], sm[ee, 16 * t + r, 4 * s + w])


def test_pack_fp8_ref_matches_the_byte_definition():
    rng = np.random.default_rng(1)
    for e, n, k in ((2, 32, 512), (1, 16, 256)):
        spt = k // 256
        q = rng.integers(0, 256, (e, n, k), dtype=np.uint8)
        qo = _pack_fp8_ref(q, n, k)
        for ee in range(e):
            for blk in range(n // 16 * spt):
                t, s = divmod(blk, spt)
                for p in range(4):
                    for lane in range(64):
                        src = q[ee, 16 * t + (lane & 15), 256 * s + 64 * p + 16 * (lane >> 4):][:16]
                        np.testing.assert_array_equal(qo[ee, blk * 4096 + p * 1024 + 16 * lane:][:16], src)
