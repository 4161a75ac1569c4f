"""CPU checks of the C ABI: the library loads, exports every symbol include/drama_moe.h declares,
and the reference-side entry points have the argument lists of the Rust bindings in
apiplant/drama-rs src/ffi.rs (checked when the reference checkout is present)."""
import ctypes
import os
import re
import subprocess

import pytest

import dramamoe as D

REF_FFI = "/root/reference/src/ffi.rs"
# src/ffi.rs bindings that belong to subsystems outside the MoE path (attention, DeltaNet,
# embedding, sampling, frame bookkeeping) and are deliberately not part of this library
OUT_OF_SCOPE = {"dr_rmsnorm", "dr_embed", "dr_tower_in", "dr_qk_norm_rope", "dr_attn_prefill", "dr_attn_decode",
                "dr_attn_part_floats", "dr_conv", "dr_gdn", "dr_sample_init", "dr_sample_main", "dr_sample_head",
                "dr_frame_end"}


def test_library_exports_every_declared_symbol():
    lib = D.lib()
    assert lib.missing == [], f"declared in include/drama_moe.h but not exported: {lib.missing}"
    nm = subprocess.run(["nm", "-D", "--defined-only", D.LIB_PATH], capture_output=True, text=True, check=True).stdout
    exported = set(re.findall(r" T (dr_[a-z0-9_]+)", nm))
    declared = set(lib.protos)
    assert declared <= exported
    assert exported <= declared, f"exported but not declared: {exported - declared}"


def test_header_parses_and_has_reference_names():
    protos = D.parse_header()
    assert len(protos) >= 40
    for name in ("dr_router_topk", "dr_moe_decode", "dr_moe_prefill", "dr_moe_permute", "dr_moe_combine",
                 "dr_graph_begin", "dr_gemm"):
        assert name in protos


def test_error_strings_and_shape_errors_without_gpu():
    lib = D.lib()
    assert lib.cdll.dr_error_string(-1) == b"unsupported shape"
    # shape gates are checked on the host before any launch, so they run without a device
    assert lib.raw("dr_moe_decode")(*([None] * 15), 4096, 512, 8, None, 0.0, None, 0, None) == -1
    assert lib.raw("dr_moe_prefill")(*([None] * 9), 256, 2048, 256, None) == -1
    assert lib.raw("dr_moe_group")(None, 9000, 256, None, None, None, None) == -1
    # top-k with grouping: more than 8192 pairs, no counter, topk > e
    assert lib.raw("dr_moe_topk_group")(None, 1025, 256, 8, 257, *([None] * 9)) == -1
    assert lib.raw("dr_moe_topk_group")(None, 300, 256, 8, 257, *([None] * 9)) == -1
    assert lib.raw("dr_moe_topk_group")(None, 300, 4, 8, 5, *([None] * 9)) == -1
    assert lib.raw("dr_moe_group_rows")(None, 1025, 8, 256, None, None, None, None, None) == -1
    assert lib.raw("dr_moe_prefill_rows_bf16s")(*([None] * 4), None, 300, None, None, None, None, None, 256, 4096,
                                                512, None) == -1
    assert lib.raw("dr_gemv_q4_bf16s")(None, None, None, None, None, 10, 1000, None) == -1
    # fused small-batch FP8 router + experts: (router_w, nw, eps, e, 8 weight pointers, x, logits, idx,
    # wts, sgate, counter, tags, res, act, y, yb, rows, h, i, topk, st); shapes are rejected before
    # any pointer is used, then null router / buffers
    f = lib.raw("dr_moe_decode_rows_routed_fp8_bf16s")
    base = [1, 1, 1e-6, 256] + [1] * 19 + [4, 2048, 512, 8, None]
    for pos, bad in ((3, 7), (3, 257), (23, 0), (23, 65), (24, 1024), (25, 256), (26, 4)):
        a = list(base)
        a[pos] = bad
        assert f(*a) == -1, (pos, bad)
    for pos in (0, 13, 17, 18):
        a = list(base)
        a[pos] = None
        assert f(*a) == -1, pos


def _rust_decls(text):
    out = {}
    for m in re.finditer(r"pub fn (dr_[a-z0-9_]+)\s*\(([^)]*)\)\s*(->\s*([^;]+))?;", text, re.S):
        args = [a.strip() for a in m.group(2).split(",") if a.strip()]
        kinds = []
        for a in args:
            ty = a.split(":", 1)[1].strip()
            kinds.append("ptr" if ty.startswith("*") or ty in ("Stream", "GraphExec") else ty)
        out[m.group(1)] = kinds
    return out


_C_OF_RUST = {"i32": "int", "u32": "uint32_t", "usize": "size_t", "f32": "float"}


@pytest.mark.skipif(not os.path.exists(REF_FFI), reason="reference checkout not present")
def test_reference_bindings_match_header():
    rust = _rust_decls(open(REF_FFI).read())
    ours = D.parse_header()
    checked = 0
    for name, kinds in rust.items():
        if name in OUT_OF_SCOPE or name.startswith(("dr_rvq", "dr_im2col", "dr_vq", "dr_tconv", "dr_epilogue",
                                                      "dr_dwconv", "dr_layernorm", "dr_rmsnorm_plain", "dr_codec",
                                                      "dr_swiglu16", "dr_conv_out", "dr_gemm_f16")):
            continue
        assert name in ours, f"{name} (src/ffi.rs) is not declared"
        ck = ours[name][1]
        assert len(ck) == len(kinds), f"{name}: {len(ck)} args, reference has {len(kinds)}"
        for i, (a, b) in enumerate(zip(ck, kinds)):
            a = "ptr" if a.startswith("dr_") and a.endswith("_t") else a
            assert a == _C_OF_RUST.get(b, b), f"{name} arg {i}: {a} vs reference {b}"
        checked += 1
    assert checked >= 25


def test_oracle_is_not_linked_into_the_product():
    nm = subprocess.run(["nm", "-D", D.LIB_PATH], capture_output=True, text=True, check=True).stdout
    ldd = subprocess.run(["ldd", D.LIB_PATH], capture_output=True, text=True).stdout
    assert "liboracle" not in ldd
    assert not re.search(r" U or_", nm)


def test_integration_bindings_match_header():
    """The Rust extern block INTEGRATION.md gives a maintainer binds only declared entry points,
    each with the header's argument count and kinds (pointers, i32, u32, usize, f32)."""
    text = open(os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "INTEGRATION.md")).read()
    rust = _rust_decls(text)
    ours = D.parse_header()
    assert len(rust) >= 15
    for name, kinds in rust.items():
        assert name in ours, f"{name} (INTEGRATION.md) is not declared in include/drama_moe.h"
        ck = ours[name][1]
        assert len(ck) == len(kinds), f"{name}: header has {len(ck)} args, INTEGRATION.md {len(kinds)}"
        for i, (a, b) in enumerate(zip(ck, kinds)):
            a = "ptr" if a.startswith("dr_") and a.endswith("_t") else a
            assert a == _C_OF_RUST.get(b, b), f"{name} arg {i}: {a} vs INTEGRATION.md {b}"


def test_pack_entry_points_refuse_overlap_without_gpu():
    """dr_moe_pack_q4 / dr_moe_pack_fp8 return -1 before any launch when an output overlaps an
    input (host pointers: nothing is dereferenced on this path)."""
    lib = D.lib()
    buf = ctypes.create_string_buffer(1 << 20)
    base = ctypes.addressof(buf)
    q4 = lib.raw("dr_moe_pack_q4")
    # e = 1, n = 16, k = 256: 2048 bytes of weights, 256 bytes of scale words
    assert q4(base, base + 4096, 1, 16, 256, base + 1024, base + 8192, None) == -1  # q_out over q
    assert q4(base, base + 4096, 1, 16, 256, base + 16384, base + 4096, None) == -1  # sm_out is sm
    assert q4(base, base + 4096, 1, 16, 256, base + 16384, base + 17000, None) == -1  # q_out over sm_out
    f8 = lib.raw("dr_moe_pack_fp8")
    assert f8(base, 1, 16, 256, base + 2048, None) == -1  # 4096 bytes each, overlapping by half
