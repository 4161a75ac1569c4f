"""Python view of libdramamoe.so (the gfx950 C ABI declared in include/drama_moe.h).

The ctypes signatures are read from the header itself, so the binding cannot drift from the
declared ABI.  Device memory and streams come from torch (ROCm build): pass tensor.data_ptr()
and torch.cuda.current_stream().cuda_stream.  There is no fallback: if the library is missing
this module raises, and every entry point runs the HIP kernels.
"""
from __future__ import annotations

import ctypes as C
import os
import re
import subprocess

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
LIB_PATH = os.path.join(HERE, "libdramamoe.so")
HEADER = os.path.join(ROOT, "include", "drama_moe.h")

_TYPES = {
    "int": C.c_int,
    "float": C.c_float,
    "size_t": C.c_size_t,
    "void": None,
    "uint32_t": C.c_uint32,
}


def parse_header(path: str = HEADER) -> dict[str, tuple[str, list[str]]]:
    """Returns {name: (return type, [argument types])} for every prototype in the header."""
    text = open(path).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    text = re.sub(r"#.*", "", text)
    protos = {}
    for m in re.finditer(r"((?:const\s+)?[A-Za-z_][A-Za-z0-9_]*\s*\*?)\s*(dr_[a-z0-9_]+)\s*\(([^;]*?)\)\s*;", text, re.S):
        ret, name, args = m.group(1).strip(), m.group(2), m.group(3).strip()
        argl = [] if args in ("", "void") else [a.strip() for a in args.split(",")]
        types = []
        for a in argl:
            a = re.sub(r"\s+", " ", a)
            if "*" in a:
                types.append("ptr")
            else:
                toks = a.replace("const ", "").split(" ")
                types.append(toks[0] if len(toks) > 1 else toks[0])
        protos[name] = (ret, types)
    return protos


def _ctype(t: str):
    if t == "ptr" or t.endswith("_t") and t not in _TYPES:
        return C.c_void_p
    return _TYPES[t]


def _ret_type(r: str):
    if "*" in r:
        return C.c_char_p if "char" in r else C.c_void_p
    return _TYPES[r]


def header_define(name: str, path: str = HEADER) -> int:
    """Integer value of a #define in the header (e.g. DR_STEP_LL_WORDS)."""
    m = re.search(r"#define\s+" + name + r"\s+(\d+)", open(path).read())
    if not m:
        raise KeyError(name)
    return int(m.group(1))


class DramaMoeError(RuntimeError):
    pass


class Lib:
    """Loaded library with every header prototype bound; calls raise on a nonzero return."""

    def __init__(self, path: str = LIB_PATH):
        if not os.path.exists(path):
            raise DramaMoeError(
                f"{path} is missing: build it with `make -C {HERE}` (or __graft_entry__.build()); "
                "there is no CPU fallback")
        self.cdll = C.CDLL(path)
        self.protos = parse_header()
        self.missing = []
        for name, (ret, args) in self.protos.items():
            try:
                fn = getattr(self.cdll, name)
            except AttributeError:
                self.missing.append(name)
                continue
            fn.restype = _ret_type(ret)
            fn.argtypes = [_ctype(a) for a in args]

    def raw(self, name: str):
        return getattr(self.cdll, name)

    def __getattr__(self, name: str):
        if not name.startswith("dr_"):
            raise AttributeError(name)
        fn = getattr(self.cdll, name)
        ret = self.protos[name][0]

        def call(*args):
            rc = fn(*args)
            if ret == "int" and rc != 0:
                msg = self.cdll.dr_error_string(rc).decode() if rc != -1 else "unsupported shape"
                raise DramaMoeError(f"{name} returned {rc}: {msg}")
            return rc

        return call


_lib: Lib | None = None
STEP_LL_WORDS = header_define("DR_STEP_LL_WORDS")


def build() -> None:
    subprocess.run(["make", "-s", "-j8", "-C", HERE], check=True)


def lib() -> Lib:
    global _lib
    if _lib is None:
        _lib = Lib()
    return _lib


def stream_ptr(stream=None) -> int:
    import torch

    s = stream if stream is not None else torch.cuda.current_stream()
    return s.cuda_stream


def ptr(t) -> int | None:
    """Device pointer of a torch tensor (None stays NULL)."""
    if t is None:
        return None
    assert t.is_contiguous(), "buffers must be contiguous"
    return t.data_ptr()
