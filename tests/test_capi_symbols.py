"""CPU checks of the C ABI: the library loads and exports exactly what the
header declares; size queries answer without a GPU."""

import ctypes
import os
import re

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "mtplx_amd.h")
LIB = os.path.join(ROOT, "mtplx_amd", "libmtplx_amd.so")


def _declared():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(mtp_[a-z0-9_]+)\s*\(", text)))


@pytest.fixture(scope="module")
def lib():
    if not os.path.exists(LIB):
        pytest.fail("libmtplx_amd.so is not built (run python -m mtplx_amd.build)")
    return ctypes.CDLL(LIB)


def test_every_declared_symbol_is_exported(lib):
    names = _declared()
    assert len(names) >= 20
    missing = [n for n in names if not hasattr(lib, n)]
    assert not missing, missing


def test_python_binding_matches_header():
    from mtplx_amd._lib import SIGNATURES
    assert sorted(SIGNATURES) == _declared()


def test_size_queries_without_gpu(lib):
    lib.mtp_sampler_workspace_bytes.restype = ctypes.c_size_t
    lib.mtp_attn_workspace_bytes.restype = ctypes.c_size_t
    lib.mtp_qmv_workspace_bytes.restype = ctypes.c_size_t
    assert lib.mtp_sampler_workspace_bytes(7, 151936, 20) == (7 * 38 * 536 + 255) // 256 * 256
    # wide laws (top_k 0 or > 64): per row an id/prob law and a residual area
    row = ((16 + 4 * 151936 + 15) // 16 * 16 + 8 * 151936 + 255) // 256 * 256
    assert lib.mtp_sampler_workspace_bytes(7, 151936, 0) == (7 * 38 * 536 + 255) // 256 * 256 + 2 * 7 * row
    assert lib.mtp_attn_workspace_bytes(8, 8, 32768, 0) == 8 * 8 * 32 * (32 * 128 + 64) * 4
    # tail split: a fixed 64 KiB area of arrival counters first (shared by
    # every shape), then two fp32 [16][64] partials per CU (256 when no device
    # is visible, as here).
    assert lib.mtp_qmv_workspace_bytes(4, 17408, 5120, 0) == 65536 + 2 * 256 * 16 * 64 * 4


def test_error_path_reports_message(lib):
    lib.mtp_last_error.restype = ctypes.c_char_p
    rc = lib.mtp_qmv_affine4(None, None, None, None, None, 4, 8, 100, 64, None, 0, None)
    assert rc == -1
    assert b"K=" in lib.mtp_last_error() or b"M=" in lib.mtp_last_error()


def _struct_fields(text: str, name: str, typedef: bool) -> list[tuple[str, str]]:
    """(field, kind) of struct ``name`` in C source text, in declaration
    order; kind is "ptr", "int", "float", "size_t" or "longlong"."""
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    text = re.sub(r"//[^\n]*", "", text)
    head = rf"typedef\s+struct\s+{name}\s*\{{" if typedef else rf"(?<!typedef )struct\s+{name}\s*\{{"
    m = re.search(head + r"(.*?)\}", text, flags=re.S)
    assert m, name
    out = []
    for decl in m.group(1).split(";"):
        decl = " ".join(decl.split())
        if not decl:
            continue
        base = re.match(r"(const\s+)?(unsigned\s+)?(long long|[A-Za-z_0-9]+)", decl).group(3)
        for part in decl[decl.index(base) + len(base):].split(","):
            ptr = "*" in part or "POINTER" in part
            field = part.replace("*", "").replace("const", "").strip()
            kind = "ptr" if ptr else {"int": "int", "int32_t": "int", "float": "float", "size_t": "size_t",
                                      "long long": "longlong"}[base]
            out.append((field, kind))
    return out


def _ctypes_fields(cls) -> list[tuple[str, str]]:
    kinds = {ctypes.c_int: "int", ctypes.c_float: "float", ctypes.c_size_t: "size_t", ctypes.c_longlong: "longlong",
             ctypes.c_void_p: "ptr"}
    out = []
    for name, ct in cls._fields_:
        out.append((name, "ptr" if issubclass(ct, ctypes._Pointer) else kinds[ct]))
    return out


@pytest.mark.parametrize("name,cls,mirror", [
    ("mtp_rope_out", "RopeOut", "qmv_args.hpp"),
    ("mtp_qmv_args", "QmvArgs", "qmv_args.hpp"),
    ("mtp_qmm_args", "QmmArgs", "qmv_args.hpp"),
    ("mtp_attn_blocks_args", "AttnBlocksArgs", "attn_vt.hpp"),
])
def test_argument_blocks_match_header(name, cls, mirror):
    """Each argument block of the C ABI has the same fields, in the same order
    and of the same kinds, in the header, in the C++ mirror the library is
    compiled against, and in the Python binding."""
    from mtplx_amd import _lib
    want = _struct_fields(open(HEADER).read(), name, typedef=True)
    assert len(want) >= 8
    src = open(os.path.join(ROOT, "mtplx_amd", "csrc", mirror)).read()
    assert _struct_fields(src, name, typedef=False) == want
    assert _ctypes_fields(getattr(_lib, cls)) == want
