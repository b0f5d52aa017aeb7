"""The C-ABI library loads without a GPU and exports every entry point include/unok.h declares,
with the argument counts the ctypes binding uses (no compute calls are made here)."""
import ctypes
import re
from pathlib import Path

import pytest

from uno_amd import _native as N

ROOT = Path(__file__).resolve().parents[1]


def _header_decls():
    text = (ROOT / "include" / "unok.h").read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    decls = {}
    for m in re.finditer(r"(?:const\s+)?[\w]+\*?\s+(unok_\w+)\s*\(([^)]*)\)\s*;", text):
        args = m.group(2).strip()
        n = 0 if args in ("", "void") else len([a for a in args.split(",") if a.strip()])
        decls[m.group(1)] = n
    return decls


def test_library_built():
    if not N.LIB_PATH.exists():
        pytest.skip("libunok.so not built (run __graft_entry__.build())")
    N.lib()


def test_header_and_binding_agree():
    decls = _header_decls()
    assert len(decls) >= 30
    assert set(decls) == set(N.SIGNATURES), set(decls) ^ set(N.SIGNATURES)
    for name, n in decls.items():
        assert len(N.SIGNATURES[name][1]) == n, (name, n, len(N.SIGNATURES[name][1]))


def test_every_symbol_exported():
    if not N.LIB_PATH.exists():
        pytest.skip("libunok.so not built")
    lib = ctypes.CDLL(str(N.LIB_PATH))
    for name in _header_decls():
        assert hasattr(lib, name), name
    assert lib.unok_abi_version() == 1


def test_argument_errors_need_no_gpu():
    """Argument validation runs before any launch and reports through unok_last_error."""
    if not N.LIB_PATH.exists():
        pytest.skip("libunok.so not built")
    lib = N.lib()
    rc = lib.unok_gemm_nt(7, 0, 4, 4, 4, None, 4, None, 4, None, 0, None, 0, 0, 0, None, None, None, 4, None, 0,
                          None, 1.0, None)
    assert rc == -1
    assert b"in_dtype" in lib.unok_last_error()
    with pytest.raises(ValueError):
        N.check(rc, "unok_gemm_nt")
