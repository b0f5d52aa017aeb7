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


def _args(name, **over):
    """Arguments for ``name`` from its ctypes signature: 0 for integers and floats, null pointers,
    then the positional overrides given as ``a<index>=value``."""
    types = N.SIGNATURES[name][1]
    args = [None if t in (ctypes.c_void_p,) or hasattr(t, "contents") else (0.0 if t is ctypes.c_float else 0)
            for t in types]
    for k, v in over.items():
        args[int(k[1:])] = v
    return args


# (entry point, positional overrides, return code, text of the message): each call is rejected by
# the entry point's own argument checks before any HIP call, so it needs no GPU.
BAD_CALLS = [
    ("unok_gemm_nt", dict(a0=1, a1=1, a2=-1), -1, "negative size"),
    ("unok_gemm_nt_swiglu", dict(a0=100, a1=256, a2=64), -1, "multiples of 256"),
    ("unok_gemm_nt_swiglu_bwd", dict(a0=-1), -1, "negative size"),
    ("unok_gemm_nt_rows", dict(a0=-1), -1, "negative size"),
    ("unok_gemm_nt_rows", dict(a0=128, a1=256, a2=100), -1, "multiple of 128"),
    ("unok_gemm_tn", dict(a0=1, a1=-1), -1, "negative size"),
    ("unok_gemm_tn_noalloc", dict(a0=1, a1=64, a2=256, a3=100000), -1, "scratch"),
    ("unok_gemm_nt_qkv_rope", dict(a0=256, a1=64, a2=0, a3=1), -1, "bad sizes"),
    ("unok_rmsnorm_fwd", dict(a0=1, a1=4, a2=3), -2, "rmsnorm"),
    ("unok_qknorm_rope_fwd", dict(a0=1, a1=1, a2=4, a3=1, a4=1, a5=96), -1, "head dim"),
    ("unok_swiglu_fwd", dict(a0=1, a1=4, a2=3), -2, "swiglu"),
    ("unok_embedding", dict(a0=2, a1=1, a2=3), -2, "multiple of 16"),
    ("unok_rows_copy", dict(a0=3, a1=1), -2, "multiples of 16"),
    ("unok_attn_fwd", dict(a0=7, a1=128, a2=1, a3=1, a4=128), -1, "dtype"),
    ("unok_attn_fwd_split", dict(a0=128, a1=0), -1, "S=0"),
    ("unok_decode_prep", dict(a0=1, a1=1, a2=3, a3=2), -1, "nq=3 nk=2"),
    ("unok_bd_prepare", dict(a0=-1), -1, "negative shape"),
    ("unok_lmhead_ce_stats", dict(a0=1, a1=256, a2=64, a4=64, a6=64, a11=1), -1, "blocks"),
    ("unok_ce_parts_reduce", dict(a0=1, a1=0), -1, "bad sizes"),
    ("unok_row_lse_update", dict(a0=1, a1=4, a2=8, a4=4), -1, "ldz=4"),
    ("unok_row_argmax_update", dict(a0=1, a1=-1), -1, "R=-1"),
    ("unok_ce_grad_chunk", dict(a0=1, a1=4, a2=8, a4=8, a12=4), -1, "lddz=4"),
    ("unok_ce_grad_chunk", dict(a0=9, a1=4, a2=8, a4=8, a12=8), -1, "bad dtype"),
    ("unok_softmax_stats", dict(a0=1, a1=-1), -1, "softmax_stats"),
    ("unok_tv_bwd", dict(a0=1, a1=2, a2=8, a4=8, a6=8, a15=4), -1, "tv_bwd"),
    ("unok_kl_fwd", dict(a0=1, a1=2, a2=8, a4=4, a6=8), -1, "kl_fwd"),
    ("unok_sum_scaled", dict(a0=-1), -1, "sum_scaled"),
    ("unok_grad_clip_coef", dict(a3=0), -1, "nparts=0"),
    ("unok_adamw_step", dict(a11=0), -1, "step must be >= 1"),
    ("unok_cast_copy", dict(a0=5, a1=8), -1, "bad dtype"),
    ("unok_transpose_jobs", dict(a0=1, a2=-1), -1, "njobs=-1"),
]


@pytest.mark.parametrize("name,over,code,text", BAD_CALLS, ids=[f"{c[0]}-{i}" for i, c in enumerate(BAD_CALLS)])
def test_entry_points_reject_bad_arguments(name, over, code, text):
    """Each entry point checks sizes, strides and dtypes first and reports through unok_last_error."""
    if not N.LIB_PATH.exists():
        pytest.skip("libunok.so not built")
    lib = N.lib()
    rc = getattr(lib, name)(*_args(name, **over))
    msg = lib.unok_last_error().decode()
    assert rc == code, (name, rc, msg)
    assert text in msg, (name, msg)
    with pytest.raises(ValueError if code == -1 else RuntimeError):
        N.check(rc, name)
