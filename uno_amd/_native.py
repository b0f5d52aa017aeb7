"""ctypes binding of the C-ABI in ``include/unok.h`` (library ``uno_amd/libunok.so``).

The library is built in-tree by ``uno_amd.build`` (``__graft_entry__.build()``). There is no
fallback: if the library is missing or a kernel fails, the call raises.
"""
from __future__ import annotations

import ctypes as C
import threading
from pathlib import Path

import torch

LIB_PATH = Path(__file__).resolve().parent / "libunok.so"

F32, BF16 = 0, 1
_EINVAL, _EALIGN, _EUNSUPPORTED = -1, -2, -3

_i, _i64, _p, _f = C.c_int, C.c_int64, C.c_void_p, C.c_float
_u64 = C.c_uint64
_ip = C.POINTER(C.c_int)

# name -> (restype, argtypes); must match include/unok.h exactly.
SIGNATURES: dict[str, tuple] = {
    "unok_abi_version": (_i, []),
    "unok_last_error": (C.c_char_p, []),
    "unok_gemm_nt": (_i, [_i, _i, _i, _i, _i, _p, _i64, _p, _i64, _p, _i64, _p, _i64, _i,
                          _i, _ip, _ip, _p, _i64, _p, _i64, _p, _f, _p]),
    "unok_gemm_nt_swiglu": (_i, [_i, _i, _i, _p, _i64, _p, _i64, _p, _i64, _p, _i64, _i, _p, _i64, _p, _i64, _p]),
    "unok_gemm_nt_swiglu_bwd": (_i, [_i, _i, _i, _p, _i64, _p, _i64, _p, _i64, _p, _i64, _i, _p, _i64, _p, _i64,
                                     _p]),
    "unok_gemm_nt_rows_workspace": (_i64, [_i, _i, _i, _i, _i, _i]),
    "unok_gemm_nt_rows": (_i, [_i, _i, _i, _p, _i64, _p, _i64, _p, _i64, _i, _p, _i64, _i, _i, _ip, _ip, _p, _i64,
                               _p, _i64, _p, _i, _i, _p, _i64, _p]),
    "unok_gemm_tn_workspace": (_i64, [_i, _i, _i]),
    "unok_gemm_tn": (_i, [_i, _i, _i, _i, _p, _i64, _p, _i64, _p, _i64, _f, _f, _p, _i64, _p]),
    "unok_gemm_tn_noalloc": (_i, [_i, _i, _i, _i, _p, _i64, _p, _i64, _p, _i64, _f, _f, _p]),
    "unok_rmsnorm_fwd": (_i, [_i, _i, _i, _p, _i64, _p, _p, _i64, _p, _f, _p]),
    "unok_rmsnorm_bwd": (_i, [_i, _i, _i, _p, _p, _p, _p, _p, _p, _p]),
    "unok_qknorm_rope_fwd": (_i, [_i, _i, _i, _i, _i, _i, _p, _i64, _p, _p, _p, _p, _f, _p, _p, _p, _i64, _p, _p]),
    "unok_qknorm_rope_bwd": (_i, [_i, _i, _i, _i, _i, _i, _i, _p, _p, _p, _i64, _p, _p, _p, _p, _p, _p, _i64, _p]),
    "unok_rope_table": (_i, [_i, _i, _p, _p, _p, _p]),
    "unok_gemm_nt_qkv_rope": (_i, [_i, _i, _i, _i, _p, _i64, _p, _i64, _p, _i64, _p, _i64, _i, _i, _ip, _ip, _p, _p,
                                   _p, _p, _p, _i, _f, _p, _p, _p, _p, _p, _p]),
    "unok_swiglu_fwd": (_i, [_i, _i, _i, _p, _i64, _p, _p]),
    "unok_swiglu_bwd": (_i, [_i, _i, _i, _p, _p, _i64, _p, _i64, _p]),
    "unok_embedding": (_i, [_i, _i, _i, _p, _p, _i64, _p, _p]),
    "unok_rows_copy": (_i, [_i, _i, _p, _i64, _p, _p, _i64, _p, _p]),
    "unok_attn_fwd": (_i, [_i, _i, _i, _i, _i, _p, _i64, _p, _i64, _p, _i64, _p, _i64, _p, _i64,
                           _p, _p, _i64, _p, _f, _p]),
    "unok_attn_fwd_split": (_i, [_i, _i, _i, _p, _i64, _p, _i64, _p, _i64, _p, _p, _i64, _p, _f, _p]),
    "unok_attn_split_combine": (_i, [_i, _i, _i, _p, _i64, _p, _p, _p, _i64, _p]),
    "unok_decode_prep": (_i, [_i, _i, _i, _i, _i, _p, _i64, _p, _p, _p, _p, _f, _p, _p, _i, _p, _p]),
    "unok_attn_bwd": (_i, [_i, _i, _i, _i, _i, _i, _i, _p, _i64, _p, _i64, _p, _i64, _p, _i64, _p, _i64,
                           _p, _p, _p, _i64, _p, _p, _i64, _p, _p, _i64, _p, _i64, _p, _i64, _f, _p]),
    "unok_attn_bwd_qknorm": (_i, [_i, _i, _i, _i, _p, _i64, _p, _i64, _p, _i64, _p, _i64, _p, _i64, _p, _p, _i64,
                                  _p, _p, _i64, _p, _p, _i64, _p, _p, _p, _p, _p, _p, _i, _p, _i64, _f, _p]),
    "unok_bd_prepare": (_i, [_i, _i, _p, _p, _p, _i, _i, _i, _i, _u64, _p, _p, _p, _p, _p, _p, _p, _p, _p,
                             _p, _p, _p]),
    "unok_bd_region": (_i, [_i, _i, _p, _p, _p]),
    "unok_bd_compact": (_i, [_i64, _p, _p, _p, _p, _p, _p]),
    "unok_row_lse_update": (_i, [_i, _i, _i, _p, _i64, _i, _p, _p, _p, _p, _i, _p]),
    "unok_lmhead_ce_stats": (_i, [_i, _i, _i, _p, _i64, _p, _i64, _p, _i, _p, _p, _i64, _p, _p, _i64, _p]),
    "unok_ce_parts_reduce": (_i, [_i, _i, _p, _p, _i64, _p, _p, _p]),
    "unok_lmhead_ce_grad": (_i, [_i, _i, _i, _p, _i64, _p, _i64, _p, _i, _p, _p, _p, _p, _p, _i64, _p]),
    "unok_row_argmax_update": (_i, [_i, _i, _i, _p, _i64, _i, _p, _p, _i, _p]),
    "unok_ce_finish": (_i, [_i, _p, _p, _p, _p, _p, _p, _p, _p]),
    "unok_ce_grad_chunk": (_i, [_i, _i, _i, _p, _i64, _i, _p, _p, _p, _p, _p, _p, _i64, _p]),
    "unok_softmax_stats": (_i, [_i, _i, _i, _p, _i64, _p, _p, _p]),
    "unok_tv_fwd": (_i, [_i, _i, _i, _p, _i64, _p, _i64, _p, _p, _p, _p, _p, _p, _p]),
    "unok_tv_bwd": (_i, [_i, _i, _i, _p, _i64, _p, _i64, _p, _p, _p, _p, _p, _p, _p, _p, _i64, _p]),
    "unok_kl_fwd": (_i, [_i, _i, _i, _p, _i64, _p, _i64, _p, _p, _p, _p, _p, _p]),
    "unok_kl_bwd": (_i, [_i, _i, _i, _p, _i64, _p, _i64, _p, _p, _p, _p, _p, _p, _p, _p, _i64, _p]),
    "unok_sum_scaled": (_i, [_i64, _p, _p, _p, _p]),
    "unok_grad_clip_coef": (_i, [_i64, _p, _p, _i, _f, _p, _p]),
    "unok_adamw_step": (_i, [_i64, _p, _p, _p, _p, _p, _f, _f, _f, _f, _f, _i, _i, _p, _i64, _f, _p]),
    "unok_cast_copy": (_i, [_i, _i64, _i64, _f, _p, _p, _p]),
    "unok_transpose_jobs": (_i, [_i, _p, _i, _i64, _p, _p, _p]),
}

_lock = threading.Lock()
_lib = None


def lib():
    """Loads libunok.so once; raises if it has not been built."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is None:
            if not LIB_PATH.exists():
                raise RuntimeError(
                    f"uno_amd kernel library not found at {LIB_PATH}; build it with "
                    "`python -m uno_amd.build` (no non-HIP fallback exists)")
            handle = C.CDLL(str(LIB_PATH))
            for name, (res, args) in SIGNATURES.items():
                fn = getattr(handle, name)
                fn.restype = res
                fn.argtypes = args
            _lib = handle
    return _lib


def exported_symbols() -> list[str]:
    return list(SIGNATURES)


def check(rc: int, what: str) -> None:
    if rc == 0:
        return
    msg = lib().unok_last_error().decode(errors="replace")
    if rc == _EINVAL:
        raise ValueError(f"{what}: {msg}")
    raise RuntimeError(f"{what} failed (code {rc}): {msg}")


def call(name: str, *args) -> None:
    check(getattr(lib(), name)(*args), name)


def ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()


def dtype_code(dt: torch.dtype) -> int:
    if dt == torch.float32:
        return F32
    if dt == torch.bfloat16:
        return BF16
    raise ValueError(f"unsupported dtype {dt}; the kernels take float32 or bfloat16")


def stream() -> int:
    return torch.cuda.current_stream().cuda_stream


def int_array(values) -> C.Array:
    arr = (C.c_int * max(1, len(values)))()
    for i, v in enumerate(values):
        arr[i] = int(v)
    return arr
