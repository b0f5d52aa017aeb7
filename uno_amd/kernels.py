"""Functional wrappers over the HIP kernel library (one per C-ABI entry point).

Every wrapper validates shapes and strides on the host, allocates outputs with torch (which
owns all device memory) and enqueues the kernel on torch's current stream. There is no
non-HIP code path.
"""
from __future__ import annotations

from typing import Sequence

import torch

from . import _native as N


def _rowmajor(t: torch.Tensor, name: str) -> None:
    if t.dim() != 2:
        raise RuntimeError(f"{name} must be 2-D, got shape {tuple(t.shape)}")
    if t.shape[1] > 1 and t.stride(1) != 1:
        raise RuntimeError(f"{name} must have unit stride along its last dimension")
    if not t.is_cuda:
        raise RuntimeError(f"{name} must be a device tensor")


def _ld(t: torch.Tensor) -> int:
    return t.stride(0) if t.shape[0] > 1 else max(t.shape[1], 1)


def gemm_nt(a: torch.Tensor, b: torch.Tensor, *, a2: torch.Tensor | None = None,
            b2: torch.Tensor | None = None, segments: Sequence[tuple[int, int]] | None = None,
            out: torch.Tensor | None = None, residual: torch.Tensor | None = None,
            gate: torch.Tensor | None = None, alpha: float = 1.0,
            out_dtype: torch.dtype | None = None) -> torch.Tensor:
    """out = alpha * gate (.) (a @ b.T + a2[:, seg] @ b2.T) + residual.

    a [M,K], b [N,K]; a2 [M,*], b2 [N,K2] (the LoRA extension); ``segments`` is a list of
    (n_end, a2_col) pairs: output columns < n_end (and >= the previous end) use
    a2[:, a2_col:a2_col+K2]. ``gate`` is a [M] bool/uint8 row gate on the product.
    """
    _rowmajor(a, "a")
    _rowmajor(b, "b")
    M, K = a.shape
    Nn = b.shape[0]
    if b.shape[1] != K:
        raise RuntimeError(f"gemm_nt: inner dims differ: a {tuple(a.shape)} b {tuple(b.shape)}")
    if b.dtype != a.dtype:
        raise RuntimeError("gemm_nt: a and b dtypes differ")
    out_dtype = out_dtype or (out.dtype if out is not None else a.dtype)
    if out is None:
        out = torch.empty((M, Nn), device=a.device, dtype=out_dtype)
    _rowmajor(out, "out")
    if tuple(out.shape) != (M, Nn) or out.dtype != out_dtype:
        raise RuntimeError("gemm_nt: out has the wrong shape or dtype")
    K2 = 0
    seg_end, seg_col = [], []
    if a2 is not None:
        _rowmajor(a2, "a2")
        _rowmajor(b2, "b2")
        if a2.dtype != a.dtype or b2.dtype != a.dtype:
            raise RuntimeError("gemm_nt: extension dtypes must match a")
        if a2.shape[0] != M or b2.shape[0] != Nn:
            raise RuntimeError("gemm_nt: extension operand shapes do not match M/N")
        K2 = b2.shape[1]
        segs = list(segments) if segments else [(Nn, 0)]
        for n_end, col in segs:
            if col + K2 > a2.shape[1]:
                raise RuntimeError("gemm_nt: extension segment exceeds a2 columns")
        seg_end = [s[0] for s in segs]
        seg_col = [s[1] for s in segs]
    if residual is not None:
        _rowmajor(residual, "residual")
        if tuple(residual.shape) != (M, Nn) or residual.dtype != out_dtype:
            raise RuntimeError("gemm_nt: residual must match out")
    if gate is not None:
        if gate.dtype not in (torch.bool, torch.uint8) or gate.numel() != M or not gate.is_contiguous():
            raise RuntimeError("gemm_nt: gate must be a contiguous bool/uint8 vector of length M")
    N.call("unok_gemm_nt", N.dtype_code(a.dtype), N.dtype_code(out_dtype), M, Nn, K,
           N.ptr(a), _ld(a), N.ptr(b), _ld(b),
           N.ptr(a2), _ld(a2) if a2 is not None else 0, N.ptr(b2), _ld(b2) if b2 is not None else 0, K2,
           len(seg_end), N.int_array(seg_end), N.int_array(seg_col),
           N.ptr(out), _ld(out), N.ptr(residual), _ld(residual) if residual is not None else 0,
           N.ptr(gate), float(alpha), N.stream())
    return out


def gemm_tn(a: torch.Tensor, b: torch.Tensor, *, out: torch.Tensor | None = None,
            alpha: float = 1.0, beta: float = 0.0) -> torch.Tensor:
    """out[P,Q] (fp32) = beta * out + alpha * a[Mrows,P].T @ b[Mrows,Q] (split-K over rows)."""
    _rowmajor(a, "a")
    _rowmajor(b, "b")
    if a.shape[0] != b.shape[0] or a.dtype != b.dtype:
        raise RuntimeError("gemm_tn: operands must share rows and dtype")
    Mr, P = a.shape
    Q = b.shape[1]
    if out is None:
        out = torch.empty((P, Q), device=a.device, dtype=torch.float32)
        beta = 0.0
    _rowmajor(out, "out")
    if out.dtype != torch.float32 or tuple(out.shape) != (P, Q):
        raise RuntimeError("gemm_tn: out must be fp32 [P,Q]")
    ws_bytes = int(N.lib().unok_gemm_tn_workspace(Mr, P, Q))
    ws = torch.empty(max(ws_bytes // 4, 1), device=a.device, dtype=torch.float32)
    N.call("unok_gemm_tn", N.dtype_code(a.dtype), Mr, P, Q, N.ptr(a), _ld(a), N.ptr(b), _ld(b),
           N.ptr(out), _ld(out), float(alpha), float(beta), N.ptr(ws), ws_bytes, N.stream())
    return out
