"""Functional wrappers over the HIP kernel library (one per C-ABI entry point).

Every wrapper validates shapes and strides on the host, allocates outputs with torch (which
owns all device memory) and enqueues the kernel on torch's current stream. There is no
non-HIP code path.
"""
from __future__ import annotations

from typing import Sequence

import torch

from . import _native as N


class LaunchRecorder:
    """Brackets selected GEMM launches with HIP events (torch's current stream, which is the
    stream the kernels run on) to measure their live duration inside a timed region."""

    def __init__(self, predicate):
        self.predicate = predicate
        self.records = []   # (start_event, end_event, flops, (M, N, K, K2))

    def elapsed(self):
        torch.cuda.synchronize()
        ms = [r[0].elapsed_time(r[1]) for r in self.records]
        fl = [r[2] for r in self.records]
        return ms, fl

    def shapes(self):
        return [r[3] for r in self.records]


_recorder: LaunchRecorder | None = None


def set_recorder(rec: LaunchRecorder | None) -> None:
    global _recorder
    _recorder = rec


def nt_uses_256_tiles(M: int, N: int, seg_end, K: int = 0) -> bool:
    """Mirror of the tile choice in unok_gemm_nt for bf16 (the 256x256 MFMA kernel)."""
    if N <= 128:
        return False
    if any(e % 256 for e in list(seg_end)[:-1]):
        return False
    return ((M + 255) // 256) * ((N + 255) // 256) >= (192 if K >= 8192 else 256)


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
    rec = _recorder
    if rec is not None and rec.predicate(a.dtype, M, Nn, K, K2, seg_end):
        ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        ev0.record()
    else:
        rec = None
    N.call("unok_gemm_nt", N.dtype_code(a.dtype), N.dtype_code(out_dtype), M, Nn, K,
           N.ptr(a), _ld(a), N.ptr(b), _ld(b),
           N.ptr(a2), _ld(a2) if a2 is not None else 0, N.ptr(b2), _ld(b2) if b2 is not None else 0, K2,
           len(seg_end), N.int_array(seg_end), N.int_array(seg_col),
           N.ptr(out), _ld(out), N.ptr(residual), _ld(residual) if residual is not None else 0,
           N.ptr(gate), float(alpha), N.stream())
    if rec is not None:
        ev1.record()
        rec.records.append((ev0, ev1, 2.0 * M * Nn * (K + K2), (M, Nn, K, K2)))
    return out


def gemm_nt_rows(a: torch.Tensor, b: torch.Tensor, *, lora_a: torch.Tensor | None = None,
                 lora_b: torch.Tensor | None = None, segments: Sequence[tuple[int, int]] | None = None,
                 residual: torch.Tensor | None = None, gate: torch.Tensor | None = None,
                 swiglu: bool = False, splits: int = 0, out: torch.Tensor | None = None) -> torch.Tensor:
    """Few-row gated LoRA linear (decode and draft blocks), bf16:
    y = a b^T + h[:, seg] lora_b^T + residual with h = bf16(gate (.) a lora_a^T).

    a [M,K], b [N,K]; lora_a [R,K] (all segments' A rows), lora_b [N,r] ((alpha/r) B);
    ``segments`` is a list of (n_end, h_col) pairs: output columns < n_end (and >= the previous
    end) use h[:, h_col:h_col+r]. With ``swiglu`` the result is silu(G) * U of y = [G | U],
    [M, N/2]. ``splits`` = 0 lets the library choose the K ranges."""
    _rowmajor(a, "a")
    _rowmajor(b, "b")
    M, K = a.shape
    Nn = b.shape[0]
    if b.shape[1] != K or a.dtype != torch.bfloat16 or b.dtype != torch.bfloat16:
        raise RuntimeError(f"gemm_nt_rows: bf16 a [M,K] and b [N,K] required, got {tuple(a.shape)} {tuple(b.shape)}")
    R = r = 0
    seg_end, seg_col = [], []
    if lora_a is not None:
        _rowmajor(lora_a, "lora_a")
        _rowmajor(lora_b, "lora_b")
        if lora_a.dtype != a.dtype or lora_b.dtype != a.dtype or lora_a.shape[1] != K or lora_b.shape[0] != Nn:
            raise RuntimeError("gemm_nt_rows: LoRA operands must be bf16 lora_a [R,K] and lora_b [N,r]")
        R, r = lora_a.shape[0], lora_b.shape[1]
        segs = list(segments) if segments else [(Nn, 0)]
        seg_end = [s[0] for s in segs]
        seg_col = [s[1] for s in segs]
    ncol = Nn // 2 if swiglu else Nn
    if out is None:
        out = torch.empty((M, ncol), device=a.device, dtype=a.dtype)
    _rowmajor(out, "out")
    if tuple(out.shape) != (M, ncol) or out.dtype != a.dtype:
        raise RuntimeError("gemm_nt_rows: out has the wrong shape or dtype")
    if residual is not None:
        _rowmajor(residual, "residual")
        if swiglu or tuple(residual.shape) != (M, Nn) or residual.dtype != a.dtype:
            raise RuntimeError("gemm_nt_rows: residual must match out (and is not taken with swiglu)")
    if gate is not None:
        if gate.dtype not in (torch.bool, torch.uint8) or gate.numel() != M or not gate.is_contiguous():
            raise RuntimeError("gemm_nt_rows: gate must be a contiguous bool/uint8 vector of length M")
    epi = 1 if swiglu else 0
    nbytes = N.lib().unok_gemm_nt_rows_workspace(M, Nn, K, R, epi, int(splits))
    ws = torch.empty((nbytes + 3) // 4, device=a.device, dtype=torch.float32) if nbytes > 0 else None
    N.call("unok_gemm_nt_rows", M, Nn, K, N.ptr(a), _ld(a), N.ptr(b), _ld(b),
           N.ptr(lora_a), _ld(lora_a) if lora_a is not None else 0, R,
           N.ptr(lora_b), _ld(lora_b) if lora_b is not None else 0, r,
           len(seg_end), N.int_array(seg_end), N.int_array(seg_col),
           N.ptr(out), _ld(out), N.ptr(residual), _ld(residual) if residual is not None else 0,
           N.ptr(gate), epi, int(splits), N.ptr(ws), nbytes, N.stream())
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


def gemm_tn_noalloc(a: torch.Tensor, b: torch.Tensor, out: torch.Tensor, *, alpha: float = 1.0,
                    beta: float = 0.0) -> torch.Tensor:
    """As ``gemm_tn`` into an existing fp32 ``out``, with the split-K partials in the library's own
    per-device scratch array: nothing is allocated, by torch or by the library."""
    _rowmajor(a, "a")
    _rowmajor(b, "b")
    _rowmajor(out, "out")
    if a.shape[0] != b.shape[0] or a.dtype != b.dtype:
        raise RuntimeError("gemm_tn_noalloc: operands must share rows and dtype")
    Mr, P = a.shape
    Q = b.shape[1]
    if out.dtype != torch.float32 or tuple(out.shape) != (P, Q):
        raise RuntimeError("gemm_tn_noalloc: out must be fp32 [P,Q]")
    N.call("unok_gemm_tn_noalloc", N.dtype_code(a.dtype), Mr, P, Q, N.ptr(a), _ld(a), N.ptr(b), _ld(b),
           N.ptr(out), _ld(out), float(alpha), float(beta), N.stream())
    return out


# ------------------------------------------------------------------------------------------
# Row-wise kernels
# ------------------------------------------------------------------------------------------
def _contig(t: torch.Tensor, name: str) -> None:
    if not t.is_contiguous():
        raise RuntimeError(f"{name} must be contiguous")


def rmsnorm_fwd(x: torch.Tensor, w: torch.Tensor, eps: float, out: torch.Tensor | None = None):
    """y = round(x * rsqrt(mean(x^2) + eps) * w); returns (y, rstd[M] fp32)."""
    _rowmajor(x, "x")
    M, Hd = x.shape
    if w.numel() != Hd or w.dtype != x.dtype:
        raise RuntimeError("rmsnorm: weight must match the hidden size and dtype")
    y = out if out is not None else torch.empty((M, Hd), device=x.device, dtype=x.dtype)
    rstd = torch.empty(M, device=x.device, dtype=torch.float32)
    N.call("unok_rmsnorm_fwd", N.dtype_code(x.dtype), M, Hd, N.ptr(x), _ld(x), N.ptr(w), N.ptr(y), _ld(y),
           N.ptr(rstd), float(eps), N.stream())
    return y, rstd


def rmsnorm_bwd(dy, x, w, rstd, dres=None, out=None):
    """dx = rmsnorm backward (+ dres); ``out`` may alias ``dres``."""
    for t, n in ((dy, "dy"), (x, "x")):
        _contig(t, n)
    M, Hd = x.shape
    dx = out if out is not None else torch.empty_like(x)
    if dres is not None:
        _contig(dres, "dres")
    N.call("unok_rmsnorm_bwd", N.dtype_code(x.dtype), M, Hd, N.ptr(dy), N.ptr(x), N.ptr(w), N.ptr(rstd),
           N.ptr(dres), N.ptr(dx), N.stream())
    return dx


def qknorm_rope_fwd(qkv, nq, nk, d, wq, wk, pos, inv_freq, eps, *, out_dtype=None, with_v=False):
    """Per-head q/k RMSNorm (when wq/wk are given) then RoPE; returns (q, k, rstd), or (q, k, v, rstd)
    with ``with_v`` (v: the v heads of qkv as a contiguous [M, nk*d] copy). ``out_dtype`` (default:
    qkv's) may be bf16 for an fp32 qkv: the normalisation then sees the unrounded projection."""
    _rowmajor(qkv, "qkv")
    M = qkv.shape[0]
    out_dtype = out_dtype or qkv.dtype
    q = torch.empty((M, nq * d), device=qkv.device, dtype=out_dtype)
    k = torch.empty((M, nk * d), device=qkv.device, dtype=out_dtype)
    v = torch.empty((M, nk * d), device=qkv.device, dtype=out_dtype) if with_v else None
    rstd = torch.empty((M, nq + nk), device=qkv.device, dtype=torch.float32)
    if pos.dtype != torch.int64 or pos.numel() != M:
        raise RuntimeError("qknorm_rope: pos must be int64 [M]")
    N.call("unok_qknorm_rope_fwd", N.dtype_code(out_dtype), N.dtype_code(qkv.dtype), M, nq, nk, d, N.ptr(qkv),
           _ld(qkv), N.ptr(wq), N.ptr(wk), N.ptr(pos), N.ptr(inv_freq), float(eps), N.ptr(q), N.ptr(k), N.ptr(v),
           _ld(v) if v is not None else 0, N.ptr(rstd), N.stream())
    return (q, k, v, rstd) if with_v else (q, k, rstd)


def qknorm_rope_bwd(dq, dk, qkv, nq, nk, d, wq, wk, pos, inv_freq, rstd, dqkv):
    """Writes the q and k column blocks of ``dqkv`` ([M, (nq+2nk)*d]). dq and dk share a dtype,
    dqkv's or fp32; ``qkv`` holds the pre-norm q/k columns first (the projection output, or its q/k
    block alone) in that dtype, or in bf16 beside fp32 gradients."""
    _contig(dq, "dq")
    _contig(dk, "dk")
    if dq.dtype != dk.dtype:
        raise RuntimeError("qknorm_rope_bwd: dq and dk must share a dtype")
    M = qkv.shape[0]
    N.call("unok_qknorm_rope_bwd", N.dtype_code(dqkv.dtype), N.dtype_code(dq.dtype), N.dtype_code(qkv.dtype), M, nq,
           nk, d, N.ptr(dq), N.ptr(dk), N.ptr(qkv), _ld(qkv), N.ptr(wq), N.ptr(wk), N.ptr(pos), N.ptr(inv_freq),
           N.ptr(rstd), N.ptr(dqkv), _ld(dqkv), N.stream())
    return dqkv


def rope_table(P: int, inv_freq: torch.Tensor):
    """cos / sin [P, len(inv_freq)] of fl32(p * inv_freq[j]) for positions p < P."""
    half = inv_freq.numel()
    cos = torch.empty((P, half), device=inv_freq.device, dtype=torch.float32)
    sin = torch.empty((P, half), device=inv_freq.device, dtype=torch.float32)
    N.call("unok_rope_table", P, half, N.ptr(inv_freq), N.ptr(cos), N.ptr(sin), N.stream())
    return cos, sin


def qkv_rope_fused_ok(M: int, K: int, K2: int, nq: int, nk: int, d: int, dtype) -> bool:
    """Whether gemm_nt_qkv_rope takes this q|k|v projection (the 256 x 256 kernel's shapes)."""
    return (dtype == torch.bfloat16 and d == 128 and M % 256 == 0 and (128 * (nq + 2 * nk)) % 256 == 0
            and K % 64 == 0 and K2 % 32 == 0 and M * (nq + 2 * nk) >= 256 * 2)


def gemm_nt_qkv_rope(x, w_qkv, nq, nk, wq, wk, pos, cos_tab, sin_tab, eps, *, a2=None, b2=None, segments=None,
                     want_rstd=True, want_pre=False):
    """q|k|v projection (+ LoRA extension) with q/k RMSNorm + RoPE in the GEMM epilogue (bf16, head dim
    128). Returns (q, k, v, rstd or None, pre or None); ``pre`` = the pre-norm q/k columns in bf16."""
    _rowmajor(x, "x")
    _rowmajor(w_qkv, "w_qkv")
    M, Kd = x.shape
    if w_qkv.shape != (128 * (nq + 2 * nk), Kd):
        raise RuntimeError("gemm_nt_qkv_rope: w_qkv must be [128 (nq + 2 nk), K]")
    K2 = 0
    seg_end, seg_col = [], []
    if a2 is not None:
        _rowmajor(a2, "a2")
        _rowmajor(b2, "b2")
        K2 = b2.shape[1]
        segs = list(segments) if segments else [(w_qkv.shape[0], 0)]
        for _, col in segs:
            if col + K2 > a2.shape[1]:
                raise RuntimeError("gemm_nt_qkv_rope: extension segment exceeds a2 columns")
        seg_end = [s[0] for s in segs]
        seg_col = [s[1] for s in segs]
    if not qkv_rope_fused_ok(M, Kd, K2, nq, nk, 128, x.dtype):
        raise RuntimeError("gemm_nt_qkv_rope: shape outside the fused kernel")
    if pos.dtype != torch.int64 or pos.numel() != M:
        raise RuntimeError("gemm_nt_qkv_rope: pos must be int64 [M]")
    e = dict(device=x.device, dtype=x.dtype)
    q = torch.empty((M, 128 * nq), **e)
    k = torch.empty((M, 128 * nk), **e)
    v = torch.empty((M, 128 * nk), **e)
    rstd = torch.empty((M, nq + nk), device=x.device, dtype=torch.float32) if want_rstd else None
    pre = torch.empty((M, 128 * (nq + nk)), **e) if want_pre else None
    Nn = w_qkv.shape[0]
    rec = _recorder
    if rec is not None and rec.predicate(x.dtype, M, Nn, Kd, K2, seg_end or [Nn]):
        ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        ev0.record()
    else:
        rec = None
    N.call("unok_gemm_nt_qkv_rope", M, Kd, nq, nk, N.ptr(x), _ld(x), N.ptr(w_qkv), _ld(w_qkv), N.ptr(a2),
           _ld(a2) if a2 is not None else 0, N.ptr(b2), _ld(b2) if b2 is not None else 0, K2, len(seg_end),
           N.int_array(seg_end), N.int_array(seg_col), N.ptr(wq), N.ptr(wk), N.ptr(pos), N.ptr(cos_tab),
           N.ptr(sin_tab), cos_tab.shape[0], float(eps), N.ptr(q), N.ptr(k), N.ptr(v), N.ptr(rstd), N.ptr(pre),
           N.stream())
    if rec is not None:
        ev1.record()
        rec.records.append((ev0, ev1, 2.0 * M * Nn * (Kd + K2), (M, Nn, Kd, K2)))
    return q, k, v, rstd, pre


def gemm_nt_swiglu(a: torch.Tensor, b_interleaved: torch.Tensor, *, a2: torch.Tensor | None = None,
                   b2_interleaved: torch.Tensor | None = None, gu: torch.Tensor | None = None,
                   out: torch.Tensor | None = None) -> torch.Tensor:
    """silu(gate) * up of a @ b.T (+ a2 @ b2.T) for gate/up weight rows interleaved in blocks of 64
    (``interleave_gate_up``; b2 likewise); bf16, M and the row count of b multiples of 256, K and
    K2 = b2.shape[1] of 32. With ``gu`` ([M, rows]), also stores the product as [gate | up]."""
    _rowmajor(a, "a")
    _rowmajor(b_interleaved, "b")
    M, K = a.shape
    rows = b_interleaved.shape[0]
    if b_interleaved.shape[1] != K or a.dtype != torch.bfloat16 or b_interleaved.dtype != torch.bfloat16:
        raise RuntimeError("gemm_nt_swiglu: bf16 a [M,K] and b [N,K] required")
    K2 = 0
    if a2 is not None:
        _rowmajor(a2, "a2")
        _rowmajor(b2_interleaved, "b2")
        K2 = b2_interleaved.shape[1]
        if b2_interleaved.shape[0] != rows or a2.shape[0] != M or a2.shape[1] < K2:
            raise RuntimeError("gemm_nt_swiglu: a2 [M,>=K2] and b2 [N,K2] required")
    if gu is not None:
        _rowmajor(gu, "gu")
        if tuple(gu.shape) != (M, rows) or gu.dtype != a.dtype:
            raise RuntimeError("gemm_nt_swiglu: gu must be [M, N] in the dtype of a")
    out = out if out is not None else torch.empty((M, rows // 2), device=a.device, dtype=a.dtype)
    _rowmajor(out, "out")
    rec = _recorder
    if rec is not None and rec.predicate(a.dtype, M, rows, K, K2, [rows]):
        ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        ev0.record()
    else:
        rec = None
    N.call("unok_gemm_nt_swiglu", M, rows, K, N.ptr(a), _ld(a), N.ptr(b_interleaved), _ld(b_interleaved),
           N.ptr(a2), _ld(a2) if a2 is not None else 0, N.ptr(b2_interleaved),
           _ld(b2_interleaved) if b2_interleaved is not None else 0, K2,
           N.ptr(out), _ld(out), N.ptr(gu), _ld(gu) if gu is not None else 0, N.stream())
    if rec is not None:
        ev1.record()
        rec.records.append((ev0, ev1, 2.0 * M * rows * (K + K2), (M, rows, K, K2)))
    return out


def gemm_nt_swiglu_bwd(a: torch.Tensor, b: torch.Tensor, a2: torch.Tensor | None, b2: torch.Tensor | None,
                       gu: torch.Tensor, dgu: torch.Tensor | None = None) -> torch.Tensor:
    """dgu = SwiGLU backward of dS = a @ b.T (+ a2 @ b2.T) against gu = [gate | up]; dS is never
    stored. bf16; M and F = b.shape[0] multiples of 256."""
    for t, n in ((a, "a"), (b, "b"), (gu, "gu")):
        _rowmajor(t, n)
    M, K = a.shape
    F = b.shape[0]
    if b.shape[1] != K or tuple(gu.shape) != (M, 2 * F):
        raise RuntimeError("gemm_nt_swiglu_bwd: a [M,K], b [F,K] and gu [M,2F] required")
    K2 = 0
    if a2 is not None:
        _rowmajor(a2, "a2")
        _rowmajor(b2, "b2")
        K2 = b2.shape[1]
        if b2.shape[0] != F or a2.shape[0] != M or a2.shape[1] < K2:
            raise RuntimeError("gemm_nt_swiglu_bwd: a2 [M,>=K2] and b2 [F,K2] required")
    dgu = dgu if dgu is not None else torch.empty((M, 2 * F), device=a.device, dtype=a.dtype)
    _rowmajor(dgu, "dgu")
    rec = _recorder
    if rec is not None and rec.predicate(a.dtype, M, F, K, K2, [F]):
        ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        ev0.record()
    else:
        rec = None
    N.call("unok_gemm_nt_swiglu_bwd", M, F, K, N.ptr(a), _ld(a), N.ptr(b), _ld(b), N.ptr(a2),
           _ld(a2) if a2 is not None else 0, N.ptr(b2), _ld(b2) if b2 is not None else 0, K2, N.ptr(gu), _ld(gu),
           N.ptr(dgu), _ld(dgu), N.stream())
    if rec is not None:
        ev1.record()
        rec.records.append((ev0, ev1, 2.0 * M * F * (K + K2), (M, F, K, K2)))
    return dgu


def swiglu_fused_ok(M: int, F: int, K: int) -> bool:
    """Shapes the fused gate/up + SwiGLU product accepts."""
    return M % 256 == 0 and (2 * F) % 256 == 0 and K % 64 == 0 and K > 0


def interleave_gate_up(w_gu: torch.Tensor, F: int) -> torch.Tensor:
    """[gate; up] rows [2F, H] -> rows interleaved in blocks of 64 (gate 64 b.., then up 64 b..)."""
    H = w_gu.shape[1]
    g, u = w_gu[:F].reshape(F // 64, 64, H), w_gu[F:].reshape(F // 64, 64, H)
    return torch.stack((g, u), dim=1).reshape(2 * F, H).contiguous()


def swiglu_fwd(gu, F, out=None):
    _rowmajor(gu, "gu")
    M = gu.shape[0]
    out = out if out is not None else torch.empty((M, F), device=gu.device, dtype=gu.dtype)
    N.call("unok_swiglu_fwd", N.dtype_code(gu.dtype), M, F, N.ptr(gu), _ld(gu), N.ptr(out), N.stream())
    return out


def swiglu_bwd(dout, gu, F, dgu=None):
    _contig(dout, "dout")
    M = gu.shape[0]
    dgu = dgu if dgu is not None else torch.empty((M, 2 * F), device=gu.device, dtype=gu.dtype)
    N.call("unok_swiglu_bwd", N.dtype_code(gu.dtype), M, F, N.ptr(dout), N.ptr(gu), _ld(gu), N.ptr(dgu),
           _ld(dgu), N.stream())
    return dgu


def embedding(ids: torch.Tensor, table: torch.Tensor, out=None):
    if ids.dtype != torch.int64 or not ids.is_contiguous():
        raise RuntimeError("embedding: ids must be contiguous int64")
    _contig(table, "table")
    M = ids.numel()
    out = out if out is not None else torch.empty((M, table.shape[1]), device=table.device, dtype=table.dtype)
    N.call("unok_embedding", table.element_size(), M, table.shape[1], N.ptr(ids), N.ptr(table), table.shape[0],
           N.ptr(out), N.stream())
    return out


def rows_copy(src: torch.Tensor, dst: torch.Tensor, M: int, smap=None, dmap=None):
    """dst[dmap[r]] = src[smap[r]] for r < M (maps are int32; None = identity)."""
    _rowmajor(src, "src")
    _rowmajor(dst, "dst")
    if src.dtype != dst.dtype or src.shape[1] != dst.shape[1]:
        raise RuntimeError("rows_copy: src and dst rows differ")
    for m in (smap, dmap):
        if m is not None and (m.dtype != torch.int32 or m.numel() < M):
            raise RuntimeError("rows_copy: maps must be int32 with >= M entries")
    es = src.element_size()
    N.call("unok_rows_copy", src.shape[1] * es, M, N.ptr(src), _ld(src) * es, N.ptr(smap), N.ptr(dst),
           _ld(dst) * es, N.ptr(dmap), N.stream())
    return dst


# ------------------------------------------------------------------------------------------
# Block-diffusion attention
# ------------------------------------------------------------------------------------------
def attn_fwd(q, k1, v1, iv, Hq, Hkv, D, *, k2=None, v2=None, scale=None):
    """Returns (O [Mq, Hq*D], LSE2 [Mq, Hq] fp32 = log2-sum-exp2 of the scaled scores)."""
    _rowmajor(q, "q")
    Mq = q.shape[0]
    scale = D ** -0.5 if scale is None else scale
    if iv.dtype != torch.int32 or tuple(iv.shape) != (Mq, 8):
        raise RuntimeError("attn_fwd: interval table must be int32 [Mq, 8]")
    o = torch.empty((Mq, Hq * D), device=q.device, dtype=q.dtype)
    lse = torch.empty((Mq, Hq), device=q.device, dtype=torch.float32)
    N.call("unok_attn_fwd", N.dtype_code(q.dtype), Mq, Hq, Hkv, D, N.ptr(q), _ld(q), N.ptr(k1), _ld(k1),
           N.ptr(v1), _ld(v1), N.ptr(k2), _ld(k2) if k2 is not None else 0, N.ptr(v2),
           _ld(v2) if v2 is not None else 0, N.ptr(iv), N.ptr(o), _ld(o), N.ptr(lse), float(scale), N.stream())
    return o, lse


def attn_fwd_split(q, k, v, iv, QR: int, S: int, D: int, *, scale=None):
    """Split-key attention of decode blocks: S * QR rows, row i reading query q[i % QR] (one head)
    against k / v rows over its interval iv[i]; returns (O [S*QR, D], LSE2 [S*QR] fp32)."""
    for t, nm in ((q, "q"), (k, "k"), (v, "v")):
        _rowmajor(t, nm)
    scale = D ** -0.5 if scale is None else scale
    rows = QR * S
    if iv.dtype != torch.int32 or tuple(iv.shape) != (rows, 8) or q.shape[0] < QR:
        raise RuntimeError("attn_fwd_split: int32 iv [S*QR, 8] and q [>= QR, D] required")
    o = torch.empty((rows, D), device=q.device, dtype=q.dtype)
    lse = torch.empty(rows, device=q.device, dtype=torch.float32)
    N.call("unok_attn_fwd_split", QR, S, D, N.ptr(q), _ld(q), N.ptr(k), _ld(k), N.ptr(v), _ld(v), N.ptr(iv),
           N.ptr(o), _ld(o), N.ptr(lse), float(scale), N.stream())
    return o, lse


def attn_split_combine(o, lse, dst, QR: int, S: int, D: int, out):
    """out[dst[i]] = merge of the S partial rows s * QR + i (rows with dst[i] < 0 skipped)."""
    _rowmajor(o, "o")
    _rowmajor(out, "out")
    if dst.dtype != torch.int32 or dst.numel() < QR or lse.numel() < QR * S:
        raise RuntimeError("attn_split_combine: int32 dst [QR] and lse [S*QR] required")
    N.call("unok_attn_split_combine", QR, S, D, N.ptr(o), _ld(o), N.ptr(lse), N.ptr(dst), N.ptr(out), _ld(out),
           N.stream())
    return out


def decode_prep(qkv, wq, wk, lengths, inv_freq, eps: float, kc, vc, qd, B: int, L: int, nq: int, nk: int, D: int):
    """q/k norm + RoPE of a draft block's qkv rows [B*L, (nq+2nk)*D], its K/V rows into the caches
    kc / vc [B, nk, max_len, D] at the committed lengths, its queries into qd [B*nk*128, D]."""
    _rowmajor(qkv, "qkv")
    if qkv.dtype != torch.bfloat16 or lengths.dtype != torch.int64 or not kc.is_contiguous() or not vc.is_contiguous():
        raise RuntimeError("decode_prep: bf16 qkv, int64 lengths and contiguous caches required")
    N.call("unok_decode_prep", B, L, nq, nk, D, N.ptr(qkv), _ld(qkv), N.ptr(wq), N.ptr(wk), N.ptr(lengths),
           N.ptr(inv_freq), float(eps), N.ptr(kc), N.ptr(vc), kc.shape[2], N.ptr(qd), N.stream())
    return qd


def attn_bwd_qknorm(q, k1, v1, iv, o, lse, do, Hq, Hkv, D, k2, v2, pre, rstd, wq, wk, pos, cos_tab, sin_tab, dqkv,
                    scale=None):
    """Noisy-stream backward with the q/k RMSNorm + RoPE backward in the dQ / dK epilogues (bf16): writes
    the gradient before the norm into the q and k column blocks of ``dqkv`` and dV into its v block."""
    Mq = q.shape[0]
    scale = D ** -0.5 if scale is None else scale
    _contig(do, "do")
    _rowmajor(pre, "pre")
    _rowmajor(dqkv, "dqkv")
    if q.dtype != torch.bfloat16 or pre.dtype != torch.bfloat16 or dqkv.dtype != torch.bfloat16:
        raise RuntimeError("attn_bwd_qknorm: bf16 only")
    if pre.shape != (Mq, (Hq + Hkv) * D) or dqkv.shape != (Mq, (Hq + 2 * Hkv) * D) or k2.shape[0] != Mq:
        raise RuntimeError("attn_bwd_qknorm: pre [Mq, (Hq+Hkv) D], dqkv [Mq, (Hq+2Hkv) D] and Mq keys required")
    if pos.dtype != torch.int64 or pos.numel() != Mq:
        raise RuntimeError("attn_bwd_qknorm: pos must be int64 [Mq]")
    dsum = torch.empty((Mq, Hq), device=q.device, dtype=torch.float32)
    N.call("unok_attn_bwd_qknorm", Mq, Hq, Hkv, D, N.ptr(q), _ld(q), N.ptr(k1), _ld(k1), N.ptr(v1), _ld(v1),
           N.ptr(k2), _ld(k2), N.ptr(v2), _ld(v2), N.ptr(iv), N.ptr(o), _ld(o), N.ptr(lse), N.ptr(do), _ld(do),
           N.ptr(dsum), N.ptr(pre), _ld(pre), N.ptr(rstd), N.ptr(wq), N.ptr(wk), N.ptr(pos), N.ptr(cos_tab),
           N.ptr(sin_tab), cos_tab.shape[0], N.ptr(dqkv), _ld(dqkv), float(scale), N.stream())
    return dqkv


def attn_bwd(q, k1, v1, iv, o, lse, do, Hq, Hkv, D, *, k2=None, v2=None, ivk=None, dk=None, dv=None,
             scale=None, grad_dtype=None):
    """Returns dQ; writes dK/dV of source-2 keys into ``dk``/``dv`` when given. ``grad_dtype`` (default
    q's) is the dtype of dQ and dK, fp32 allowed for bf16 inputs; dV has q's dtype."""
    Mq = q.shape[0]
    scale = D ** -0.5 if scale is None else scale
    grad_dtype = grad_dtype or q.dtype
    _contig(do, "do")
    if dk is not None and dk.dtype != grad_dtype:
        raise RuntimeError("attn_bwd: dk must have the gradient dtype")
    dq = torch.empty((Mq, Hq * D), device=q.device, dtype=grad_dtype)
    dsum = torch.empty((Mq, Hq), device=q.device, dtype=torch.float32)
    Mk2 = k2.shape[0] if k2 is not None else 0
    N.call("unok_attn_bwd", N.dtype_code(q.dtype), N.dtype_code(grad_dtype), Mq, Mk2, Hq, Hkv, D, N.ptr(q), _ld(q),
           N.ptr(k1), _ld(k1),
           N.ptr(v1), _ld(v1), N.ptr(k2), _ld(k2) if k2 is not None else 0, N.ptr(v2),
           _ld(v2) if v2 is not None else 0, N.ptr(iv), N.ptr(ivk), N.ptr(o), _ld(o), N.ptr(lse), N.ptr(do),
           _ld(do), N.ptr(dsum), N.ptr(dq), _ld(dq), N.ptr(dk), _ld(dk) if dk is not None else 0, N.ptr(dv),
           _ld(dv) if dv is not None else 0, float(scale), N.stream())
    return dq
