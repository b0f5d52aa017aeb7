"""LM-head objectives of the Uno step on the HIP kernels.

* ``fused_weighted_ce``: CE with the diffusion 1/t weighting (training/trainer.py:267-283). In
  bf16 the LM-head GEMM's epilogue reduces each 128-column block of logits to per-row softmax
  statistics and picks the target logit; it also stores the rows' fp32 logits when they fit
  CE_STORED_LOGITS_MAX_BYTES, and the backward then forms dz = g w (softmax - onehot) from them one
  vocabulary chunk at a time. Above that size the forward stores no logits and the backward
  recomputes them chunk by chunk in a GEMM whose epilogue emits dz. Either way dz passes through
  one [rows x chunk] bf16 buffer into the data-gradient GEMM.
* ``teacher_argmax``: first-index argmax of the clean-stream logits, chunked the same way
  (training/losses.py:38-56, target source "clean_argmax").
* ``distribution_losses``: reverse KL and total variation (training/losses.py:59-183) over
  bf16 logits of the supervised rows, fp32 per-row statistics, with hand-written backward.
"""
from __future__ import annotations

import torch

from . import _native as N
from . import kernels as K

# Vocabulary columns per chunk of the CE backward (and of the fp32 / argmax chunk buffers).
DEFAULT_CE_CHUNK = 32768
# The bf16 CE keeps the LM-head logits of its rows (fp32) from the forward for the backward when
# they take at most this many bytes; beyond it the backward recomputes them inside its GEMM.
CE_STORED_LOGITS_MAX_BYTES = 6 << 30


def lm_head_logits(lm_head, x: torch.Tensor) -> torch.Tensor:
    """Plain logits (used by project_hidden_states); differentiable w.r.t. x."""
    shape = x.shape
    out = _Logits.apply(x.reshape(-1, shape[-1]), lm_head.weight, lm_head.weight_t)
    return out.view(*shape[:-1], lm_head.weight.shape[0])


class _Logits(torch.autograd.Function):
    @staticmethod
    def forward(ctx, x, w, w_t):
        x = x.contiguous()
        ctx.w_t = w_t
        return K.gemm_nt(x, w)

    @staticmethod
    def backward(ctx, dz):
        return K.gemm_nt(dz.contiguous(), ctx.w_t), None, None


def _chunks(V: int, chunk: int):
    for c0 in range(0, V, chunk):
        yield c0, min(V, c0 + chunk)


def _fused_ce_ok(h: torch.Tensor, w_lm: torch.Tensor) -> bool:
    """The GEMM-epilogue path: bf16, K a multiple of 64, and a vocabulary whose chunk ends keep the
    data-gradient GEMM's 8-element K granularity."""
    return (h.dtype == torch.bfloat16 and w_lm.dtype == torch.bfloat16 and h.shape[1] % 64 == 0
            and w_lm.shape[0] % 8 == 0 and w_lm.stride(1) == 1)


class ChunkedWeightedCE(torch.autograd.Function):
    """loss = inv_n * sum_r w_r * CE(h_r W^T, y_r); inv_n is a device scalar.

    bf16 (the step): the forward is one LM-head GEMM whose epilogue keeps per-row softmax
    statistics per 128 vocabulary columns and the target logit. When the rows' fp32 logits fit
    CE_STORED_LOGITS_MAX_BYTES, the same epilogue also stores them and the backward forms dz
    (bf16, one [rows x chunk] buffer) from them with a row kernel, chunk by chunk; otherwise it
    recomputes the logits inside a GEMM whose epilogue writes dz. Both give the same dz bit for
    bit (the same logits, the same arithmetic), which feeds the data-gradient GEMM.
    fp32 (parity mode) and other shapes: the logits of one vocabulary chunk at a time go through a
    chunk buffer and the row kernels, recomputed in the backward."""

    @staticmethod
    def forward(ctx, h, w_lm, w_lm_t, targets, weights, inv_n, chunk):
        h = h.contiguous()
        R, V = h.shape[0], w_lm.shape[0]
        dev = h.device
        f32 = dict(device=dev, dtype=torch.float32)
        run_max, run_sum, zt = torch.empty(R, **f32), torch.empty(R, **f32), torch.zeros(R, **f32)
        lse = torch.empty(R, **f32)
        loss = torch.empty((), **f32)
        fused = _fused_ce_ok(h, w_lm)
        z_all = None
        if fused:
            nparts = (V + 127) // 128
            pmax, psum = torch.empty((R, nparts), **f32), torch.empty((R, nparts), **f32)
            if V % 4 == 0 and R * V * 4 <= CE_STORED_LOGITS_MAX_BYTES:
                z_all = torch.empty((R, V), **f32)
            N.call("unok_lmhead_ce_stats", R, V, h.shape[1], N.ptr(h), h.stride(0), N.ptr(w_lm), w_lm.stride(0),
                   N.ptr(targets), 0, N.ptr(pmax), N.ptr(psum), nparts, N.ptr(zt), N.ptr(z_all), V, N.stream())
            N.call("unok_ce_parts_reduce", R, nparts, N.ptr(pmax), N.ptr(psum), nparts, N.ptr(run_max),
                   N.ptr(run_sum), N.stream())
            del pmax, psum
        else:
            buf = torch.empty((R, min(chunk, V)), **f32)
            for i, (c0, c1) in enumerate(_chunks(V, chunk)):
                z = buf[:, :c1 - c0]
                K.gemm_nt(h, w_lm[c0:c1], out=z)
                N.call("unok_row_lse_update", N.F32, R, c1 - c0, N.ptr(z), buf.stride(0), c0, N.ptr(targets),
                       N.ptr(run_max), N.ptr(run_sum), N.ptr(zt), int(i == 0), N.stream())
            del buf
        N.call("unok_ce_finish", R, N.ptr(run_max), N.ptr(run_sum), N.ptr(zt), N.ptr(weights), N.ptr(inv_n),
               N.ptr(lse), N.ptr(loss), N.stream())
        ctx.save = (h, w_lm, w_lm_t, targets, weights, inv_n, lse, chunk, fused, z_all)
        return loss

    @staticmethod
    def backward(ctx, g):
        h, w_lm, w_lm_t, targets, weights, inv_n, lse, chunk, fused, z_all = ctx.save
        ctx.save = None
        R, V = h.shape[0], w_lm.shape[0]
        g = g.reshape(1).float().contiguous()
        f32 = dict(device=h.device, dtype=torch.float32)
        width = min(chunk, V)
        dz = torch.empty((R, (width + 7) // 8 * 8), device=h.device, dtype=h.dtype)
        dh = torch.zeros(h.shape, **f32)
        buf = None if fused else torch.empty((R, width), **f32)
        for c0, c1 in _chunks(V, chunk):
            d = dz[:, :c1 - c0]
            if z_all is not None:
                N.call("unok_ce_grad_chunk", N.dtype_code(h.dtype), R, c1 - c0, N.ptr(z_all[:, c0:]), z_all.stride(0),
                       c0, N.ptr(lse), N.ptr(targets), N.ptr(weights), N.ptr(g), N.ptr(inv_n), N.ptr(d), dz.stride(0),
                       N.stream())
            elif fused:
                N.call("unok_lmhead_ce_grad", R, c1 - c0, h.shape[1], N.ptr(h), h.stride(0), N.ptr(w_lm[c0:c1]),
                       w_lm.stride(0), N.ptr(targets), c0, N.ptr(lse), N.ptr(weights), N.ptr(g), N.ptr(inv_n),
                       N.ptr(dz), dz.stride(0), N.stream())
            else:
                z = buf[:, :c1 - c0]
                K.gemm_nt(h, w_lm[c0:c1], out=z)
                N.call("unok_ce_grad_chunk", N.dtype_code(h.dtype), R, c1 - c0, N.ptr(z), buf.stride(0), c0,
                       N.ptr(lse), N.ptr(targets), N.ptr(weights), N.ptr(g), N.ptr(inv_n), N.ptr(d), dz.stride(0),
                       N.stream())
            K.gemm_nt(d, w_lm_t[:, c0:c1], out=dh, residual=dh)
        return dh.to(h.dtype), None, None, None, None, None, None


def fused_weighted_ce(lm_head, h_rows: torch.Tensor, targets: torch.Tensor, weights: torch.Tensor,
                      inv_n: torch.Tensor, chunk: int = DEFAULT_CE_CHUNK) -> torch.Tensor:
    if h_rows.shape[0] == 0:
        return h_rows.sum() * 0.0
    return ChunkedWeightedCE.apply(h_rows, lm_head.weight, lm_head.weight_t, targets.contiguous(),
                                   weights.contiguous().float(), inv_n, chunk)


@torch.no_grad()
def teacher_argmax(lm_head, h_rows: torch.Tensor, chunk: int = DEFAULT_CE_CHUNK) -> torch.Tensor:
    R, V = h_rows.shape[0], lm_head.weight.shape[0]
    h_rows = h_rows.contiguous()
    best_val = torch.empty(R, device=h_rows.device, dtype=torch.float32)
    best_idx = torch.empty(R, device=h_rows.device, dtype=torch.int64)
    if R == 0:
        return best_idx
    buf = torch.empty((R, min(chunk, V)), device=h_rows.device, dtype=h_rows.dtype)
    for i, (c0, c1) in enumerate(_chunks(V, chunk)):
        z = buf[:, :c1 - c0]
        K.gemm_nt(h_rows, lm_head.weight[c0:c1], out=z)
        N.call("unok_row_argmax_update", N.dtype_code(z.dtype), R, c1 - c0, N.ptr(z), buf.stride(0), c0,
               N.ptr(best_val), N.ptr(best_idx), int(i == 0), N.stream())
    return best_idx


@torch.no_grad()
def logits_argmax(z: torch.Tensor) -> torch.Tensor:
    """First-index argmax of each row of given [R, V] logits (fp32 or bf16) on the argmax kernel."""
    if z.dim() != 2:
        raise RuntimeError(f"logits must be [rows, vocab], got {tuple(z.shape)}")
    if z.shape[1] > 1 and z.stride(1) != 1:
        z = z.contiguous()
    R, V = z.shape
    best_val = torch.empty(R, device=z.device, dtype=torch.float32)
    best_idx = torch.empty(R, device=z.device, dtype=torch.int64)
    if R:
        N.call("unok_row_argmax_update", N.dtype_code(z.dtype), R, V, N.ptr(z), z.stride(0) if R > 1 else V, 0,
               N.ptr(best_val), N.ptr(best_idx), 1, N.stream())
    return best_idx


class DistributionLoss(torch.autograd.Function):
    """kind 'tv': sum |p_s - p_t| * inv_n;  kind 'kl': sum p_s (log p_s - log p_t) * inv_n.
    Student logits are computed from h_s (differentiable), teacher logits from h_t (detached)."""

    @staticmethod
    def forward(ctx, h_s, h_t, w_lm, w_lm_t, inv_n, kind):
        h_s, h_t = h_s.contiguous(), h_t.contiguous()
        R, V = h_s.shape[0], w_lm.shape[0]
        zs = K.gemm_nt(h_s, w_lm)
        zt = K.gemm_nt(h_t, w_lm)
        f32 = dict(device=h_s.device, dtype=torch.float32)
        ms, ss, mt, st = (torch.empty(R, **f32) for _ in range(4))
        dt = N.dtype_code(zs.dtype)
        N.call("unok_softmax_stats", dt, R, V, N.ptr(zs), V, N.ptr(ms), N.ptr(ss), N.stream())
        N.call("unok_softmax_stats", dt, R, V, N.ptr(zt), V, N.ptr(mt), N.ptr(st), N.stream())
        rows = torch.empty(R, **f32)
        extra = torch.empty(R, **f32)
        if kind == "tv":
            N.call("unok_tv_fwd", dt, R, V, N.ptr(zs), V, N.ptr(zt), V, N.ptr(ms), N.ptr(ss), N.ptr(mt), N.ptr(st),
                   N.ptr(rows), N.ptr(extra), N.stream())
        elif kind == "kl":
            N.call("unok_kl_fwd", dt, R, V, N.ptr(zs), V, N.ptr(zt), V, N.ptr(ms), N.ptr(ss), N.ptr(mt), N.ptr(st),
                   N.ptr(rows), N.stream())
            extra = rows
        else:
            raise ValueError(kind)
        loss = torch.empty((), **f32)
        N.call("unok_sum_scaled", R, N.ptr(rows), N.ptr(inv_n), N.ptr(loss), N.stream())
        ctx.save = (zs, zt, ms, ss, mt, st, extra, inv_n, w_lm_t, kind)
        return loss

    @staticmethod
    def backward(ctx, g):
        zs, zt, ms, ss, mt, st, extra, inv_n, w_lm_t, kind = ctx.save
        ctx.save = None
        R, V = zs.shape
        g = g.reshape(1).float().contiguous()
        dt = N.dtype_code(zs.dtype)
        fn = "unok_tv_bwd" if kind == "tv" else "unok_kl_bwd"
        N.call(fn, dt, R, V, N.ptr(zs), V, N.ptr(zt), V, N.ptr(ms), N.ptr(ss), N.ptr(mt), N.ptr(st), N.ptr(extra),
               N.ptr(g), N.ptr(inv_n), N.ptr(zs), V, N.stream())
        dh = K.gemm_nt(zs, w_lm_t)
        return dh, None, None, None, None, None


def distribution_loss(lm_head, h_s, h_t, inv_n, kind: str) -> torch.Tensor:
    if h_s.shape[0] == 0:
        return h_s.sum() * 0.0
    return DistributionLoss.apply(h_s, h_t.detach(), lm_head.weight, lm_head.weight_t, inv_n, kind)


class LogitsDistributionLoss(torch.autograd.Function):
    """TV / reverse KL over given logits (the losses.py call surface); gradient w.r.t. student."""

    @staticmethod
    def forward(ctx, zs, zt, inv_n, kind):
        zs, zt = zs.contiguous(), zt.contiguous()
        R, V = zs.shape
        f32 = dict(device=zs.device, dtype=torch.float32)
        ms, ss, mt, st = (torch.empty(R, **f32) for _ in range(4))
        dt = N.dtype_code(zs.dtype)
        if zt.dtype != zs.dtype:
            raise RuntimeError("student and teacher logits must share a dtype")
        N.call("unok_softmax_stats", dt, R, V, N.ptr(zs), V, N.ptr(ms), N.ptr(ss), N.stream())
        N.call("unok_softmax_stats", dt, R, V, N.ptr(zt), V, N.ptr(mt), N.ptr(st), N.stream())
        rows, extra = torch.empty(R, **f32), torch.empty(R, **f32)
        if kind == "tv":
            N.call("unok_tv_fwd", dt, R, V, N.ptr(zs), V, N.ptr(zt), V, N.ptr(ms), N.ptr(ss), N.ptr(mt), N.ptr(st),
                   N.ptr(rows), N.ptr(extra), N.stream())
        else:
            N.call("unok_kl_fwd", dt, R, V, N.ptr(zs), V, N.ptr(zt), V, N.ptr(ms), N.ptr(ss), N.ptr(mt), N.ptr(st),
                   N.ptr(rows), N.stream())
            extra = rows
        loss = torch.empty((), **f32)
        N.call("unok_sum_scaled", R, N.ptr(rows), N.ptr(inv_n), N.ptr(loss), N.stream())
        ctx.save = (zs, zt, ms, ss, mt, st, extra, inv_n, kind)
        return loss

    @staticmethod
    def backward(ctx, g):
        zs, zt, ms, ss, mt, st, extra, inv_n, kind = ctx.save
        ctx.save = None
        R, V = zs.shape
        g = g.reshape(1).float().contiguous()
        grad = torch.empty_like(zs)
        fn = "unok_tv_bwd" if kind == "tv" else "unok_kl_bwd"
        N.call(fn, N.dtype_code(zs.dtype), R, V, N.ptr(zs), V, N.ptr(zt), V, N.ptr(ms), N.ptr(ss), N.ptr(mt),
               N.ptr(st), N.ptr(extra), N.ptr(g), N.ptr(inv_n), N.ptr(grad), V, N.stream())
        return grad, None, None, None
