"""Decoder-layer math of the conditional-LoRA block-diffusion step on the HIP kernels.

The reference runs one transformer pass over 2L rows per sequence ([noisy | clean] per
segment, training/modeling.py:65-81, 116-147) with LoRA gated to the noisy rows
(training/lora.py:164-174) and back-propagates through all 2L rows. Here the two streams are
computed separately, which is exact for this mask and gate:

* the clean stream has LoRA off and attends only to clean keys (causal), so it does not
  depend on the LoRA weights: it runs forward-only and keeps only its per-layer K/V;
* the noisy stream (LoRA on) attends to the clean K/V of strictly earlier blocks plus its own
  block; it is the only stream with a backward pass. Each noisy decoder layer is one
  autograd Function whose backward drives the fused kernels and accumulates the LoRA
  gradients straight into the flat gradient buffer of the adapter (see adapter.LoraState).

Per layer (x = RMSNorm(h)):  q|k|v = x W_qkv^T + s B (x A)   -> q/k RMSNorm + RoPE
                            h += attn(q, k, v) W_o^T + s B_o (attn A_o)
                            h += down(silu(gate) * up) with gate|up one fused projection.
"""
from __future__ import annotations

from dataclasses import dataclass

import torch

from . import kernels as K


@dataclass
class LayerWeights:
    """Frozen weights of one decoder layer (fused projections plus transposed copies)."""
    w_qkv: torch.Tensor      # [q+2kv, H]
    w_qkv_t: torch.Tensor    # [H, q+2kv]
    w_o: torch.Tensor        # [H, q]
    w_o_t: torch.Tensor      # [q, H]
    w_gu: torch.Tensor       # [2F, H]
    w_gu_t: torch.Tensor     # [H, 2F]
    w_d: torch.Tensor        # [H, F]
    w_d_t: torch.Tensor      # [F, H]
    ln_in: torch.Tensor
    ln_post: torch.Tensor
    q_norm: torch.Tensor | None
    k_norm: torch.Tensor | None
    w_gu_i: torch.Tensor | None = None   # [2F, H], gate/up rows interleaved in blocks of 64


@dataclass
class Geometry:
    nq: int
    nk: int
    d: int
    H: int
    F: int
    eps: float

    @property
    def q(self):
        return self.nq * self.d

    @property
    def kv(self):
        return self.nk * self.d


@dataclass
class StreamContext:
    """Per-forward data shared by all layers: positions, interval tables, clean K/V, RoPE angles."""
    pos: torch.Tensor            # [M] int64 positions of stream rows
    inv_freq: torch.Tensor       # [d/2] fp32
    iv_noisy: torch.Tensor       # [M, 8] int32
    iv_clean: torch.Tensor       # [M, 8] int32
    clean_k: list                # per layer [M, kv]
    clean_v: list
    rope_cos: torch.Tensor | None = None   # [P, d/2] fp32 tables for the fused q|k|v epilogue
    rope_sin: torch.Tensor | None = None


def _qkv_dtype(x: torch.Tensor):
    """Element type of the q/k/v projection output. A bf16 step keeps it in fp32: the q/k
    normalisation and rotation then round once, at their output (the step's LoRA gradients are most
    sensitive to the precision of q and k); v is copied out in bf16 for the attention kernels."""
    return torch.float32 if x.dtype == torch.bfloat16 else x.dtype


def project_qk_v(x1, lw: LayerWeights, g: Geometry, sc: StreamContext, a2=None, b2=None, segments=None,
                 for_backward: bool = False):
    """q/k/v projection (with its LoRA extension), q/k norm and RoPE: (x_qk, q, k, v, rstd), where x_qk
    holds the pre-norm q/k columns first (what the q/k norm backward reads): the fp32 projection
    output, or, when the GEMM applies the norm and RoPE in its epilogue, their bf16 copy (only with
    ``for_backward``; None otherwise)."""
    K2 = b2.shape[1] if b2 is not None else 0
    if sc.rope_cos is not None and K.qkv_rope_fused_ok(x1.shape[0], x1.shape[1], K2, g.nq, g.nk, g.d, x1.dtype):
        q, k, v, rstd, pre = K.gemm_nt_qkv_rope(x1, lw.w_qkv, g.nq, g.nk, lw.q_norm, lw.k_norm, sc.pos, sc.rope_cos,
                                                sc.rope_sin, g.eps, a2=a2, b2=b2, segments=segments,
                                                want_rstd=for_backward, want_pre=for_backward)
        return pre, q, k, v, rstd
    qkv = K.gemm_nt(x1, lw.w_qkv, a2=a2, b2=b2, segments=segments, out_dtype=_qkv_dtype(x1))
    if qkv.dtype == x1.dtype:
        q, k, rstd = K.qknorm_rope_fwd(qkv, g.nq, g.nk, g.d, lw.q_norm, lw.k_norm, sc.pos, sc.inv_freq, g.eps)
        v = qkv[:, g.q + g.kv:]   # a strided view: the attention kernels take V's row stride, no copy
    else:
        q, k, v, rstd = K.qknorm_rope_fwd(qkv, g.nq, g.nk, g.d, lw.q_norm, lw.k_norm, sc.pos, sc.inv_freq, g.eps,
                                          out_dtype=x1.dtype, with_v=True)
    return qkv, q, k, v, rstd


def clean_layer(h: torch.Tensor, lw: LayerWeights, g: Geometry, sc: StreamContext):
    """Forward-only clean-stream layer; returns (h_out, k, v) with k/v kept for the noisy stream."""
    M = h.shape[0]
    x1, _ = K.rmsnorm_fwd(h, lw.ln_in, g.eps)
    _, q, k, v, _ = project_qk_v(x1, lw, g, sc)
    o, _ = K.attn_fwd(q, k, v, sc.iv_clean, g.nq, g.nk, g.d)
    h1 = K.gemm_nt(o, lw.w_o, residual=h)
    x2, _ = K.rmsnorm_fwd(h1, lw.ln_post, g.eps)
    if lw.w_gu_i is not None and x2.dtype == torch.bfloat16 and K.swiglu_fused_ok(M, g.F, g.H):
        s = K.gemm_nt_swiglu(x2, lw.w_gu_i)      # gate/up product with SwiGLU in its epilogue
    else:
        s = K.swiglu_fwd(K.gemm_nt(x2, lw.w_gu), g.F)
    h2 = K.gemm_nt(s, lw.w_d, residual=h1)
    return h2, k, v


def clean_layer_kv(h: torch.Tensor, lw: LayerWeights, g: Geometry, sc: StreamContext):
    """The K and V a clean-stream layer hands the noisy stream, without the layer's output (its
    attention, o projection and MLP): the same kernels and values as clean_layer's k and v."""
    x1, _ = K.rmsnorm_fwd(h, lw.ln_in, g.eps)
    _, _, k, v, _ = project_qk_v(x1, lw, g, sc)
    return k, v


def noisy_layer_forward(h0, lw: LayerWeights, lora, li: int, g: Geometry, sc: StreamContext, need_output: bool = True):
    """Forward of one noisy-stream layer; returns (h2 or None, the activations its backward reads).
    Deterministic: a second call on the same inputs reproduces every buffer bit for bit, which the
    recompute policy relies on. ``need_output=False`` (recompute) skips the down projection's output."""
    r = lora.rank
    q_end, k_end = g.q, g.q + g.kv
    on = lora.group_active     # a fused group with no adapter runs as a plain product
    x1, rstd1 = K.rmsnorm_fwd(h0, lw.ln_in, g.eps)
    h_qkv = K.gemm_nt(x1, lora.a_c(li, "qkv")) if on("qkv") else None
    qkv, q, k, v, rstd_qk = project_qk_v(
        x1, lw, g, sc, a2=h_qkv, b2=lora.sb_c(li, "qkv") if on("qkv") else None,
        segments=[(q_end, 0), (k_end, r), (k_end + g.kv, 2 * r)] if on("qkv") else None, for_backward=True)
    o, lse = K.attn_fwd(q, sc.clean_k[li], sc.clean_v[li], sc.iv_noisy, g.nq, g.nk, g.d, k2=k, v2=v)
    h_o = K.gemm_nt(o, lora.a_c(li, "o")) if on("o") else None
    h1 = K.gemm_nt(o, lw.w_o, a2=h_o, b2=lora.sb_c(li, "o") if on("o") else None, residual=h0)
    x2, rstd2 = K.rmsnorm_fwd(h1, lw.ln_post, g.eps)
    h_gu = K.gemm_nt(x2, lora.a_c(li, "gu")) if on("gu") else None
    fused = lw.w_gu_i is not None and x2.dtype == torch.bfloat16 and K.swiglu_fused_ok(x2.shape[0], g.F, x2.shape[1])
    sb_gu_i = lora.sb_gu_i(li) if fused and on("gu") else None
    if fused and (not on("gu") or (sb_gu_i is not None and (2 * r) % 32 == 0)):
        # gate/up product with its LoRA terms, SwiGLU in the epilogue; [gate | up] kept for backward
        gu = torch.empty((x2.shape[0], 2 * g.F), device=x2.device, dtype=x2.dtype)
        s = K.gemm_nt_swiglu(x2, lw.w_gu_i, a2=h_gu, b2_interleaved=sb_gu_i, gu=gu)
    else:
        gu = K.gemm_nt(x2, lw.w_gu, a2=h_gu, b2=lora.sb_c(li, "gu") if on("gu") else None,
                       segments=[(g.F, 0), (2 * g.F, r)] if on("gu") else None)
        s = K.swiglu_fwd(gu, g.F)
    h_d = K.gemm_nt(s, lora.a_c(li, "d")) if on("d") else None
    h2 = K.gemm_nt(s, lw.w_d, a2=h_d, b2=lora.sb_c(li, "d") if on("d") else None, residual=h1) \
        if need_output else None
    return h2, (h0, x1, rstd1, h_qkv, qkv, q, k, v, rstd_qk, o, lse, h_o, h1, x2, rstd2, h_gu, gu, s, h_d)


def saved_bytes_per_row(g: Geometry, rank: int, elem: int, fused_qkv: bool = True) -> int:
    """Bytes of activations one noisy-stream layer keeps per token row for its backward
    (``fused_qkv``: the q|k|v epilogue keeps bf16 pre-norm q/k; otherwise a bf16 step keeps the fp32
    projection output)."""
    stored = 4 * g.H + g.q + g.kv + g.q + 3 * g.F + 7 * rank
    if elem == 2 and not fused_qkv:
        qkv = (g.q + 2 * g.kv) * 4 + g.kv * elem
    else:
        qkv = (g.q + 2 * g.kv) * elem
    return stored * elem + qkv + 4 * (2 + g.nq + g.nk + g.nq)


def _lora_inner_grads(lora, li: int, group: str, dy, h, cols, scale):
    """For a fused group [c0, c1) column ranges of its output gradient dy: the inner gradients
    g = dy (s B) (columns of the returned [M, parts * r]) and dB += s dy^T h. Projections without
    an adapter get zero columns (their A rows are zero, so g A adds nothing, but unset memory
    could hold non-finite values) and no weight gradient. None when the group has no adapter."""
    from .adapter import GROUPS
    if not lora.group_active(group):
        return None
    r = lora.rank
    out = torch.empty((dy.shape[0], len(cols) * r), device=dy.device, dtype=dy.dtype)
    sbt = lora.sb_t(li, group)
    gbg = lora.grad_b(li, group)
    for j, ((c0, c1), name) in enumerate(zip(cols, GROUPS[group])):
        if not lora.is_target(name):
            out[:, j * r:(j + 1) * r].zero_()
            continue
        K.gemm_nt(dy[:, c0:c1], sbt[:, c0:c1], out=out[:, j * r:(j + 1) * r])
        K.gemm_tn(dy[:, c0:c1], h[:, j * r:(j + 1) * r], out=gbg[c0:c1], alpha=scale, beta=1.0)
    return out


class NoisyLayer(torch.autograd.Function):
    """One noisy-stream decoder layer with fused gated LoRA (forward and backward). With
    ``recompute`` the layer keeps only its input and reruns its forward in the backward."""

    @staticmethod
    def forward(ctx, h0, anchor, lw: LayerWeights, lora, li: int, g: Geometry, sc: StreamContext,
                recompute: bool = False):
        del anchor
        h2, bufs = noisy_layer_forward(h0, lw, lora, li, g, sc)
        ctx.lw, ctx.lora, ctx.li, ctx.g, ctx.sc = lw, lora, li, g, sc
        if recompute:
            ctx.bufs, ctx.h0 = None, h0
        else:
            ctx.bufs, ctx.h0 = bufs, None
        return h2

    @staticmethod
    def backward(ctx, dh2):
        lw, lora, li, g, sc = ctx.lw, ctx.lora, ctx.li, ctx.g, ctx.sc
        bufs = ctx.bufs
        if bufs is None:
            _, bufs = noisy_layer_forward(ctx.h0, lw, lora, li, g, sc, need_output=False)
        (h0, x1, rstd1, h_qkv, qkv, q, k, v, rstd_qk, o, lse, h_o, h1, x2, rstd2, h_gu, gu, s, h_d) = bufs
        ctx.bufs = ctx.h0 = bufs = None
        dh2 = dh2.contiguous()
        M = dh2.shape[0]
        r, sc_l = lora.rank, lora.scale
        q_end, k_end = g.q, g.q + g.kv
        ga, gb = lora.grad_a, lora.grad_b
        on = lora.group_active
        # ---- down projection ----------------------------------------------------------
        g_d = K.gemm_nt(dh2, lora.sb_t(li, "d")) if on("d") else None                 # [M, r]
        if on("d"):
            K.gemm_tn(dh2, h_d, out=gb(li, "d"), alpha=sc_l, beta=1.0)                # dB_d
        a_t_d = lora.a_t(li, "d") if on("d") else None
        if dh2.dtype == torch.bfloat16 and M % 256 == 0 and g.F % 256 == 0 and g.H % 64 == 0 and r % 32 == 0:
            # dS = dh2 W_d + g_d A_d never leaves the GEMM: its epilogue applies the SwiGLU backward
            dgu = K.gemm_nt_swiglu_bwd(dh2, lw.w_d_t, g_d, a_t_d, gu)
        else:
            ds = K.gemm_nt(dh2, lw.w_d_t, a2=g_d, b2=a_t_d)                            # [M, F]
            dgu = K.swiglu_bwd(ds, gu, g.F)
            del ds
        if on("d"):
            K.gemm_tn(g_d, s, out=ga(li, "d"), beta=1.0)                              # dA_d
        # ---- gate | up -----------------------------------------------------------------
        g_gu = _lora_inner_grads(lora, li, "gu", dgu, h_gu, ((0, g.F), (g.F, 2 * g.F)), sc_l)
        dx2 = K.gemm_nt(dgu, lw.w_gu_t, a2=g_gu, b2=lora.a_t(li, "gu") if on("gu") else None)
        if on("gu"):
            K.gemm_tn(g_gu, x2, out=ga(li, "gu"), beta=1.0)
        del dgu
        dh1 = K.rmsnorm_bwd(dx2, h1, lw.ln_post, rstd2, dres=dh2)
        del dx2
        # ---- o projection --------------------------------------------------------------
        g_o = K.gemm_nt(dh1, lora.sb_t(li, "o")) if on("o") else None
        if on("o"):
            K.gemm_tn(dh1, h_o, out=gb(li, "o"), alpha=sc_l, beta=1.0)
        do = K.gemm_nt(dh1, lw.w_o_t, a2=g_o, b2=lora.a_t(li, "o") if on("o") else None)
        if on("o"):
            K.gemm_tn(g_o, o, out=ga(li, "o"), beta=1.0)
        # ---- attention -----------------------------------------------------------------
        # dq and dk in the q/k/v projection's precision (fp32 for a bf16 step) up to the q/k norm
        # backward, which writes the bf16 q/k gradient blocks of dqkv; dv goes straight into dqkv
        dqkv = torch.empty((M, g.q + 2 * g.kv), device=dh2.device, dtype=dh2.dtype)
        if qkv.dtype == torch.bfloat16 and qkv.shape[1] == k_end and sc.rope_cos is not None:
            # the fused forward kept the bf16 pre-norm q/k: the attention backward applies the q/k
            # norm + RoPE backward to its fp32 dQ / dK accumulators and writes dqkv directly
            K.attn_bwd_qknorm(q, sc.clean_k[li], sc.clean_v[li], sc.iv_noisy, o, lse, do, g.nq, g.nk, g.d, k, v,
                              qkv, rstd_qk, lw.q_norm, lw.k_norm, sc.pos, sc.rope_cos, sc.rope_sin, dqkv)
            del do
        else:
            gdt = _qkv_dtype(dh2)
            dk = torch.empty((M, g.kv), device=dh2.device, dtype=gdt)
            dq = K.attn_bwd(q, sc.clean_k[li], sc.clean_v[li], sc.iv_noisy, o, lse, do, g.nq, g.nk, g.d,
                            k2=k, v2=v, ivk=sc.iv_noisy, dk=dk, dv=dqkv[:, k_end:], grad_dtype=gdt)
            del do
            K.qknorm_rope_bwd(dq, dk, qkv, g.nq, g.nk, g.d, lw.q_norm, lw.k_norm, sc.pos, sc.inv_freq, rstd_qk, dqkv)
            del dq, dk
        # ---- q | k | v -----------------------------------------------------------------
        g_qkv = _lora_inner_grads(lora, li, "qkv", dqkv, h_qkv, ((0, q_end), (q_end, k_end), (k_end, k_end + g.kv)),
                                  sc_l)
        if on("qkv"):
            K.gemm_tn(g_qkv, x1, out=ga(li, "qkv"), beta=1.0)
        dh0 = None
        if ctx.needs_input_grad[0]:
            dx1 = K.gemm_nt(dqkv, lw.w_qkv_t, a2=g_qkv, b2=lora.a_t(li, "qkv") if on("qkv") else None)
            dh0 = K.rmsnorm_bwd(dx1, h0, lw.ln_in, rstd1, dres=dh1)
        return dh0, None, None, None, None, None, None, None


class FinalNorm(torch.autograd.Function):
    """Final RMSNorm of the noisy stream."""

    @staticmethod
    def forward(ctx, h, w, eps, anchor):
        del anchor
        y, rstd = K.rmsnorm_fwd(h, w, eps)
        ctx.bufs = (h, w, rstd)
        return y

    @staticmethod
    def backward(ctx, dy):
        h, w, rstd = ctx.bufs
        ctx.bufs = None
        return K.rmsnorm_bwd(dy.contiguous(), h, w, rstd), None, None, None


class ScatterStreams(torch.autograd.Function):
    """Writes the noisy and clean streams into the [B*2L, H] concatenated layout."""

    @staticmethod
    def forward(ctx, noisy, clean, noisy_src, clean_src):
        M = noisy.shape[0]
        out = torch.empty((2 * M, noisy.shape[1]), device=noisy.device, dtype=noisy.dtype)
        K.rows_copy(noisy, out, M, dmap=noisy_src)
        K.rows_copy(clean, out, M, dmap=clean_src)
        ctx.noisy_src = noisy_src
        ctx.M = M
        return out

    @staticmethod
    def backward(ctx, dout):
        dout = dout.contiguous()
        dn = torch.empty((ctx.M, dout.shape[1]), device=dout.device, dtype=dout.dtype)
        K.rows_copy(dout, dn, ctx.M, smap=ctx.noisy_src)
        return dn, None, None, None


class GatherRows(torch.autograd.Function):
    """out[i] = x[idx[i]] (int32 idx); backward scatters into zeros."""

    @staticmethod
    def forward(ctx, x, idx):
        out = torch.empty((idx.numel(), x.shape[1]), device=x.device, dtype=x.dtype)
        K.rows_copy(x, out, idx.numel(), smap=idx)
        ctx.idx, ctx.rows = idx, x.shape[0]
        return out

    @staticmethod
    def backward(ctx, dout):
        dx = torch.zeros((ctx.rows, dout.shape[1]), device=dout.device, dtype=dout.dtype)
        K.rows_copy(dout.contiguous(), dx, ctx.idx.numel(), dmap=ctx.idx)
        return dx, None
