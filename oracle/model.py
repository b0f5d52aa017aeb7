"""Qwen3 decoder with token-gated LoRA, fp32, one pass over the 2L concatenated rows.

Restates the base decoder math of transformers/models/qwen3/modeling_qwen3.py (RMSNorm in
fp32, per-head q/k RMSNorm before rotary embedding, rotate_half RoPE, GQA, SwiGLU) with PEFT
LoRA on q/k/v/o/gate/up/down: y = x W^T + s * ((m (.) (x A^T)) B^T), s = alpha/r, m the token
gate (training/lora.py:164-174). Attention uses an explicit dense boolean mask. Pinned by
tests/test_oracle_model.py against transformers' Qwen3Model (gate off) and against merged
LoRA weights W + s*B@A (gate on).
"""
from __future__ import annotations

from dataclasses import dataclass, field

import torch
import torch.nn.functional as F

LORA_MODULES = ("q_proj", "k_proj", "v_proj", "o_proj", "gate_proj", "up_proj", "down_proj")


@dataclass
class Cfg:
    vocab_size: int
    hidden_size: int
    intermediate_size: int
    num_hidden_layers: int
    num_attention_heads: int
    num_key_value_heads: int
    head_dim: int
    rms_norm_eps: float = 1e-6
    rope_theta: float = 1e6
    qk_norm: bool = True
    lora_rank: int = 8
    lora_alpha: float = 16.0
    lora_targets: tuple = field(default=LORA_MODULES)

    @property
    def lora_scale(self) -> float:
        return self.lora_alpha / self.lora_rank


def module_shapes(cfg: Cfg) -> dict[str, tuple[int, int]]:
    """(out, in) of every LoRA-capable projection."""
    H, d = cfg.hidden_size, cfg.head_dim
    q, kv, f = cfg.num_attention_heads * d, cfg.num_key_value_heads * d, cfg.intermediate_size
    return {"q_proj": (q, H), "k_proj": (kv, H), "v_proj": (kv, H), "o_proj": (H, q),
            "gate_proj": (f, H), "up_proj": (f, H), "down_proj": (H, f)}


def module_path(i: int, name: str) -> str:
    group = "self_attn" if name in ("q_proj", "k_proj", "v_proj", "o_proj") else "mlp"
    return f"model.layers.{i}.{group}.{name}"


def rms_norm(x: torch.Tensor, w: torch.Tensor, eps: float) -> torch.Tensor:
    # fp32 statistics as in Qwen3RMSNorm (fp64 inputs stay fp64 for finite-difference checks)
    xf = x if x.dtype == torch.float64 else x.float()
    var = xf.pow(2).mean(-1, keepdim=True)
    return w * (xf * torch.rsqrt(var + eps)).to(x.dtype)


def rope_cos_sin(pos: torch.Tensor, head_dim: int, theta: float):
    inv = 1.0 / (theta ** (torch.arange(0, head_dim, 2, dtype=torch.int64).float() / head_dim))
    freqs = pos.float()[..., None] * inv
    emb = torch.cat((freqs, freqs), dim=-1)
    return emb.cos(), emb.sin()


def rotate_half(x):
    h = x.shape[-1] // 2
    return torch.cat((-x[..., h:], x[..., :h]), dim=-1)


def lora_linear(x, W, A, B, gate, scale):
    y = x @ W.T
    if A is None:
        return y
    A, B = A.to(x.dtype), B.to(x.dtype)   # adapters compute in the activation dtype
    h = x @ A.T
    if gate is not None:
        h = h * gate.to(h.dtype)[..., None]
    return y + scale * (h @ B.T)


def _keep(x, name):
    return x


def decoder(params: dict, lora: dict, cfg: Cfg, ids: torch.Tensor, pos: torch.Tensor, mask: torch.Tensor,
            gate: torch.Tensor | None, rnd=None) -> torch.Tensor:
    """ids/pos [B,T]; mask [B,T,T] bool (query, key); gate [B,T] -> final-norm hidden [B,T,H].

    ``rnd(x, point)``, when given, is applied to the activation stored at each named point (x1, qkv,
    qk, o, resid, x2, gu, sw, final, and the LoRA weights/inner product lora_w, lora_h): a hook for
    studying where the rounding of a bf16 implementation enters; the default leaves values as they
    are."""
    rnd = rnd or _keep
    Bsz, T = ids.shape
    Hq, Hkv, d = cfg.num_attention_heads, cfg.num_key_value_heads, cfg.head_dim
    s = cfg.lora_scale
    h = params["model.embed_tokens.weight"][ids]
    cos, sin = rope_cos_sin(pos, d, cfg.rope_theta)
    # cos/sin are cast to the activation dtype as in Qwen3RotaryEmbedding (no-op in fp32)
    dt = params["model.embed_tokens.weight"].dtype
    cos, sin = cos[:, None].to(dt), sin[:, None].to(dt)  # [B,1,T,d]
    bias = torch.zeros(mask.shape, dtype=torch.float32).masked_fill(~mask, float("-inf"))[:, None]

    def lin(i, name, x):
        p = module_path(i, name)
        A, B = lora.get(p + ".lora_A.weight"), lora.get(p + ".lora_B.weight")
        if A is None or rnd is _keep:
            return lora_linear(x, params[p + ".weight"], A, B, gate, s)
        A, sB = rnd(A.to(x.dtype), "lora_w"), rnd(s * B.to(x.dtype), "lora_w")
        hh = x @ A.T
        if gate is not None:
            hh = hh * gate.to(hh.dtype)[..., None]
        return x @ params[p + ".weight"].T + rnd(hh, "lora_h") @ sB.T

    for i in range(cfg.num_hidden_layers):
        pre = f"model.layers.{i}."
        x = rnd(rms_norm(h, params[pre + "input_layernorm.weight"], cfg.rms_norm_eps), "x1")
        q = rnd(lin(i, "q_proj", x), "qkv").view(Bsz, T, Hq, d)
        k = rnd(lin(i, "k_proj", x), "qkv").view(Bsz, T, Hkv, d)
        v = rnd(lin(i, "v_proj", x), "qkv").view(Bsz, T, Hkv, d)
        if cfg.qk_norm:
            q = rms_norm(q, params[pre + "self_attn.q_norm.weight"], cfg.rms_norm_eps)
            k = rms_norm(k, params[pre + "self_attn.k_norm.weight"], cfg.rms_norm_eps)
        q, k, v = q.transpose(1, 2), k.transpose(1, 2), v.transpose(1, 2)
        q = rnd(q * cos + rotate_half(q) * sin, "qk")
        k = rnd(k * cos + rotate_half(k) * sin, "qk")
        rep = Hq // Hkv
        k = k.repeat_interleave(rep, dim=1)
        v = v.repeat_interleave(rep, dim=1)
        scores = (q @ k.transpose(-1, -2)) * d ** -0.5 + bias
        # softmax in fp32 then back to the activation dtype (eager Qwen3 attention)
        attn = torch.softmax(scores.float() if scores.dtype != torch.float64 else scores, dim=-1).to(q.dtype) @ v
        attn = rnd(attn.transpose(1, 2).reshape(Bsz, T, Hq * d), "o")
        h = rnd(h + lin(i, "o_proj", attn), "resid")
        x = rnd(rms_norm(h, params[pre + "post_attention_layernorm.weight"], cfg.rms_norm_eps), "x2")
        mlp = rnd(F.silu(rnd(lin(i, "gate_proj", x), "gu")) * rnd(lin(i, "up_proj", x), "gu"), "sw")
        h = rnd(h + lin(i, "down_proj", mlp), "resid")
    return rnd(rms_norm(h, params["model.norm.weight"], cfg.rms_norm_eps), "final")


def init_params(cfg: Cfg, seed: int, std: float = 0.02, dtype=torch.float32) -> dict:
    """Random-init N(0, std) weights, unit norm weights (CPU generator, reproducible)."""
    g = torch.Generator().manual_seed(seed)

    def normal(*shape):
        return (torch.randn(*shape, generator=g) * std).to(dtype)

    p = {"model.embed_tokens.weight": normal(cfg.vocab_size, cfg.hidden_size)}
    for i in range(cfg.num_hidden_layers):
        pre = f"model.layers.{i}."
        for name, (o, n) in module_shapes(cfg).items():
            p[module_path(i, name) + ".weight"] = normal(o, n)
        p[pre + "input_layernorm.weight"] = torch.ones(cfg.hidden_size, dtype=dtype)
        p[pre + "post_attention_layernorm.weight"] = torch.ones(cfg.hidden_size, dtype=dtype)
        if cfg.qk_norm:
            p[pre + "self_attn.q_norm.weight"] = torch.ones(cfg.head_dim, dtype=dtype)
            p[pre + "self_attn.k_norm.weight"] = torch.ones(cfg.head_dim, dtype=dtype)
    p["model.norm.weight"] = torch.ones(cfg.hidden_size, dtype=dtype)
    p["lm_head.weight"] = normal(cfg.vocab_size, cfg.hidden_size)
    return p


def init_lora(cfg: Cfg, seed: int, b_std: float = 0.02) -> dict:
    """A ~ kaiming-uniform(a=sqrt(5)) = U(-1/sqrt(in), 1/sqrt(in)); B ~ N(0, b_std); fp32."""
    g = torch.Generator().manual_seed(seed)
    out = {}
    r = cfg.lora_rank
    for i in range(cfg.num_hidden_layers):
        for name, (o, n) in module_shapes(cfg).items():
            if name not in cfg.lora_targets:
                continue
            p = module_path(i, name)
            bound = 1.0 / n ** 0.5
            out[p + ".lora_A.weight"] = (torch.rand(r, n, generator=g) * 2 - 1) * bound
            out[p + ".lora_B.weight"] = torch.randn(o, r, generator=g) * b_std
    return out
