"""Qwen3-architecture block-diffusion model for the Uno step (MI355X-native).

Provides the model-side interface the reference step calls (training/trainer.py:198-209,
training/modeling.py:15-62,116-147), which in the reference comes from the remote model code:
  * ``UnoQwen3ForCausalLM.prepare_for_bd_training(input_ids, model_position_ids, prompt_mask)``
    returning (concat_ids, concat_pos, attention_mask, noised_positions, noise_levels, p_mask);
  * ``.model(input_ids=, attention_mask=, position_ids=, ...).last_hidden_state``;
  * ``.lm_head``, ``.config.block_size``, ``.config.noise``;
  * module-level ``modify_padded_position_ids_2d`` and ``calculate_token_nums``.

Storage is laid out for HBM capacity rather than for module boundaries: each layer keeps its
projections fused (q|k|v and gate|up) plus transposed copies of every frozen weight, so every
large product of forward and backward is a K-contiguous MFMA GEMM. The per-projection modules
(q_proj, ..., down_proj) expose views into the fused storage under the usual names.
"""
from __future__ import annotations

import contextlib
from dataclasses import dataclass, field

import torch
from torch import nn

from . import _native as N
from . import kernels as K
from . import layers as Lyr
from .adapter import GROUPS, MODULES, LoraState, module_dims

_MASK64 = (1 << 64) - 1
_GOLDEN = 0x9E3779B97F4A7C15


def _mix64(x: int) -> int:
    """splitmix64 finaliser (nano_vllm_uno/engine/noise.py:43-50 uses the same constants)."""
    x &= _MASK64
    x = ((x ^ (x >> 30)) * 0xBF58476D1CE4E5B9) & _MASK64
    x = ((x ^ (x >> 27)) * 0x94D049BB133111EB) & _MASK64
    return x ^ (x >> 31)


def noise_key(seed: int, step: int) -> int:
    return _mix64((seed & _MASK64) + _GOLDEN * (step + 1))


@dataclass
class UnoQwen3Config:
    vocab_size: int = 4096
    hidden_size: int = 256
    intermediate_size: int = 768
    num_hidden_layers: int = 2
    num_attention_heads: int = 4
    num_key_value_heads: int = 2
    head_dim: int = 64
    rms_norm_eps: float = 1e-6
    rope_theta: float = 1e6
    qk_norm: bool = True
    block_size: int = 4
    noise: str | None = "uniform"
    mask_token_id: int | None = None
    noise_seed: int = 20260813
    intra_block: str = "bidirectional"
    tie_word_embeddings: bool = False
    use_cache: bool = False
    extra: dict = field(default_factory=dict)

    @property
    def resolved_mask_token_id(self) -> int:
        return self.vocab_size - 1 if self.mask_token_id is None else int(self.mask_token_id)


# ------------------------------------------------------------------------------------------
# Module-level helpers looked up by training/modeling.py:47-62
# ------------------------------------------------------------------------------------------
def modify_padded_position_ids_2d(position_ids: torch.Tensor) -> torch.Tensor:
    """Positions pass through unchanged (rows carry no padding markers in the training data)."""
    return position_ids.clone()


def calculate_token_nums(position_ids: torch.Tensor) -> list[torch.Tensor]:
    """Per row, the segment lengths; a segment starts at t = 0 and wherever pos[t-1] >= pos[t]."""
    B, L = position_ids.shape
    starts = torch.ones((B, L), dtype=torch.bool, device=position_ids.device)
    starts[:, 1:] = position_ids[:, :-1] >= position_ids[:, 1:]
    out = []
    for b in range(B):
        idx = torch.nonzero(starts[b]).flatten()
        ends = torch.cat([idx[1:], idx.new_tensor([L])])
        out.append(ends - idx)
    return out


def noisy_region_mask(model_position_ids: torch.Tensor) -> torch.Tensor:
    """[B, 2L] bool: the per-segment [noisy | clean] layout of the concatenated batch (True on the
    noisy copies), segments as in ``calculate_token_nums``; one device kernel, no host work."""
    if model_position_ids.dim() != 2:
        raise RuntimeError(f"model positions must be [B, L], got {tuple(model_position_ids.shape)}")
    B, L = model_position_ids.shape
    pos = model_position_ids.to(torch.int64).contiguous()
    region = torch.empty((B, 2 * L), device=pos.device, dtype=torch.bool)
    N.call("unok_bd_region", B, L, N.ptr(pos), N.ptr(region), N.stream())
    return region


# ------------------------------------------------------------------------------------------
# Attention-mask object returned by prepare_for_bd_training
# ------------------------------------------------------------------------------------------
class BlockDiffusionMask:
    """Block-diffusion attention pattern of a [B, 2L] concatenated batch, kept as per-row key
    intervals of the two streams plus the maps between the concatenated and stream layouts."""

    def __init__(self, B, L, block_size, intra_block, region, noisy_src, clean_src, iv_noisy, iv_clean,
                 noisy_ids, clean_ids, pos_stream):
        self.B, self.L, self.block_size, self.intra_block = B, L, block_size, intra_block
        self.region = region            # [B, 2L] bool: True on noisy rows
        self.noisy_src = noisy_src      # [B*L] int32 flat concat index of noisy stream row
        self.clean_src = clean_src
        self.iv_noisy = iv_noisy        # [B*L, 8] int32
        self.iv_clean = iv_clean
        self.noisy_ids = noisy_ids      # [B*L] int64
        self.clean_ids = clean_ids
        self.pos_stream = pos_stream    # [B*L] int64

    @property
    def shape(self):
        return (self.B, 1, 2 * self.L, 2 * self.L)

    def to_dense(self) -> torch.Tensor:
        """[B, 2L, 2L] bool over the concatenated layout (CPU; for inspection and tests)."""
        B, L = self.B, self.L
        ivn, ivc = self.iv_noisy.cpu(), self.iv_clean.cpu()
        ns, cs = self.noisy_src.cpu().long(), self.clean_src.cpu().long()
        dense = torch.zeros((B * 2 * L, B * 2 * L), dtype=torch.bool)
        ar = torch.arange(B * L)
        # clean queries -> clean keys in [lo1, hi1)
        cq = cs
        lo, hi = ivc[:, 0].long(), ivc[:, 1].long()
        allow = (ar[None, :] >= lo[:, None]) & (ar[None, :] < hi[:, None])
        dense[cq[:, None], cs[None, :]] = allow
        lo1, hi1, lo2, hi2 = (ivn[:, i].long() for i in range(4))
        a1 = (ar[None, :] >= lo1[:, None]) & (ar[None, :] < hi1[:, None])
        a2 = (ar[None, :] >= lo2[:, None]) & (ar[None, :] < hi2[:, None])
        dense[ns[:, None], cs[None, :]] = a1
        dense[ns[:, None], ns[None, :]] = a2
        out = torch.zeros((B, 2 * L, 2 * L), dtype=torch.bool)
        for b in range(B):
            out[b] = dense[b * 2 * L:(b + 1) * 2 * L, b * 2 * L:(b + 1) * 2 * L]
        return out


def bd_prepare(input_ids, model_position_ids, prompt_mask, *, block_size: int, mask_token_id: int,
               noise: str = "uniform", intra_block: str = "bidirectional", seed: int = 20260813, step: int = 0,
               device=None, region: torch.Tensor | None = None):
    """Device-side block-diffusion preparation; returns (concat_ids [B,2L], concat_pos [B,2L],
    BlockDiffusionMask, noised [B,L] bool, noise level per token [B,L] fp32, p_mask [n_noised])."""
    if noise not in ("uniform", "mask"):
        raise RuntimeError(f"Unsupported noise mode {noise!r}.")
    if intra_block not in ("bidirectional", "causal"):
        raise ValueError(f"intra_block must be 'bidirectional' or 'causal', got {intra_block!r}")
    B, L = input_ids.shape
    dev = torch.device(device) if device is not None else input_ids.device
    ids = input_ids.to(dev, torch.int64).contiguous()
    pos = model_position_ids.to(dev, torch.int64).contiguous()
    prompt = prompt_mask.to(dev, torch.bool).contiguous()
    if tuple(pos.shape) != (B, L) or tuple(prompt.shape) != (B, L):
        raise RuntimeError("prepare_for_bd_training: positions and prompt mask must match input_ids")
    key = noise_key(seed, step)
    i64 = dict(device=dev, dtype=torch.int64)
    i32 = dict(device=dev, dtype=torch.int32)
    concat_ids = torch.empty((B, 2 * L), **i64)
    concat_pos = torch.empty((B, 2 * L), **i64)
    if region is None:
        region = torch.empty((B, 2 * L), device=dev, dtype=torch.bool)
    elif tuple(region.shape) != (B, 2 * L) or region.dtype != torch.bool or not region.is_contiguous():
        raise RuntimeError("prepare_for_bd_training: region buffer must be a contiguous [B, 2L] bool tensor")
    noised = torch.empty((B, L), device=dev, dtype=torch.bool)
    tfull = torch.empty((B, L), device=dev, dtype=torch.float32)
    noisy_src, clean_src = torch.empty(B * L, **i32), torch.empty(B * L, **i32)
    iv_noisy, iv_clean = torch.empty((B * L, 8), **i32), torch.empty((B * L, 8), **i32)
    noisy_ids, clean_ids = torch.empty(B * L, **i64), torch.empty(B * L, **i64)
    N.call("unok_bd_prepare", B, L, N.ptr(ids), N.ptr(pos), N.ptr(prompt), int(block_size), int(mask_token_id),
           int(noise == "mask"), int(intra_block == "causal"), key, N.ptr(concat_ids), N.ptr(concat_pos),
           N.ptr(region), N.ptr(noised), N.ptr(tfull), N.ptr(noisy_src), N.ptr(clean_src), N.ptr(iv_noisy),
           N.ptr(iv_clean), N.ptr(noisy_ids), N.ptr(clean_ids), N.stream())
    p_buf = torch.empty(max(B * L, 1), device=dev, dtype=torch.float32)
    count = torch.empty(2, **i32)
    N.call("unok_bd_compact", B * L, N.ptr(noised), N.ptr(tfull), N.ptr(pos), N.ptr(p_buf), N.ptr(count), N.stream())
    n_noised, max_pos = (int(v) for v in count.tolist())   # one host synchronisation for both
    mask = BlockDiffusionMask(B, L, int(block_size), intra_block, region, noisy_src, clean_src, iv_noisy, iv_clean,
                              noisy_ids, clean_ids, pos.view(-1))
    mask.max_pos = max_pos
    return concat_ids, concat_pos, mask, noised, tfull, p_buf[:n_noised]


@dataclass
class UnoModelOutput:
    last_hidden_state: torch.Tensor

    def __getitem__(self, k):
        return getattr(self, k)


# ------------------------------------------------------------------------------------------
# Modules
# ------------------------------------------------------------------------------------------
class _Frozen(nn.Module):
    def __init__(self, weight: torch.Tensor):
        super().__init__()
        self.weight = nn.Parameter(weight, requires_grad=False)


class UnoRMSNorm(_Frozen):
    def __init__(self, weight, eps):
        super().__init__(weight)
        self.variance_epsilon = eps

    def forward(self, x):
        shape = x.shape
        y, _ = K.rmsnorm_fwd(x.reshape(-1, shape[-1]).contiguous(), self.weight, self.variance_epsilon)
        return y.view(shape)


class _LoraWeight(nn.Module):
    def __init__(self, view: torch.Tensor, grad_view: torch.Tensor, state: LoraState):
        super().__init__()
        self.weight = nn.Parameter(view, requires_grad=True)
        state.bind_parameter(self.weight, grad_view)


class UnoProjection(nn.Module):
    """A frozen linear whose weight is a view into the layer's fused storage. With an adapter
    attached it carries PEFT-style ``lora_A`` / ``lora_B`` ModuleDicts (views into the flat
    LoRA storage) and ``use_dora`` / ``scaling`` / ``r`` attributes."""

    def __init__(self, weight: torch.Tensor, weight_t: torch.Tensor):
        super().__init__()
        self.weight = nn.Parameter(weight, requires_grad=False)
        self.weight_t = weight_t
        self.out_features, self.in_features = weight.shape

    def forward(self, x):
        shape = x.shape
        y = K.gemm_nt(x.reshape(-1, shape[-1]).contiguous(), self.weight)
        return y.view(*shape[:-1], self.out_features)


class UnoLMHead(nn.Module):
    def __init__(self, weight: torch.Tensor, weight_t: torch.Tensor):
        super().__init__()
        self.weight = nn.Parameter(weight, requires_grad=False)
        self.weight_t = weight_t

    def forward(self, x):
        from .objectives import lm_head_logits
        return lm_head_logits(self, x)


class UnoAttention(nn.Module):
    def __init__(self, layer):
        super().__init__()
        g = layer.geo
        q, kv = g.q, g.kv
        self.q_proj = UnoProjection(layer.w_qkv[:q], layer.w_qkv_t[:, :q])
        self.k_proj = UnoProjection(layer.w_qkv[q:q + kv], layer.w_qkv_t[:, q:q + kv])
        self.v_proj = UnoProjection(layer.w_qkv[q + kv:], layer.w_qkv_t[:, q + kv:])
        self.o_proj = UnoProjection(layer.w_o, layer.w_o_t)
        if layer.q_norm_w is not None:
            self.q_norm = UnoRMSNorm(layer.q_norm_w, g.eps)
            self.k_norm = UnoRMSNorm(layer.k_norm_w, g.eps)


class UnoMLP(nn.Module):
    def __init__(self, layer):
        super().__init__()
        F = layer.geo.F
        self.gate_proj = UnoProjection(layer.w_gu[:F], layer.w_gu_t[:, :F])
        self.up_proj = UnoProjection(layer.w_gu[F:], layer.w_gu_t[:, F:])
        self.down_proj = UnoProjection(layer.w_d, layer.w_d_t)


class UnoDecoderLayer(nn.Module):
    def __init__(self, cfg: UnoQwen3Config, geo: Lyr.Geometry, device, dtype):
        super().__init__()
        self.geo = geo
        H, F, q, kv = geo.H, geo.F, geo.q, geo.kv
        e = dict(device=device, dtype=dtype)
        self.register_buffer("w_qkv", torch.zeros(q + 2 * kv, H, **e), persistent=False)
        self.register_buffer("w_qkv_t", torch.zeros(H, q + 2 * kv, **e), persistent=False)
        self.register_buffer("w_o", torch.zeros(H, q, **e), persistent=False)
        self.register_buffer("w_o_t", torch.zeros(q, H, **e), persistent=False)
        self.register_buffer("w_gu", torch.zeros(2 * F, H, **e), persistent=False)
        self.register_buffer("w_gu_t", torch.zeros(H, 2 * F, **e), persistent=False)
        # gate/up rows interleaved in blocks of 64 for the fused clean-stream gate/up + SwiGLU
        # product (when the shapes allow it)
        fuse = F % 128 == 0 and dtype == torch.bfloat16
        self.register_buffer("w_gu_i", torch.zeros(2 * F, H, **e) if fuse else None, persistent=False)
        self.register_buffer("w_d", torch.zeros(H, F, **e), persistent=False)
        self.register_buffer("w_d_t", torch.zeros(F, H, **e), persistent=False)
        self.q_norm_w = torch.ones(geo.d, **e) if cfg.qk_norm else None
        self.k_norm_w = torch.ones(geo.d, **e) if cfg.qk_norm else None
        self.self_attn = UnoAttention(self)
        self.mlp = UnoMLP(self)
        self.input_layernorm = UnoRMSNorm(torch.ones(H, **e), geo.eps)
        self.post_attention_layernorm = UnoRMSNorm(torch.ones(H, **e), geo.eps)

    def weights(self) -> Lyr.LayerWeights:
        qn = self.self_attn.q_norm.weight if hasattr(self.self_attn, "q_norm") else None
        kn = self.self_attn.k_norm.weight if hasattr(self.self_attn, "k_norm") else None
        return Lyr.LayerWeights(self.w_qkv, self.w_qkv_t, self.w_o, self.w_o_t, self.w_gu, self.w_gu_t, self.w_d,
                                self.w_d_t, self.input_layernorm.weight, self.post_attention_layernorm.weight, qn, kn,
                                self.w_gu_i)

    @torch.no_grad()
    def refresh_transposed(self):
        for a, b in (("w_qkv", "w_qkv_t"), ("w_o", "w_o_t"), ("w_gu", "w_gu_t"), ("w_d", "w_d_t")):
            getattr(self, b).copy_(getattr(self, a).t())
        if self.w_gu_i is not None:
            self.w_gu_i.copy_(K.interleave_gate_up(self.w_gu, self.geo.F))


class UnoQwen3Model(nn.Module):
    """The decoder. Its forward takes the concatenated [B, 2L] batch and a BlockDiffusionMask."""

    def __init__(self, cfg: UnoQwen3Config, device, dtype):
        super().__init__()
        self.config = cfg
        self.geo = Lyr.Geometry(cfg.num_attention_heads, cfg.num_key_value_heads, cfg.head_dim, cfg.hidden_size,
                                cfg.intermediate_size, cfg.rms_norm_eps)
        e = dict(device=device, dtype=dtype)
        self.embed_tokens = _Frozen(torch.zeros(cfg.vocab_size, cfg.hidden_size, **e))
        self.layers = nn.ModuleList(UnoDecoderLayer(cfg, self.geo, device, dtype) for _ in range(cfg.num_hidden_layers))
        self.norm = UnoRMSNorm(torch.ones(cfg.hidden_size, **e), cfg.rms_norm_eps)
        d = cfg.head_dim
        inv = 1.0 / (cfg.rope_theta ** (torch.arange(0, d, 2, dtype=torch.int64).float() / d))
        self.register_buffer("inv_freq", inv.to(device), persistent=False)
        self._uno_lora: LoraState | None = None
        # Activation recompute of the noisy stream: False (keep every layer's activations), True
        # (every layer reruns its forward in the backward), or "auto" (the fewest layers that make
        # the kept activations fit the HBM budget).
        self.recompute = "auto"
        self.recompute_budget_bytes: int | None = None   # "auto": None = free HBM minus a reserve
        self.recompute_reserve_bytes = 24 << 30
        self.last_recompute_plan: list[bool] = []
        self._auto_plan = None      # (shape/budget key, plan) of the last "auto" decision
        # Whether the clean stream's final hidden states are computed. With False, the last layer
        # of the clean stream produces only the K/V the noisy stream reads (its attention, o
        # projection and MLP, and the final norm, feed nothing else), and the clean rows of the
        # output are zeros: for callers whose loss reads no teacher (CE on data targets).
        self.clean_final_needed = True

    def _rope_tables(self, P: int):
        """cos / sin tables of the positions < P (kept, and reused for smaller P)."""
        cached = getattr(self, "_rope_cache", None)
        if cached is None or cached[0] < P:
            cached = (P, *K.rope_table(P, self.inv_freq))
            self._rope_cache = cached
        return cached[1], cached[2]

    def recompute_plan(self, rows: int, rank: int, elem: int) -> list[bool]:
        """Which noisy-stream layers keep only their input for the backward (recompute) this step.
        "auto" keeps as many layers' activations as the budget allows and recomputes the rest,
        spread evenly over the depth."""
        n = len(self.layers)
        if self.recompute is True:
            plan = [True] * n
        elif not self.recompute:
            plan = [False] * n
        elif self.recompute == "auto":
            key = (rows, rank, elem, self.recompute_budget_bytes, self.recompute_reserve_bytes)
            if self._auto_plan is not None and self._auto_plan[0] == key:
                self.last_recompute_plan = list(self._auto_plan[1])
                return self.last_recompute_plan
            per_layer = Lyr.saved_bytes_per_row(self.geo, rank, elem) * rows
            input_only = self.geo.H * elem * rows
            budget = self.recompute_budget_bytes
            if budget is None:
                # free HBM plus what torch's allocator holds unused (the previous step's activations)
                dev = self.embed_tokens.weight.device
                free, _ = torch.cuda.mem_get_info(dev)
                cached = torch.cuda.memory_reserved(dev) - torch.cuda.memory_allocated(dev)
                budget = free + cached - self.recompute_reserve_bytes
            if budget >= n * per_layer:
                keep = n
            else:
                keep = max(0, min(n, int((budget - n * input_only) // max(per_layer - input_only, 1))))
            plan = [False] * n
            drop = n - keep
            for i in range(drop):                 # recompute `drop` layers spread over the depth
                plan[(i * n) // drop] = True
            self._auto_plan = (key, list(plan))
        else:
            raise ValueError(f"recompute must be True, False or 'auto', got {self.recompute!r}")
        self.last_recompute_plan = plan
        return plan

    def forward(self, input_ids=None, attention_mask=None, position_ids=None, output_attentions=False,
                output_hidden_states=False, return_dict=True, use_cache=False, **kwargs):
        del output_attentions, output_hidden_states, return_dict, use_cache, kwargs
        mask = attention_mask
        if not isinstance(mask, BlockDiffusionMask):
            raise TypeError("UnoQwen3Model expects the BlockDiffusionMask produced by prepare_for_bd_training.")
        B, L = mask.B, mask.L
        if input_ids is not None and tuple(input_ids.shape) != (B, 2 * L):
            raise RuntimeError(f"input_ids shape {tuple(input_ids.shape)} does not match the mask ({B}, {2 * L}).")
        lora = self._uno_lora
        if lora is not None:
            lora.sync_for_forward()
            gate = lora.token_mask
            if gate is None:
                raise RuntimeError("Set the Uno LoRA token mask before the model forward.")
            if tuple(gate.shape) != (B, 2 * L):
                raise RuntimeError("Uno LoRA mask and activation shapes differ: "
                                   f"mask={tuple(gate.shape)}, output={(B, 2 * L)}.")
            # The layout step hands the same region tensor to the router and to the mask, so the
            # identity test settles the usual case without a device comparison.
            if gate is not mask.region and not torch.equal(gate.to(mask.region.device), mask.region):
                raise RuntimeError("The two-stream decoder requires the LoRA token mask to be the noisy region "
                                   "of the block-diffusion layout.")
        g = self.geo
        sc = Lyr.StreamContext(mask.pos_stream, self.inv_freq, mask.iv_noisy, mask.iv_clean, [], [])
        sc.rope_cos, sc.rope_sin = self._rope_tables(max(L, getattr(mask, "max_pos", L - 1) + 1))
        lws = [layer.weights() for layer in self.layers]
        emb = self.embed_tokens.weight
        with torch.no_grad():
            hc = K.embedding(mask.clean_ids, emb)
            for li, lw in enumerate(lws):
                if li == len(lws) - 1 and not self.clean_final_needed:
                    k, v = Lyr.clean_layer_kv(hc, lw, g, sc)
                    hc = None
                else:
                    hc, k, v = Lyr.clean_layer(hc, lw, g, sc)
                sc.clean_k.append(k)
                sc.clean_v.append(v)
            if hc is not None:
                clean_final, _ = K.rmsnorm_fwd(hc, self.norm.weight, g.eps)
            else:
                clean_final = torch.zeros((mask.B * mask.L, g.H), device=emb.device, dtype=emb.dtype)
            del hc
        hn = K.embedding(mask.noisy_ids, emb)
        if lora is None:
            raise RuntimeError("The Uno decoder needs a LoRA adapter attached (create_lora_model).")
        plan = self.recompute_plan(hn.shape[0], lora.rank, hn.element_size())
        for li, lw in enumerate(lws):
            hn = Lyr.NoisyLayer.apply(hn, lora.anchor, lw, lora, li, g, sc, plan[li])
        noisy_final = Lyr.FinalNorm.apply(hn, self.norm.weight, g.eps, lora.anchor)
        hidden = Lyr.ScatterStreams.apply(noisy_final, clean_final, mask.noisy_src, mask.clean_src)
        out = hidden.view(B, 2 * L, g.H)
        # The two streams themselves, for extract_uno_regions: the same rows as out[region] and
        # out[~region], and the gradient then reaches the decoder without a scatter and a gather.
        out._uno_streams = (noisy_final, clean_final, mask.region)
        return UnoModelOutput(out)


class UnoQwen3ForCausalLM(nn.Module):
    def __init__(self, cfg: UnoQwen3Config, device="cuda", dtype=torch.bfloat16):
        super().__init__()
        self.config = cfg
        self.dtype = dtype
        self.noise = cfg.noise
        self.model = UnoQwen3Model(cfg, device, dtype)
        e = dict(device=device, dtype=dtype)
        w = torch.zeros(cfg.vocab_size, cfg.hidden_size, **e)
        self.lm_head = UnoLMHead(w, torch.zeros(cfg.hidden_size, cfg.vocab_size, **e))
        self._bd_step = 0
        self._layout = None      # (model positions, region mask) of the last prepare_uno_layout
        self._staged = None      # prepared batch for the next forward (stage_prepared_batch)

    @property
    def device(self):
        return self.lm_head.weight.device

    # ---- weights ---------------------------------------------------------------------------
    @torch.no_grad()
    def load_weights(self, params: dict) -> None:
        """Loads HF-style names (model.layers.N.self_attn.q_proj.weight, ..., lm_head.weight)."""
        own = dict(self.named_parameters())
        for name, value in params.items():
            if name not in own:
                raise KeyError(f"unknown weight {name}")
            own[name].copy_(value.to(own[name].dtype))
        self.refresh_transposed()

    @torch.no_grad()
    def refresh_transposed(self) -> None:
        for layer in self.model.layers:
            layer.refresh_transposed()
        self.lm_head.weight_t.copy_(self.lm_head.weight.t())

    @torch.no_grad()
    def random_init(self, seed: int, std: float = 0.02) -> None:
        """N(0, std) for every projection, embedding and LM head; unit norms (on device)."""
        gen = torch.Generator(device=self.device).manual_seed(seed)
        for name, p in self.named_parameters():
            if name.endswith("norm.weight") or "layernorm" in name:
                p.fill_(1.0)
        for layer in self.model.layers:
            for buf in (layer.w_qkv, layer.w_o, layer.w_gu, layer.w_d):
                buf.normal_(0.0, std, generator=gen)
        self.model.embed_tokens.weight.normal_(0.0, std, generator=gen)
        self.lm_head.weight.normal_(0.0, std, generator=gen)
        self.refresh_transposed()

    # ---- the reference's model-side call contract ---------------------------------------------
    def remember_layout(self, model_position_ids: torch.Tensor, region: torch.Tensor) -> None:
        """Called by prepare_uno_layout: a later prepare_for_bd_training on the same positions
        writes its region into this tensor, so the router's mask and the attention mask are one
        object."""
        self._layout = (model_position_ids, region)

    def prepare_for_bd_training(self, input_ids, model_position_ids, prompt_mask, *, step: int | None = None):
        """Noises non-prompt tokens per block, builds the [noisy | clean] concatenation and the
        block-diffusion attention mask (call contract: training/trainer.py:198-209)."""
        cfg = self.config
        if step is None:
            step = self._bd_step
        self._bd_step = step + 1
        region = None
        if self._layout is not None and self._layout[0] is model_position_ids:
            region = self._layout[1]
        self._layout = None
        return bd_prepare(input_ids, model_position_ids, prompt_mask, block_size=int(cfg.block_size),
                          mask_token_id=cfg.resolved_mask_token_id, noise=cfg.noise or "uniform",
                          intra_block=cfg.intra_block, seed=cfg.noise_seed, step=step, device=self.device,
                          region=region)

    @contextlib.contextmanager
    def stage_prepared_batch(self, concatenated_input_ids, concatenated_position_ids, attention_mask):
        """Within the block, a forward of this model (through any wrapper) runs the decoder on the
        prepared [noisy | clean] batch and returns {"hidden_states": (last_hidden_state,)}."""
        if self._staged is not None:
            raise RuntimeError("a prepared batch is already staged on this model")
        self._staged = (concatenated_input_ids, concatenated_position_ids, attention_mask)
        try:
            yield
        finally:
            self._staged = None

    def forward(self, *args, **kwargs):
        if self._staged is None:
            raise NotImplementedError(
                "UnoQwen3ForCausalLM runs the Uno step only: stage a prepared block-diffusion batch "
                "(run_prepared_uno_forward) before calling it.")
        ids, pos, mask = self._staged
        out = self.model(input_ids=ids, attention_mask=mask, position_ids=pos, output_attentions=False,
                         output_hidden_states=False, return_dict=True, use_cache=False)
        return {"hidden_states": (out.last_hidden_state,)}


# ------------------------------------------------------------------------------------------
# LoRA adapter (PEFT-compatible names and shapes)
# ------------------------------------------------------------------------------------------
class LoraAdapterModel(nn.Module):
    """PEFT LoraModel analogue: ``.model`` is the wrapped base model."""

    def __init__(self, model):
        super().__init__()
        self.model = model

    def forward(self, *args, **kwargs):
        return self.model(*args, **kwargs)


class UnoLoraModel(nn.Module):
    """PeftModelForCausalLM analogue. Trainable tensors are exactly the lora_A / lora_B weights,
    named ``base_model.model.model.layers.N.{self_attn,mlp}.X_proj.lora_{A,B}.default.weight``."""

    def __init__(self, base: UnoQwen3ForCausalLM, rank: int, alpha: float, dropout: float = 0.0,
                 init: str = "gaussian_b", seed: int = 0, b_std: float = 0.02, targets=MODULES):
        super().__init__()
        if dropout != 0.0:
            raise NotImplementedError("LoRA dropout is not supported by the fused path (Uno uses 0.0).")
        self.base_model = LoraAdapterModel(base)
        self.state = LoraState(base.config, rank, alpha, base.device, base.dtype, targets=targets)
        self.state.token_mask = None
        base.model._uno_lora = self.state
        st = self.state
        for li, layer in enumerate(base.model.layers):
            for name in st.targets:
                mod = getattr(layer.self_attn if name in ("q_proj", "k_proj", "v_proj", "o_proj") else layer.mlp, name)
                mod.lora_A = nn.ModuleDict({"default": _LoraWeight(st.a_view(st.master, li, name),
                                                                   st.a_view(st.grad, li, name), st)})
                mod.lora_B = nn.ModuleDict({"default": _LoraWeight(st.b_view(st.master, li, name),
                                                                   st.b_view(st.grad, li, name), st)})
                mod.use_dora = {"default": False}
                mod.scaling = {"default": st.scale}
                mod.r = {"default": st.rank}
        self.init_lora(init, seed, b_std)

    @torch.no_grad()
    def init_lora(self, init: str, seed: int, b_std: float = 0.02) -> None:
        """A ~ kaiming-uniform(a=sqrt(5)) = U(+-1/sqrt(in)); B ~ N(0, b_std) ("gaussian_b") or 0 ("zeros_b")."""
        st = self.state
        gen = torch.Generator(device=st.device).manual_seed(seed)
        for li in range(len(st.slots)):
            for name in st.targets:
                a = st.a_view(st.master, li, name)
                bound = 1.0 / a.shape[1] ** 0.5
                a.uniform_(-bound, bound, generator=gen)
                b = st.b_view(st.master, li, name)
                if init == "gaussian_b":
                    b.normal_(0.0, b_std, generator=gen)
                elif init == "zeros_b":
                    b.zero_()
                else:
                    raise ValueError(f"unknown LoRA init {init!r}")
        st.refresh_copies()

    @torch.no_grad()
    def load_lora(self, tensors: dict) -> None:
        """Loads {'model.layers.N....X_proj.lora_A.weight': tensor} (PEFT adapter names). The set
        must be complete: every adapter tensor exactly once, with its exact shape; a partial or
        mismatched file raises before anything is written."""
        def key(name: str) -> str:
            return name.replace("base_model.model.", "", 1).replace(".default", "")

        own = {key(n): p for n, p in self.named_parameters() if p.requires_grad}
        given = {}
        for k, v in tensors.items():
            kk = key(k)
            if kk not in own:
                raise KeyError(f"unknown LoRA tensor {k}")
            if kk in given:
                raise ValueError(f"LoRA tensor {kk} given twice")
            if tuple(v.shape) != tuple(own[kk].shape):
                raise ValueError(f"LoRA tensor {k} has shape {tuple(v.shape)}, expected {tuple(own[kk].shape)}")
            given[kk] = v
        missing = sorted(set(own) - set(given))
        if missing:
            raise ValueError(f"adapter is incomplete: {len(missing)} of {len(own)} LoRA tensors missing "
                             f"(first: {missing[0]})")
        for kk, v in given.items():
            own[kk].copy_(v.to(own[kk].dtype))
        self.state.refresh_copies()

    def lora_tensors(self) -> dict:
        return {n.replace(".default", ""): p for n, p in self.named_parameters() if p.requires_grad}

    def get_base_model(self):
        return self.base_model.model

    def forward(self, *args, **kwargs):
        return self.base_model(*args, **kwargs)

    def __getattr__(self, name):
        try:
            return super().__getattr__(name)
        except AttributeError:
            return getattr(self.base_model.model, name)
