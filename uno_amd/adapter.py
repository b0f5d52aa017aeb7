"""Flat storage of all LoRA adapters of a model (MI355X-first layout).

Every ``lora_A`` / ``lora_B`` tensor (PEFT shapes: A [r, in], B [out, r], fp32 master weights as
in training/lora.py:83-91) is a view into ONE flat fp32 buffer; gradients, AdamW moments and
the compute copies are parallel buffers with the same layout. The layout is

    [ A region: per layer  A_q A_k A_v A_o A_gate A_up A_down ]
    [ B region: per layer  B_q B_k B_v B_o B_gate B_up B_down ]

so that each fused projection's adapters are contiguous (A_qkv = [A_q; A_k; A_v] is a [3r, H]
matrix; B_qkv = [B_q; B_k; B_v] is [q+2kv, r]), the optimizer is one flat pass, and the
compute copy (B scaled by alpha/r) is refreshed by that same pass. Transposed compute copies
(A^T per group, (sB)^T per group) feed the data-gradient GEMMs and are rebuilt by one batched
transpose launch after every update. For the gate/up product with the SwiGLU epilogue, whose
weight rows alternate in blocks of 64 (64 gate rows, then the same features' up rows), sB of
gate/up is also kept in that row order with K = 2r columns: [sB_gate, 0] on gate rows and
[0, sB_up] on up rows, so one LoRA extension over h = x [A_gate; A_up]^T serves both.
"""
from __future__ import annotations

from dataclasses import dataclass

import torch

from . import _native as N

MODULES = ("q_proj", "k_proj", "v_proj", "o_proj", "gate_proj", "up_proj", "down_proj")
GROUPS = {"qkv": ("q_proj", "k_proj", "v_proj"), "o": ("o_proj",), "gu": ("gate_proj", "up_proj"),
          "d": ("down_proj",)}


def module_dims(cfg) -> dict[str, tuple[int, int]]:
    """(out, in) per projection."""
    H, d = cfg.hidden_size, cfg.head_dim
    q, kv, f = cfg.num_attention_heads * d, cfg.num_key_value_heads * d, cfg.intermediate_size
    return {"q_proj": (q, H), "k_proj": (kv, H), "v_proj": (kv, H), "o_proj": (H, q),
            "gate_proj": (f, H), "up_proj": (f, H), "down_proj": (H, f)}


@dataclass
class _Slot:
    a_off: int
    b_off: int
    out: int
    inp: int


class LoraState:
    def __init__(self, cfg, rank: int, alpha: float, device, compute_dtype: torch.dtype,
                 targets=MODULES):
        targets = tuple(targets)
        unknown = [t for t in targets if t not in MODULES]
        if not targets or unknown or len(set(targets)) != len(targets):
            raise ValueError(f"LoRA targets must be distinct names from {list(MODULES)}; got {list(targets)}.")
        self.cfg = cfg
        self.rank = int(rank)
        self.alpha = float(alpha)
        self.scale = self.alpha / self.rank
        # Every projection keeps its slot in the flat layout, so each fused group's adapters stay
        # contiguous; an untargeted projection's slot holds zeros and is never exposed as a
        # parameter. Its forward term s B (x A^T) and its gradients are then exactly zero, and
        # AdamW (no weight decay on a zero weight, zero moments) keeps it at zero.
        self.targets = targets
        self.compute_dtype = compute_dtype
        self.device = torch.device(device)
        dims = module_dims(cfg)
        r = self.rank
        self.slots: list[dict[str, _Slot]] = []
        a = 0
        for _ in range(cfg.num_hidden_layers):
            layer = {}
            for name in MODULES:
                out, inp = dims[name]
                layer[name] = _Slot(a, 0, out, inp)
                a += r * inp
            self.slots.append(layer)
        self.n_a = a
        b = a
        for layer in self.slots:
            for name in MODULES:
                layer[name].b_off = b
                b += layer[name].out * r
        self.numel = b
        f32 = dict(device=self.device, dtype=torch.float32)
        self.master = torch.zeros(self.numel, **f32)
        self.grad = torch.zeros(self.numel, **f32)
        self.exp_avg = torch.zeros(self.numel, **f32)
        self.exp_avg_sq = torch.zeros(self.numel, **f32)
        self.copy = torch.empty(self.numel, device=self.device, dtype=compute_dtype)
        self.copy_t = torch.empty(self.numel, device=self.device, dtype=compute_dtype)
        self.step = 0
        # master._version at the last refresh of the compute copies (None: never refreshed)
        self._copies_version = None
        # (parameter, gradient view, master address) of every lora_A / lora_B tensor
        self._bindings: list[tuple[torch.nn.Parameter, torch.Tensor, int]] = []
        self._build_transpose_jobs()
        self._build_gate_up_interleaved()
        # autograd anchor: the decoder's stream Functions take it as an input so that backward
        # runs; the LoRA gradients are accumulated straight into ``grad`` by the kernels.
        self.anchor = torch.zeros(1, **f32).requires_grad_(True)

    # ---- targets ----------------------------------------------------------------------
    def is_target(self, name: str) -> bool:
        return name in self.targets

    def group_active(self, group: str) -> bool:
        """Whether any projection of a fused group carries an adapter."""
        return any(n in self.targets for n in GROUPS[group])

    # ---- views of the fp32 master / grad ----------------------------------------------
    def a_view(self, buf: torch.Tensor, layer: int, name: str) -> torch.Tensor:
        s = self.slots[layer][name]
        return buf[s.a_off:s.a_off + self.rank * s.inp].view(self.rank, s.inp)

    def b_view(self, buf: torch.Tensor, layer: int, name: str) -> torch.Tensor:
        s = self.slots[layer][name]
        return buf[s.b_off:s.b_off + s.out * self.rank].view(s.out, self.rank)

    def group_a(self, buf: torch.Tensor, layer: int, group: str) -> torch.Tensor:
        names = GROUPS[group]
        first = self.slots[layer][names[0]]
        rows = self.rank * len(names)
        return buf[first.a_off:first.a_off + rows * first.inp].view(rows, first.inp)

    def group_b(self, buf: torch.Tensor, layer: int, group: str) -> torch.Tensor:
        names = GROUPS[group]
        first = self.slots[layer][names[0]]
        rows = sum(self.slots[layer][n].out for n in names)
        return buf[first.b_off:first.b_off + rows * self.rank].view(rows, self.rank)

    # ---- transposed compute copies ------------------------------------------------------
    def _build_transpose_jobs(self):
        jobs = []
        self._t_views = []
        tile = 0
        for li in range(len(self.slots)):
            views = {}
            for g in GROUPS:
                for kind in ("a", "b"):
                    src = self.group_a(self.copy, li, g) if kind == "a" else self.group_b(self.copy, li, g)
                    rows, cols = src.shape
                    src_off = src.storage_offset() - self.copy.storage_offset()
                    dst_off = src_off   # same footprint, transposed shape
                    jobs.append([src_off, rows, cols, dst_off, tile, 0, 0, 0])
                    tile += ((rows + 63) // 64) * ((cols + 63) // 64)
                    views[(g, kind)] = self.copy_t[dst_off:dst_off + rows * cols].view(cols, rows)
            self._t_views.append(views)
        self._jobs = torch.tensor(jobs, dtype=torch.int64, device=self.device)
        self._tiles = tile

    def _build_gate_up_interleaved(self):
        F, r, L = self.slots[0]["gate_proj"].out, self.rank, len(self.slots)
        self._sb_gu_i = None
        if F % 64 or L == 0:
            return
        # zero once; the refresh writes only the gate half of gate rows and the up half of up rows
        self._sb_gu_i = torch.zeros((L, F // 64, 2, 64, 2 * r), device=self.device, dtype=self.compute_dtype)
        lstride = self.slots[1]["gate_proj"].b_off - self.slots[0]["gate_proj"].b_off if L > 1 else 0
        for li in range(1, L):
            assert self.slots[li]["gate_proj"].b_off - self.slots[li - 1]["gate_proj"].b_off == lstride
        # sB_gate / sB_up of every layer as [L, 2, F/64, 64, r] (gate rows then up rows per layer)
        self._sb_gu_src = self.copy.as_strided((L, 2, F // 64, 64, r), (lstride, F * r, 64 * r, r, 1),
                                               self.copy.storage_offset() + self.slots[0]["gate_proj"].b_off)

    def _refresh_gate_up_interleaved(self) -> None:
        if self._sb_gu_i is None:
            return
        r = self.rank
        self._sb_gu_i[:, :, 0, :, :r].copy_(self._sb_gu_src[:, 0])
        self._sb_gu_i[:, :, 1, :, r:].copy_(self._sb_gu_src[:, 1])

    def sb_gu_i(self, layer: int) -> torch.Tensor | None:
        """sB of gate/up as [2F, 2r] in the interleaved row order (see the module docstring)."""
        if self._sb_gu_i is None:
            return None
        t = self._sb_gu_i[layer]
        return t.view(-1, t.shape[-1])

    def a_t(self, layer: int, group: str) -> torch.Tensor:
        """A_group^T [in, rows] compute copy."""
        return self._t_views[layer][(group, "a")]

    def sb_t(self, layer: int, group: str) -> torch.Tensor:
        """(s * B_group)^T [r, out_rows] compute copy."""
        return self._t_views[layer][(group, "b")]

    def a_c(self, layer: int, group: str) -> torch.Tensor:
        return self.group_a(self.copy, layer, group)

    def sb_c(self, layer: int, group: str) -> torch.Tensor:
        return self.group_b(self.copy, layer, group)

    def grad_a(self, layer: int, group: str) -> torch.Tensor:
        return self.group_a(self.grad, layer, group)

    def grad_b(self, layer: int, group: str) -> torch.Tensor:
        return self.group_b(self.grad, layer, group)

    def refresh_copies(self) -> None:
        """Rebuilds the compute copies from the master weights."""
        N.call("unok_cast_copy", N.dtype_code(self.compute_dtype), self.numel, self.n_a, float(self.scale),
               N.ptr(self.master), N.ptr(self.copy), N.stream())
        self.refresh_transposes()
        self._copies_version = self.master._version

    def bind_parameter(self, param: torch.nn.Parameter, grad_view: torch.Tensor) -> None:
        """Registers a lora_A / lora_B parameter (a view of ``master``) and its gradient view."""
        param.grad = grad_view
        self._bindings.append((param, grad_view, param.data_ptr()))

    def sync_for_forward(self) -> None:
        """Makes the adapters consistent whatever updated them since the last forward.

        * Weights: any in-place update of the parameters (torch optimizers, ``copy_``, init)
          advances the version counter that all views of ``master`` share; the compute copies
          are rebuilt when it moved. (Writes through ``param.data`` bypass the counter: call
          ``refresh_copies`` after them.) A parameter whose storage was replaced is an error,
          since the kernels read ``master``.
        * Gradients: the kernels accumulate into the flat ``grad`` buffer. A parameter whose
          ``.grad`` was set to None (``zero_grad(set_to_none=True)``) gets its view back, zeroed;
          one whose ``.grad`` was replaced by another tensor has that tensor's values copied in.
        """
        for param, _, addr in self._bindings:
            if param.data_ptr() != addr:
                raise RuntimeError("A LoRA parameter no longer views the adapter storage (its .data was "
                                   "replaced); update adapters in place instead.")
        if self.master._version != self._copies_version:
            self.refresh_copies()
        unbound = [(p, g) for p, g, _ in self._bindings if p.grad is not g]
        if not unbound:
            return
        if len(unbound) == len(self._bindings) and all(p.grad is None for p, _ in unbound):
            self.grad.zero_()
            for p, g in unbound:
                p.grad = g
            return
        with torch.no_grad():
            for p, g in unbound:
                if p.grad is None:
                    g.zero_()
                else:
                    if tuple(p.grad.shape) != tuple(g.shape):
                        raise RuntimeError(f"gradient of shape {tuple(p.grad.shape)} set on a LoRA tensor of "
                                           f"shape {tuple(g.shape)}")
                    g.copy_(p.grad)
                p.grad = g

    def refresh_transposes(self) -> None:
        N.call("unok_transpose_jobs", N.dtype_code(self.compute_dtype), N.ptr(self._jobs), self._jobs.shape[0],
               self._tiles, N.ptr(self.copy), N.ptr(self.copy_t), N.stream())
        self._refresh_gate_up_interleaved()

    def zero_grad(self) -> None:
        self.grad.zero_()
