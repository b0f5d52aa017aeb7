"""Fused multi-tensor AdamW over the flat LoRA state (one clip pass + one update pass).

Semantics: torch.nn.utils.clip_grad_norm_(max_norm) followed by torch.optim.AdamW with
weight_decay (training/train.py:282-288: betas (0.9, 0.999), eps 1e-8, wd 0, max_grad_norm 1.0).
The clip coefficient stays on the device (no host synchronisation); the update pass also
refreshes the compute copies of the adapters.
"""
from __future__ import annotations

import torch

from . import _native as N
from .adapter import LoraState


class FusedLoraAdamW:
    def __init__(self, state: LoraState, lr: float = 1e-4, betas=(0.9, 0.999), eps: float = 1e-8,
                 weight_decay: float = 0.0, max_grad_norm: float | None = 1.0):
        self.state = state
        self.lr, self.betas, self.eps, self.weight_decay = lr, betas, eps, weight_decay
        self.max_grad_norm = max_grad_norm
        self.nparts = 1024
        dev = state.device
        self._parts = torch.empty(self.nparts, device=dev, dtype=torch.float32)
        self.clip = torch.ones(2, device=dev, dtype=torch.float32)   # [grad norm, clip coef]

    def step(self, lr: float | None = None) -> None:
        st = self.state
        lr = self.lr if lr is None else lr
        clip_ptr = None
        if self.max_grad_norm is not None:
            N.call("unok_grad_clip_coef", st.numel, N.ptr(st.grad), N.ptr(self._parts), self.nparts,
                   float(self.max_grad_norm), N.ptr(self.clip), N.stream())
            clip_ptr = N.ptr(self.clip)
        st.step += 1
        N.call("unok_adamw_step", st.numel, N.ptr(st.master), N.ptr(st.grad), N.ptr(st.exp_avg),
               N.ptr(st.exp_avg_sq), clip_ptr, float(lr), float(self.betas[0]), float(self.betas[1]),
               float(self.eps), float(self.weight_decay), st.step, N.dtype_code(st.compute_dtype), N.ptr(st.copy),
               st.n_a, float(st.scale), N.stream())
        st.refresh_transposes()

    def zero_grad(self, set_to_none: bool = False) -> None:
        del set_to_none   # gradients are views into the flat buffer and are always kept
        self.state.zero_grad()

    @property
    def grad_norm(self) -> torch.Tensor:
        return self.clip[0]
