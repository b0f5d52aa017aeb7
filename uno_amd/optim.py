"""Fused multi-tensor AdamW over the flat LoRA state (one optional clip pass + one update pass).

Semantics: torch.optim.AdamW (training/train.py:282-288: betas (0.9, 0.999), eps 1e-8, weight
decay 0) over every lora_A / lora_B tensor, optionally preceded by
torch.nn.utils.clip_grad_norm_(max_norm) (the Trainer's max_grad_norm 1.0). It is a
torch.optim.Optimizer, so LR schedulers and the HF Trainer drive it unchanged, but the update
is one kernel over the adapter's flat fp32 buffers instead of a loop over 7 x layers x 2 tensors;
the same pass refreshes the bf16 compute copies the GEMMs read. The clip coefficient stays on the
device (no host synchronisation).
"""
from __future__ import annotations

import torch

from . import _native as N
from .adapter import LoraState

_FROM_CONSTRUCTOR = object()


class FusedLoraAdamW(torch.optim.Optimizer):
    def __init__(self, state: LoraState, lr: float = 1e-4, betas=(0.9, 0.999), eps: float = 1e-8,
                 weight_decay: float = 0.0, max_grad_norm: float | None = 1.0):
        params = [p for p, _, _ in state._bindings]
        if not params:
            raise RuntimeError("FusedLoraAdamW: the adapter has no bound LoRA parameters")
        super().__init__(params, dict(lr=lr, betas=tuple(betas), eps=eps, weight_decay=weight_decay))
        self.lora_state = state
        self.max_grad_norm = max_grad_norm
        self.nparts = 1024
        dev = state.device
        self._parts = torch.empty(self.nparts, device=dev, dtype=torch.float32)
        self.clip = torch.ones(2, device=dev, dtype=torch.float32)   # [grad norm, clip coef]

    def _hyper(self):
        """The flat pass takes one set of hyper-parameters: every group must agree."""
        keys = ("lr", "betas", "eps", "weight_decay")
        first = self.param_groups[0]
        for g in self.param_groups[1:]:
            if any(g[k] != first[k] for k in keys):
                raise ValueError("FusedLoraAdamW updates all LoRA tensors in one pass; its parameter groups "
                                 "must share lr, betas, eps and weight_decay")
        return first["lr"], first["betas"], first["eps"], first["weight_decay"]

    @torch.no_grad()
    def step(self, closure=None, lr: float | None = None, max_grad_norm=_FROM_CONSTRUCTOR):
        """One AdamW update of every adapter tensor; ``max_grad_norm`` (default: the constructor's)
        clips the global gradient norm first, None skips the clip."""
        if max_grad_norm is _FROM_CONSTRUCTOR:
            max_grad_norm = self.max_grad_norm
        loss = None
        if closure is not None:
            with torch.enable_grad():
                loss = closure()
        st = self.lora_state
        bound = [p.grad is g for p, g, _ in st._bindings]
        if not any(bound):
            return loss          # no gradients at all: torch's AdamW leaves every tensor untouched
        if not all(bound):
            st.sync_for_forward()   # adopt replaced / cleared gradients into the flat buffer
        glr, (b1, b2), eps, wd = self._hyper()
        lr = glr if lr is None else lr
        clip_ptr = None
        if max_grad_norm is not None:
            N.call("unok_grad_clip_coef", st.numel, N.ptr(st.grad), N.ptr(self._parts), self.nparts,
                   float(max_grad_norm), N.ptr(self.clip), N.stream())
            clip_ptr = N.ptr(self.clip)
        st.step += 1
        N.call("unok_adamw_step", st.numel, N.ptr(st.master), N.ptr(st.grad), N.ptr(st.exp_avg),
               N.ptr(st.exp_avg_sq), clip_ptr, float(lr), float(b1), float(b2), float(eps), float(wd), st.step,
               N.dtype_code(st.compute_dtype), N.ptr(st.copy), st.n_a, float(st.scale), N.stream())
        # The kernel wrote master through its pointer (no version bump) and the bf16 copies in the
        # same pass; the transposed copies follow here, so the copies stay current.
        st.refresh_transposes()
        return loss

    def zero_grad(self, set_to_none: bool = True) -> None:
        """Zeroes the flat gradient buffer in one pass; the per-tensor views stay bound (a later
        forward would rebind and zero them anyway), whatever ``set_to_none`` says."""
        del set_to_none
        st = self.lora_state
        st.grad.zero_()
        for p, g, _ in st._bindings:
            if p.grad is not g:
                p.grad = g

    def state_dict(self):
        st = self.lora_state
        return {"param_groups": [{k: v for k, v in g.items() if k != "params"} for g in self.param_groups],
                "lora_flat": {"step": st.step, "exp_avg": st.exp_avg, "exp_avg_sq": st.exp_avg_sq}}

    def load_state_dict(self, state_dict) -> None:
        st = self.lora_state
        flat = state_dict["lora_flat"]
        for name in ("exp_avg", "exp_avg_sq"):
            if tuple(flat[name].shape) != (st.numel,):
                raise ValueError(f"{name} holds {flat[name].numel()} values, the adapter {st.numel}")
        st.exp_avg.copy_(flat["exp_avg"])
        st.exp_avg_sq.copy_(flat["exp_avg_sq"])
        st.step = int(flat["step"])
        groups = state_dict["param_groups"]
        if len(groups) != len(self.param_groups):
            raise ValueError("optimizer state has a different number of parameter groups")
        for g, saved in zip(self.param_groups, groups):
            g.update({k: v for k, v in saved.items() if k != "params"})

    @property
    def grad_norm(self) -> torch.Tensor:
        return self.clip[0]
