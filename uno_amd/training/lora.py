"""LoRA attachment and token-conditional routing (semantics of training/lora.py in the reference).

The adapters are PEFT-shaped (A [r, in], B [out, r], fp32, scaling alpha/r, no dropout), stored
flat (uno_amd.adapter.LoraState). ``TokenwiseLoraRouter`` keeps the reference's interface: the
token mask it is given gates the low-rank update per row, which the fused GEMMs apply.
"""
from __future__ import annotations

import json
from dataclasses import dataclass
from pathlib import Path
from typing import Iterable

import torch

from .config import LoraSettings
from .constants import DEFAULT_MODEL_ID, DEFAULT_MODEL_REVISION, SUPPORTED_LORA_MODULES

_SHORTHAND = {"q": "q_proj", "k": "k_proj", "v": "v_proj", "o": "o_proj"}


def resolve_lora_targets(specification: str) -> tuple[str, ...]:
    spec = specification.strip().lower()
    if spec == "all":
        return SUPPORTED_LORA_MODULES
    if spec and set(spec) <= set(_SHORTHAND):
        if len(set(spec)) != len(spec):
            raise ValueError(f"LoRA target shorthand contains duplicates: {specification!r}.")
        return tuple(_SHORTHAND[c] for c in spec)
    targets = tuple(p.strip() for p in specification.split(",") if p.strip())
    if not targets:
        raise ValueError("LoRA targets cannot be empty.")
    bad = sorted(set(targets) - set(SUPPORTED_LORA_MODULES))
    if bad:
        raise ValueError(f"Unsupported LoRA target(s): {bad}. Supported projection names are "
                         f"{list(SUPPORTED_LORA_MODULES)}.")
    if len(set(targets)) != len(targets):
        raise ValueError(f"LoRA target list contains duplicates: {specification!r}.")
    return targets


def validate_target_modules(model, targets: Iterable[str]) -> dict[str, int]:
    targets = tuple(targets)
    n_layers = getattr(model.config, "num_hidden_layers", None)
    if not isinstance(n_layers, int) or n_layers <= 0:
        raise RuntimeError("The base model must declare config.num_hidden_layers.")
    counts = {t: sum(name.endswith(f".{t}") for name, _ in model.named_modules()) for t in targets}
    wrong = {t: c for t, c in counts.items() if c != n_layers}
    if wrong:
        raise RuntimeError("Requested LoRA projections are not present exactly once per transformer layer "
                           f"(expected {n_layers} each): {wrong}.")
    return counts


def create_lora_model(model, settings: LoraSettings, *, init: str = "gaussian_b", seed: int = 0):
    """Attaches the only trainable weights of Uno training; returns (lora_model, targets)."""
    from ..model import UnoLoraModel

    settings.validate()
    targets = resolve_lora_targets(settings.target)
    validate_target_modules(model, targets)
    lora_model = UnoLoraModel(model, settings.rank, settings.resolved_alpha, settings.dropout, init=init, seed=seed)
    if tuple(sorted(targets)) != tuple(sorted(lora_model.state.targets)):
        raise NotImplementedError(f"targets {targets} are not supported by the fused path")
    validate_only_lora_trainable(lora_model)
    return lora_model, targets


def validate_only_lora_trainable(model) -> tuple[int, int]:
    trainable, n_train, n_total = [], 0, 0
    for name, p in model.named_parameters():
        n_total += p.numel()
        if p.requires_grad:
            trainable.append(name)
            n_train += p.numel()
    if not trainable:
        raise RuntimeError("No trainable LoRA tensors were found.")
    bad = [n for n in trainable if "lora_A" not in n and "lora_B" not in n]
    if bad:
        raise RuntimeError(f"Only LoRA A/B tensors may be trainable; found {bad[:5]}.")
    return n_train, n_total


def make_saved_adapter_portable(adapter_dir) -> None:
    adapter_dir = Path(adapter_dir)
    cfg_path = adapter_dir / "adapter_config.json"
    cfg = json.loads(cfg_path.read_text())
    cfg["base_model_name_or_path"] = DEFAULT_MODEL_ID
    cfg["revision"] = DEFAULT_MODEL_REVISION
    cfg_path.write_text(json.dumps(cfg, indent=2, sort_keys=True) + "\n")
    readme = adapter_dir / "README.md"
    if readme.is_file():
        lines = readme.read_text().splitlines()
        for i, line in enumerate(lines):
            if line.startswith("base_model:"):
                lines[i] = f"base_model: {DEFAULT_MODEL_ID}"
                readme.write_text("\n".join(lines) + "\n")
                break


def save_adapter(lora_model, adapter_dir) -> Path:
    """Writes a PEFT-format adapter (adapter_model.safetensors + adapter_config.json) whose tensor
    names are those the inference loader reads (base_model.model.model.layers.N....lora_A.weight)."""
    from safetensors.torch import save_file

    adapter_dir = Path(adapter_dir)
    adapter_dir.mkdir(parents=True, exist_ok=True)
    tensors = {n: p.detach().float().cpu().contiguous() for n, p in lora_model.lora_tensors().items()}
    save_file(tensors, str(adapter_dir / "adapter_model.safetensors"))
    st = lora_model.state
    cfg = {"peft_type": "LORA", "task_type": "CAUSAL_LM", "r": st.rank, "lora_alpha": st.alpha,
           "lora_dropout": 0.0, "bias": "none", "target_modules": list(st.targets),
           "base_model_name_or_path": DEFAULT_MODEL_ID, "revision": DEFAULT_MODEL_REVISION,
           "inference_mode": False, "use_dora": False}
    (adapter_dir / "adapter_config.json").write_text(json.dumps(cfg, indent=2, sort_keys=True) + "\n")
    return adapter_dir


def load_adapter(lora_model, adapter_dir) -> None:
    from safetensors.torch import load_file

    lora_model.load_lora(load_file(str(Path(adapter_dir) / "adapter_model.safetensors")))


@dataclass
class TokenwiseLoraRouter:
    """Gates the LoRA update on clean teacher rows: only rows where the mask is True get it."""

    model: object

    def __post_init__(self) -> None:
        self.token_mask: torch.Tensor | None = None
        self.handles = []
        validate_only_lora_trainable(self.model)
        states = []
        for module in self.model.modules():
            if getattr(module, "lora_A", None) is None:
                continue
            if any(getattr(module, "use_dora", {}).values()):
                raise RuntimeError("Token-conditional Uno routing does not support DoRA.")
            self.handles.append(module)
        if not self.handles:
            raise RuntimeError("No PEFT LoRA-A layers were found for conditional routing.")
        m = self.model
        while hasattr(m, "module"):
            m = m.module
        state = getattr(m, "state", None)
        if state is not None:
            states.append(state)
        self._states = states

    def set_token_mask(self, token_mask: torch.Tensor) -> None:
        self.token_mask = token_mask
        for st in self._states:
            st.token_mask = token_mask

    def close(self) -> None:
        for st in self._states:
            st.token_mask = None
        self.handles.clear()
