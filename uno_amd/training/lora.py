"""LoRA attachment and token-conditional routing (semantics of training/lora.py in the reference).

The adapters are PEFT-shaped (A [r, in], B [out, r], fp32, scaling alpha/r, no dropout), stored
flat (uno_amd.adapter.LoraState). ``TokenwiseLoraRouter`` keeps the reference's interface: the
token mask it is given gates the low-rank update per row, which the fused GEMMs apply.
"""
from __future__ import annotations

import json
from collections import Counter
from dataclasses import dataclass
from pathlib import Path
from typing import Iterable

import torch

from .config import LoraSettings
from .constants import DEFAULT_MODEL_ID, DEFAULT_MODEL_REVISION, SUPPORTED_LORA_MODULES

# One-letter names of the attention projections, usable as a compact target string ("qkvo").
_LETTER_TARGETS = {"q": "q_proj", "k": "k_proj", "v": "v_proj", "o": "o_proj"}


def resolve_lora_targets(specification: str) -> tuple[str, ...]:
    """Projection names from a target specification: "all", a string of attention letters
    ("qv", "qkvo"), or a comma-separated list of projection names. Errors and their text follow
    training/lora.py:14-43."""
    text = specification.strip().lower()
    if text == "all":
        return tuple(SUPPORTED_LORA_MODULES)
    if text and set(text) <= _LETTER_TARGETS.keys():
        if len(set(text)) != len(text):
            raise ValueError(f"LoRA target shorthand contains duplicates: {specification!r}.")
        return tuple(_LETTER_TARGETS[c] for c in text)
    names = tuple(part.strip() for part in specification.split(",") if part.strip())
    if not names:
        raise ValueError("LoRA targets cannot be empty.")
    unknown = sorted(set(names) - set(SUPPORTED_LORA_MODULES))
    if unknown:
        raise ValueError(f"Unsupported LoRA target(s): {unknown}. Supported projection names are "
                         f"{list(SUPPORTED_LORA_MODULES)}.")
    if len(set(names)) != len(names):
        raise ValueError(f"LoRA target list contains duplicates: {specification!r}.")
    return names


def validate_target_modules(model, targets: Iterable[str]) -> dict[str, int]:
    """Every target must name exactly one module per decoder layer; returns the counts
    (training/lora.py:46-63)."""
    layers = getattr(getattr(model, "config", None), "num_hidden_layers", None)
    if type(layers) is not int or layers <= 0:
        raise RuntimeError("The base model must declare config.num_hidden_layers.")
    leaf_names = Counter(name.rsplit(".", 1)[-1] for name, _ in model.named_modules() if name)
    counts = {t: leaf_names.get(t, 0) for t in targets}
    off = {t: c for t, c in counts.items() if c != layers}
    if off:
        raise RuntimeError("Requested LoRA projections are not present exactly once per transformer "
                           f"layer (expected {layers} each): {off}.")
    return counts


def create_lora_model(model, settings: LoraSettings, *, init: str = "gaussian_b", seed: int = 0):
    """Attaches the only trainable weights of Uno training; returns (lora_model, targets)."""
    from ..model import UnoLoraModel

    settings.validate()
    targets = resolve_lora_targets(settings.target)
    validate_target_modules(model, targets)
    lora_model = UnoLoraModel(model, settings.rank, settings.resolved_alpha, settings.dropout, init=init, seed=seed,
                              targets=targets)
    validate_only_lora_trainable(lora_model)
    return lora_model, targets


def validate_only_lora_trainable(model) -> tuple[int, int]:
    """Only lora_A / lora_B tensors may train; returns (trainable, total) parameter counts."""
    params = list(model.named_parameters())
    trainable = [(n, p) for n, p in params if p.requires_grad]
    if not trainable:
        raise RuntimeError("No trainable LoRA tensors were found.")
    other = [n for n, _ in trainable if "lora_A" not in n and "lora_B" not in n]
    if other:
        raise RuntimeError(f"Only LoRA A/B tensors may be trainable; found {other[:5]}.")
    return sum(p.numel() for _, p in trainable), sum(p.numel() for _, p in params)


def make_saved_adapter_portable(adapter_dir) -> None:
    """Points a saved adapter's metadata at the pinned Hub base model (adapter_config.json and,
    when present, the model card's base_model line) instead of a local cache path."""
    adapter_dir = Path(adapter_dir)
    cfg_path = adapter_dir / "adapter_config.json"
    cfg = json.loads(cfg_path.read_text())
    cfg.update(base_model_name_or_path=DEFAULT_MODEL_ID, revision=DEFAULT_MODEL_REVISION)
    cfg_path.write_text(json.dumps(cfg, indent=2, sort_keys=True) + "\n")
    card = adapter_dir / "README.md"
    if card.is_file():
        text = card.read_text().splitlines()
        hit = next((i for i, line in enumerate(text) if line.startswith("base_model:")), None)
        if hit is not None:
            text[hit] = f"base_model: {DEFAULT_MODEL_ID}"
            card.write_text("\n".join(text) + "\n")


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
