"""Objective and LoRA settings (semantics of training/config.py:23-77 in the reference)."""
from __future__ import annotations

import math
from dataclasses import dataclass
from typing import Literal

from .constants import DEFAULT_CE_ALPHA, DEFAULT_KL_BETA, DEFAULT_LORA_ALPHA_RATIO, DEFAULT_TV_GAMMA

CeTarget = Literal["teacher", "ground_truth"]


@dataclass(frozen=True)
class UnoObjectiveConfig:
    """Loss weights alpha (CE), beta (reverse KL), gamma (TV) and the CE target source."""

    ce_target: CeTarget = "teacher"
    noise: str = "uniform"
    reverse_kl: bool = True
    teacher_base_only: bool = True
    ce_weight: float = DEFAULT_CE_ALPHA
    kl_weight: float = DEFAULT_KL_BETA
    tv_weight: float = DEFAULT_TV_GAMMA

    def validate(self) -> None:
        if self.ce_target not in ("teacher", "ground_truth"):
            raise ValueError("ce_target must be either 'teacher' or 'ground_truth'.")
        if self.noise != "uniform":
            raise ValueError("Public Uno training supports uniform noise only.")
        if not self.reverse_kl:
            raise ValueError("Public Uno training supports reverse KL only.")
        if not self.teacher_base_only:
            raise ValueError("The Uno teacher must use frozen base weights only.")
        weights = (self.ce_weight, self.kl_weight, self.tv_weight)
        for w in weights:
            if isinstance(w, bool) or not isinstance(w, (int, float)):
                raise ValueError("Uno loss weights must be numeric.")
            if not math.isfinite(w) or w < 0:
                raise ValueError("Uno loss weights must be finite and non-negative.")
        if max(weights) <= 0:
            raise ValueError("At least one Uno loss weight must be positive.")

    @property
    def internal_ce_target(self) -> str:
        self.validate()
        return {"teacher": "clean_argmax", "ground_truth": "data"}[self.ce_target]


@dataclass(frozen=True)
class LoraSettings:
    target: str
    rank: int
    alpha: int | None
    dropout: float

    @property
    def resolved_alpha(self) -> int:
        return DEFAULT_LORA_ALPHA_RATIO * self.rank if self.alpha is None else self.alpha

    def validate(self) -> None:
        if self.rank <= 0:
            raise ValueError("LoRA rank must be positive.")
        if self.alpha is not None and self.alpha <= 0:
            raise ValueError("LoRA alpha must be positive.")
        if not (0.0 <= self.dropout < 1.0):
            raise ValueError("LoRA dropout must be in [0, 1).")
