"""Progressive block-size curriculum (the schedule the reference step reads through
``stage_for_step`` and ``set_model_block_size``, training/curriculum.py:109-112,150-156).

A plan is a list of (block size, token budget) stages consumed at a fixed number of tokens per
optimizer step. Stage boundaries are computed once, in steps, from the cumulative budgets
(boundary_i = floor(sum of budgets up to stage i / tokens_per_step)), and the block size of every
step is then a lookup into that table. The released schedule file
(training/configs/uno_3epoch_curriculum.yaml: tokens_per_step, sequence_length,
global_batch_size, seed, total_tokens, stages[{block_size, tokens}]) loads unchanged, and
``manifest``/``sha256`` describe the plan in the form the reference writes into its
curriculum-boundary checkpoints, so those checkpoints validate against this plan.
"""
from __future__ import annotations

import hashlib
import json
from dataclasses import dataclass
from itertools import accumulate
from pathlib import Path

import yaml


@dataclass(frozen=True)
class CurriculumStage:
    block_size: int
    token_budget: int
    start_step: int
    end_step: int


def _require_int(raw: dict, key: str, *, positive: bool = True, where: str = "curriculum") -> int:
    value = raw.get(key)
    if type(value) is not int:                       # bool is an int subclass and is rejected too
        raise ValueError(f"{where}: {key} must be an integer, got {value!r}.")
    if positive and value <= 0:
        raise ValueError(f"{where}: {key} must be positive, got {value}.")
    return value


class BlockCurriculumPlan:
    """Stages of strictly increasing block size, each at least one optimizer step long."""

    def __init__(self, *, tokens_per_step: int, sequence_length: int, global_batch_size: int, seed: int,
                 stages, source_path=None):
        self.tokens_per_step = tokens_per_step
        self.sequence_length = sequence_length
        self.global_batch_size = global_batch_size
        self.seed = seed
        self.stages = tuple(stages)
        self.source_path = source_path
        self._ends = [s.end_step for s in self.stages]
        self.checkpoint_reasons = {s.end_step: f"completed_block_size_{s.block_size}" for s in self.stages}

    # ---- construction ---------------------------------------------------------------------
    @classmethod
    def from_budgets(cls, budgets, *, tokens_per_step: int, sequence_length: int, global_batch_size: int,
                     seed: int = 0, source_path=None) -> "BlockCurriculumPlan":
        """``budgets``: (block_size, tokens) pairs in training order."""
        budgets = [(int(b), int(t)) for b, t in budgets]
        if not budgets:
            raise ValueError("A curriculum needs at least one stage.")
        if tokens_per_step != sequence_length * global_batch_size:
            raise ValueError(f"tokens_per_step ({tokens_per_step}) is not sequence_length x global_batch_size "
                             f"({sequence_length} x {global_batch_size}).")
        blocks = [b for b, _ in budgets]
        if any(b <= 0 for b in blocks) or any(later <= earlier for earlier, later in zip(blocks, blocks[1:])):
            raise ValueError(f"Block sizes must be positive and strictly increasing, got {blocks}.")
        if any(t <= 0 for _, t in budgets):
            raise ValueError("Every stage needs a positive token budget.")
        ends = [cum // tokens_per_step for cum in accumulate(t for _, t in budgets)]
        starts = [0] + ends[:-1]
        for (block, _), start, end in zip(budgets, starts, ends):
            if end <= start:
                raise ValueError(f"The block-size-{block} stage covers no full optimizer step.")
        stages = [CurriculumStage(b, t, s, e) for (b, t), s, e in zip(budgets, starts, ends)]
        return cls(tokens_per_step=tokens_per_step, sequence_length=sequence_length,
                   global_batch_size=global_batch_size, seed=seed, stages=stages, source_path=source_path)

    @classmethod
    def from_dict(cls, raw: dict, source_path: Path | None = None) -> "BlockCurriculumPlan":
        if not isinstance(raw, dict):
            raise ValueError("A curriculum must be a mapping.")
        if raw.get("replay"):
            raise ValueError("Replaying smaller block sizes is not supported.")
        items = raw.get("stages")
        if not isinstance(items, list) or not items:
            raise ValueError("Curriculum stages must be a non-empty list.")
        budgets = []
        for i, item in enumerate(items):
            if not isinstance(item, dict):
                raise ValueError(f"Curriculum stage {i} is not a mapping.")
            where = f"curriculum stage {i}"
            budgets.append((_require_int(item, "block_size", where=where), _require_int(item, "tokens", where=where)))
        plan = cls.from_budgets(budgets, tokens_per_step=_require_int(raw, "tokens_per_step"),
                                sequence_length=_require_int(raw, "sequence_length"),
                                global_batch_size=_require_int(raw, "global_batch_size"),
                                seed=_require_int(raw, "seed", positive=False), source_path=source_path)
        declared = raw.get("total_tokens")
        if declared is not None and declared != plan.total_tokens:
            raise ValueError(f"total_tokens is {declared}, the stage budgets sum to {plan.total_tokens}.")
        return plan

    @classmethod
    def from_yaml(cls, path) -> "BlockCurriculumPlan":
        p = Path(path).expanduser().resolve()
        if not p.is_file():
            raise FileNotFoundError(f"Curriculum file not found: {p}")
        return cls.from_dict(yaml.safe_load(p.read_text()), p)

    @classmethod
    def fixed(cls, block_size: int, steps: int, sequence_length: int, batch: int, seed: int = 0):
        """One stage: ``block_size`` for ``steps`` optimizer steps."""
        tps = sequence_length * batch
        return cls.from_budgets([(block_size, tps * steps)], tokens_per_step=tps, sequence_length=sequence_length,
                                global_batch_size=batch, seed=seed)

    # ---- queries ----------------------------------------------------------------------------
    @property
    def max_steps(self) -> int:
        return self._ends[-1]

    @property
    def total_tokens(self) -> int:
        return sum(s.token_budget for s in self.stages)

    def stage_for_step(self, step: int) -> CurriculumStage:
        """The stage whose [start_step, end_step) holds ``step``."""
        if step < 0 or step >= self.max_steps:
            raise ValueError(f"Optimizer step {step} is not in [0, {self.max_steps}).")
        lo, hi = 0, len(self._ends) - 1
        while lo < hi:                      # first stage whose end lies beyond the step
            mid = (lo + hi) // 2
            if self._ends[mid] > step:
                hi = mid
            else:
                lo = mid + 1
        return self.stages[lo]

    def validate_runtime(self, *, world_size: int, per_device_batch: int, accumulation: int) -> None:
        runtime = world_size * per_device_batch * accumulation
        if runtime != self.global_batch_size:
            raise ValueError(f"The run's global batch is {runtime} sequences ({world_size} ranks x "
                             f"{per_device_batch} x {accumulation} accumulation); the curriculum expects "
                             f"{self.global_batch_size}.")

    def manifest(self) -> dict:
        """Canonical description (key names as in the reference's checkpoint metadata)."""
        return {
            "version": 1, "tokens_per_step": self.tokens_per_step, "sequence_length": self.sequence_length,
            "global_batch_size": self.global_batch_size, "seed": self.seed, "total_tokens": self.total_tokens,
            "max_steps": self.max_steps, "replay_smaller_blocks": False,
            "stages": [{"block_size": s.block_size, "token_budget": s.token_budget, "start_step": s.start_step,
                        "end_step": s.end_step} for s in self.stages],
        }

    def sha256(self) -> str:
        text = json.dumps(self.manifest(), sort_keys=True, separators=(",", ":"))
        return hashlib.sha256(text.encode()).hexdigest()


def set_model_block_size(model, block_size: int) -> None:
    """Writes the block size of the coming step into the base model's config."""
    from .modeling import unwrap_base_model

    config = getattr(unwrap_base_model(model), "config", None)
    if config is None or not hasattr(config, "block_size"):
        raise RuntimeError("The Uno model config has no block_size to set.")
    config.block_size = int(block_size)
