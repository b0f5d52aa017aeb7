"""Block-size curriculum (semantics of training/curriculum.py:20-171 in the reference).

Stage i ends at cumulative_tokens_i // tokens_per_step; the block size of an optimizer step is
that of the first stage whose end step is greater than the step.
"""
from __future__ import annotations

import bisect
import hashlib
import json
from dataclasses import dataclass
from pathlib import Path

import yaml


@dataclass(frozen=True)
class CurriculumStage:
    block_size: int
    token_budget: int
    start_step: int
    end_step: int


def _int_field(mapping: dict, key: str, positive: bool = True) -> int:
    value = mapping.get(key)
    if isinstance(value, bool) or not isinstance(value, int):
        raise ValueError(f"{key} must be an integer.")
    if positive and value <= 0:
        raise ValueError(f"{key} must be positive.")
    return value


class BlockCurriculumPlan:
    def __init__(self, *, source_path, tokens_per_step, sequence_length, global_batch_size, seed, stages):
        self.source_path = source_path
        self.tokens_per_step = tokens_per_step
        self.sequence_length = sequence_length
        self.global_batch_size = global_batch_size
        self.seed = seed
        self.stages = tuple(stages)
        self._ends = [s.end_step for s in self.stages]
        self.checkpoint_reasons = {s.end_step: f"completed_block_size_{s.block_size}" for s in self.stages}

    @property
    def max_steps(self) -> int:
        return self.stages[-1].end_step

    @property
    def total_tokens(self) -> int:
        return sum(s.token_budget for s in self.stages)

    @classmethod
    def from_dict(cls, raw: dict, source_path: Path | None = None) -> "BlockCurriculumPlan":
        if not isinstance(raw, dict):
            raise ValueError("Curriculum YAML must contain a mapping.")
        if raw.get("replay") not in (None, {}, False):
            raise ValueError("Smaller-block replay is not supported by the public trainer.")
        tps = _int_field(raw, "tokens_per_step")
        seq = _int_field(raw, "sequence_length")
        gbs = _int_field(raw, "global_batch_size")
        seed = _int_field(raw, "seed", positive=False)
        if tps != seq * gbs:
            raise ValueError("tokens_per_step must equal sequence_length * global_batch_size.")
        items = raw.get("stages")
        if not isinstance(items, list) or not items:
            raise ValueError("Curriculum stages must be a non-empty list.")
        stages, tokens, prev_end, prev_block = [], 0, 0, 0
        for i, item in enumerate(items):
            if not isinstance(item, dict):
                raise ValueError(f"Curriculum stage {i} must be a mapping.")
            block = _int_field(item, "block_size")
            budget = _int_field(item, "tokens")
            if block <= prev_block:
                raise ValueError("Curriculum block sizes must be strictly increasing.")
            tokens += budget
            end = tokens // tps
            if end <= prev_end:
                raise ValueError(f"Curriculum stage B={block} is shorter than one step.")
            stages.append(CurriculumStage(block, budget, prev_end, end))
            prev_end, prev_block = end, block
        total = raw.get("total_tokens")
        if total is not None and total != tokens:
            raise ValueError("total_tokens does not match the sum of stage token budgets.")
        return cls(source_path=source_path, tokens_per_step=tps, sequence_length=seq, global_batch_size=gbs,
                   seed=seed, stages=stages)

    @classmethod
    def from_yaml(cls, path) -> "BlockCurriculumPlan":
        p = Path(path).expanduser().resolve()
        if not p.is_file():
            raise FileNotFoundError(f"Curriculum file not found: {p}")
        return cls.from_dict(yaml.safe_load(p.read_text()), p)

    @classmethod
    def fixed(cls, block_size: int, steps: int, sequence_length: int, batch: int, seed: int = 0):
        """A one-stage plan (fixed block size for `steps` optimizer steps)."""
        tps = sequence_length * batch
        return cls.from_dict({"tokens_per_step": tps, "sequence_length": sequence_length,
                              "global_batch_size": batch, "seed": seed,
                              "stages": [{"block_size": block_size, "tokens": tps * steps}]})

    def stage_for_step(self, step: int) -> CurriculumStage:
        if not 0 <= step < self.max_steps:
            raise ValueError(f"Optimizer step {step} is outside [0, {self.max_steps}).")
        return self.stages[bisect.bisect_right(self._ends, step)]

    def validate_runtime(self, *, world_size: int, per_device_batch: int, accumulation: int) -> None:
        got = world_size * per_device_batch * accumulation
        if got != self.global_batch_size:
            raise ValueError(f"Curriculum global batch mismatch: runtime={got}, expected={self.global_batch_size}.")

    def manifest(self) -> dict:
        return {
            "version": 1, "tokens_per_step": self.tokens_per_step, "sequence_length": self.sequence_length,
            "global_batch_size": self.global_batch_size, "seed": self.seed, "total_tokens": self.total_tokens,
            "max_steps": self.max_steps, "replay_smaller_blocks": False,
            "stages": [{"block_size": s.block_size, "token_budget": s.token_budget, "start_step": s.start_step,
                        "end_step": s.end_step} for s in self.stages],
        }

    def sha256(self) -> str:
        return hashlib.sha256(json.dumps(self.manifest(), sort_keys=True, separators=(",", ":")).encode()).hexdigest()


def set_model_block_size(model, block_size: int) -> None:
    while hasattr(model, "module"):
        model = model.module
    base = model.get_base_model() if hasattr(model, "get_base_model") else model
    if not hasattr(base.config, "block_size"):
        raise RuntimeError("Uno training requires model.config.block_size.")
    base.config.block_size = block_size
