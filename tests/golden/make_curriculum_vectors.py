"""Writes tests/golden/curriculum_vectors.json: the reference's own curriculum manifest hash.

Run in the build container, where the reference tree is present:

    python tests/golden/make_curriculum_vectors.py

It loads training/curriculum.py from /root/reference by file path (that module needs only the
standard library and PyYAML) and, for the released schedule file and a few synthetic schedules
written as YAML, records the stage boundaries, the manifest and ``sha256()``. A boundary checkpoint
stores that hash (training/trainer.py:110-146), so a resume validates only when uno_amd's hash of
the same schedule is bit-identical; nothing else in the reference pins it.
"""
from __future__ import annotations

import importlib.util
import json
import sys
import tempfile
from pathlib import Path

import yaml

REF = Path("/root/reference/training")
OUT = Path(__file__).resolve().parent / "curriculum_vectors.json"

SYNTHETIC = [
    # one stage, the shape of the benchmark's fixed plan (4 x 4096 tokens per step, 100 steps)
    {"version": 1, "tokens_per_step": 16384, "sequence_length": 4096, "global_batch_size": 4, "seed": 0,
     "stages": [{"block_size": 16, "tokens": 1638400}]},
    # budgets that are not whole steps (the end step floors the cumulative count), no total given
    {"version": 1, "tokens_per_step": 8192, "sequence_length": 2048, "global_batch_size": 4, "seed": 7,
     "stages": [{"block_size": 4, "tokens": 100000}, {"block_size": 8, "tokens": 50001},
                {"block_size": 32, "tokens": 8193}]},
    # the 4 -> 32 sweep of the 7B configuration, one step per stage, a negative seed
    {"version": 1, "tokens_per_step": 16384, "sequence_length": 4096, "global_batch_size": 4, "seed": -3,
     "total_tokens": 65536,
     "stages": [{"block_size": 4, "tokens": 16384}, {"block_size": 8, "tokens": 16384},
                {"block_size": 16, "tokens": 16384}, {"block_size": 32, "tokens": 16384}]},
]


def _load_reference():
    spec = importlib.util.spec_from_file_location("reference_curriculum", REF / "curriculum.py")
    mod = importlib.util.module_from_spec(spec)
    sys.modules[spec.name] = mod          # its dataclasses resolve annotations through sys.modules
    spec.loader.exec_module(mod)
    return mod


def _vector(mod, path: Path, raw: dict) -> dict:
    plan = mod.BlockCurriculumPlan.from_yaml(path)
    return {"input": raw, "end_steps": [s.end_step for s in plan.stages], "max_steps": plan.max_steps,
            "manifest": plan.manifest(), "sha256": plan.sha256()}


def main() -> None:
    mod = _load_reference()
    released = REF / "configs" / "uno_3epoch_curriculum.yaml"
    vectors = {"released": _vector(mod, released, yaml.safe_load(released.read_text())), "synthetic": []}
    with tempfile.TemporaryDirectory() as tmp:
        for i, raw in enumerate(SYNTHETIC):
            p = Path(tmp) / f"plan{i}.yaml"
            p.write_text(yaml.safe_dump(raw))
            vectors["synthetic"].append(_vector(mod, p, raw))
    OUT.write_text(json.dumps(vectors, indent=1, sort_keys=True) + "\n")
    print(f"wrote {OUT}")


if __name__ == "__main__":
    main()
