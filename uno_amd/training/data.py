"""Batch collation.

* ``UnoDataCollator`` (training/data.py:209-240): one example per row, right-padded to the
  sequence length with the pad id, attention 0 and label IGNORE_INDEX.
* ``UnoPackingCollator``: several examples per row (variable-length packing). The step reads packed
  rows through ``position_ids`` (training/modeling.py:84-98): positions restart at 0 where a new
  example starts, and the layout, the noising blocks, the attention mask and the label shift all
  treat each example as its own segment, so no token attends across examples.
"""
from __future__ import annotations

from dataclasses import dataclass
from typing import Any, Sequence

import torch

from .constants import COLLATED_SEQUENCE_LENGTH, IGNORE_INDEX


@dataclass
class UnoDataCollator:
    tokenizer: Any
    sequence_length: int = COLLATED_SEQUENCE_LENGTH

    def __post_init__(self) -> None:
        if getattr(self.tokenizer, "padding_side", "right") != "right":
            raise ValueError("Uno training requires right padding.")
        if getattr(self.tokenizer, "pad_token_id", None) is None:
            raise ValueError("Uno training requires a tokenizer pad token.")

    def __call__(self, features: list[dict[str, Sequence[int]]]) -> dict[str, torch.Tensor]:
        if not features:
            raise ValueError("Cannot collate an empty batch.")
        L, pad = self.sequence_length, self.tokenizer.pad_token_id
        ids = torch.full((len(features), L), pad, dtype=torch.long)
        att = torch.zeros((len(features), L), dtype=torch.long)
        lab = torch.full((len(features), L), IGNORE_INDEX, dtype=torch.long)
        for i, f in enumerate(features):
            n = len(f["input_ids"])
            if n > L:
                raise ValueError(f"Prepared row length {n} exceeds sequence length {L}.")
            if len(f["labels"]) != n:
                raise ValueError("Prepared input IDs and labels must have equal lengths.")
            ids[i, :n] = torch.as_tensor(list(f["input_ids"]), dtype=torch.long)
            att[i, :n] = torch.as_tensor(list(f.get("attention_mask", [1] * n)), dtype=torch.long)
            lab[i, :n] = torch.as_tensor(list(f["labels"]), dtype=torch.long)
        return {"input_ids": ids, "attention_mask": att, "labels": lab}


@dataclass
class UnoPackingCollator:
    """Packs examples into rows of ``sequence_length`` tokens, first fit in arrival order (an
    example goes to the first row with room; a new row opens when none has). Each row carries
    ``position_ids`` that restart at 0 at every example; the unused tail of a row is one more
    segment of pad tokens with positions 0, 1, ..., attention 0 and label IGNORE_INDEX, so it never
    joins a real example's segment. ``rows`` fixes the number of rows per batch (an error if the
    examples need more; empty rows are all padding)."""

    tokenizer: Any
    sequence_length: int = COLLATED_SEQUENCE_LENGTH
    rows: int | None = None

    def __post_init__(self) -> None:
        if getattr(self.tokenizer, "pad_token_id", None) is None:
            raise ValueError("Uno training requires a tokenizer pad token.")
        if self.sequence_length <= 0:
            raise ValueError("sequence_length must be positive.")

    def plan(self, lengths: Sequence[int]) -> list[list[int]]:
        """Example indices per row, first fit."""
        L = self.sequence_length
        rows: list[list[int]] = []
        room: list[int] = []
        for i, n in enumerate(lengths):
            if n <= 0:
                raise ValueError(f"Example {i} is empty.")
            if n > L:
                raise ValueError(f"Example {i} has {n} tokens, more than the sequence length {L}.")
            for r, free in enumerate(room):
                if n <= free:
                    rows[r].append(i)
                    room[r] -= n
                    break
            else:
                rows.append([i])
                room.append(L - n)
        if self.rows is not None:
            if len(rows) > self.rows:
                raise ValueError(f"The examples need {len(rows)} rows of {L} tokens; the batch has {self.rows}.")
            rows += [[] for _ in range(self.rows - len(rows))]
        return rows

    def __call__(self, features: list[dict[str, Sequence[int]]]) -> dict[str, torch.Tensor]:
        if not features:
            raise ValueError("Cannot collate an empty batch.")
        for f in features:
            if len(f["labels"]) != len(f["input_ids"]):
                raise ValueError("Prepared input IDs and labels must have equal lengths.")
        layout = self.plan([len(f["input_ids"]) for f in features])
        L, pad = self.sequence_length, self.tokenizer.pad_token_id
        R = len(layout)
        ids = torch.full((R, L), pad, dtype=torch.long)
        att = torch.zeros((R, L), dtype=torch.long)
        lab = torch.full((R, L), IGNORE_INDEX, dtype=torch.long)
        pos = torch.zeros((R, L), dtype=torch.long)
        for r, members in enumerate(layout):
            t = 0
            for i in members:
                f = features[i]
                n = len(f["input_ids"])
                ids[r, t:t + n] = torch.as_tensor(list(f["input_ids"]), dtype=torch.long)
                lab[r, t:t + n] = torch.as_tensor(list(f["labels"]), dtype=torch.long)
                att[r, t:t + n] = torch.as_tensor(list(f.get("attention_mask", [1] * n)), dtype=torch.long)
                pos[r, t:t + n] = torch.arange(n)
                t += n
            pos[r, t:] = torch.arange(L - t)
        return {"input_ids": ids, "attention_mask": att, "labels": lab, "position_ids": pos}
