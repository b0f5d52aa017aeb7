"""Batch collation (semantics of training/data.py:209-240 in the reference): right-pad every
row to the sequence length with the pad id, attention 0 and label IGNORE_INDEX."""
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
