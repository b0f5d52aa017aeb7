"""Layout helpers of the Uno step (oracle restatement).

Reference: training/modeling.py:65-113 (noisy/clean layout and region split) and
training/losses.py:9-18 (next-token label shift). The remote helpers
``modify_padded_position_ids_2d`` / ``calculate_token_nums`` are not in the reference tree;
their contract is defined here from their call site (training/modeling.py:94-97): segment
lengths per row, where a packed row starts a new segment at t=0 and wherever the position
does not increase (pos[t-1] >= pos[t]) -- the same boundary rule the label shift uses.
"""
from __future__ import annotations

import torch

IGNORE_INDEX = -100


def modify_padded_position_ids_2d(position_ids: torch.Tensor) -> torch.Tensor:
    """Contract: positions are returned unchanged (rows carry no padding markers in the training data)."""
    return position_ids.clone()


def segment_starts(position_ids: torch.Tensor) -> torch.Tensor:
    """Bool [B, L]: True where a segment starts (t == 0 or pos[t-1] >= pos[t])."""
    starts = torch.zeros_like(position_ids, dtype=torch.bool)
    starts[:, 0] = True
    starts[:, 1:] = position_ids[:, :-1] >= position_ids[:, 1:]
    return starts


def calculate_token_nums(position_ids: torch.Tensor) -> list[torch.Tensor]:
    """Per row, a 1-D int64 tensor of segment lengths in order (brute-force loop)."""
    out = []
    for row in position_ids.tolist():
        lengths, cur = [], 0
        for t, p in enumerate(row):
            if t > 0 and row[t - 1] >= p:
                lengths.append(cur)
                cur = 0
            cur += 1
        lengths.append(cur)
        out.append(torch.tensor(lengths, dtype=torch.long))
    return out


def build_noisy_region_mask(num_tokens: list[torch.Tensor], sequence_length: int) -> torch.Tensor:
    """training/modeling.py:65-81: per segment, `l` Trues (noisy copy) then `l` Falses (clean)."""
    rows = []
    for lengths in num_tokens:
        parts = []
        for length in lengths.tolist():
            parts.append(torch.ones(length, dtype=torch.bool))
            parts.append(torch.zeros(length, dtype=torch.bool))
        row = torch.cat(parts)
        if row.numel() != 2 * sequence_length:
            raise RuntimeError(
                f"Uno noisy/clean layout has an invalid length: {row.numel()} for "
                f"sequence_length={sequence_length}.")
        rows.append(row)
    return torch.stack(rows)


def prepare_uno_layout(input_ids: torch.Tensor, position_ids: torch.Tensor | None):
    """training/modeling.py:84-98."""
    batch, length = input_ids.shape
    if position_ids is None:
        position_ids = torch.arange(length).unsqueeze(0).expand(batch, -1)
    model_pos = modify_padded_position_ids_2d(position_ids)
    counts = calculate_token_nums(model_pos)
    return position_ids, model_pos, build_noisy_region_mask(counts, length)


def shift_labels_for_next_token(labels: torch.Tensor, position_ids: torch.Tensor) -> torch.Tensor:
    """training/losses.py:9-18."""
    shifted = torch.full_like(labels, IGNORE_INDEX)
    shifted[:, :-1] = labels[:, 1:]
    shifted[:, :-1].masked_fill_(position_ids[:, :-1] >= position_ids[:, 1:], IGNORE_INDEX)
    return shifted


def extract_uno_regions(hidden: torch.Tensor, noisy_region_mask: torch.Tensor, sequence_length: int):
    """training/modeling.py:101-113."""
    b, _, h = hidden.shape
    noisy = hidden[noisy_region_mask].reshape(b, sequence_length, h)
    clean = hidden[~noisy_region_mask].reshape(b, sequence_length, h)
    return noisy, clean
