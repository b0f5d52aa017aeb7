"""Uno objectives on logits (call surface of training/losses.py in the reference).

The step itself (training/trainer.py counterpart) uses the fused LM-head objectives of
uno_amd.objectives, which never hold full-vocabulary logits for CE; these functions keep the
reference's logits-level interface for callers that have logits in hand.
"""
from __future__ import annotations

import torch

from ..layers import GatherRows
from ..objectives import LogitsDistributionLoss, lm_head_logits, logits_argmax
from .constants import IGNORE_INDEX


def shift_labels_for_next_token(labels: torch.Tensor, position_ids: torch.Tensor) -> torch.Tensor:
    """labels shifted left by one; IGNORE_INDEX at packed-segment boundaries and the last column."""
    shifted = torch.full_like(labels, IGNORE_INDEX)
    boundary = position_ids[:, :-1] >= position_ids[:, 1:]
    shifted[:, :-1] = torch.where(boundary, torch.full_like(labels[:, 1:], IGNORE_INDEX), labels[:, 1:])
    return shifted


def project_hidden_states(lm_head, hidden_states: torch.Tensor, masks: dict[str, torch.Tensor]):
    """LM head applied once to the union of the masked rows, then re-selected per mask
    (training/losses.py:21-35); row gathers and the GEMM run on the HIP kernels."""
    first = next(iter(masks.values()))
    union = torch.zeros_like(first, dtype=torch.bool)
    for m in masks.values():
        union |= m
    hdim = hidden_states.shape[-1]
    flat = hidden_states.reshape(-1, hdim)
    rows = torch.nonzero(union.reshape(-1)).flatten().to(torch.int32)
    if rows.numel() == 0:
        empty = hidden_states.new_empty((0, lm_head.weight.shape[0]))
        return {k: empty for k in masks}
    logits = lm_head(GatherRows.apply(flat, rows))
    pos_in_union = (union.reshape(-1).to(torch.int32).cumsum(0) - 1).to(torch.int32)
    out = {}
    for k, m in masks.items():
        sel = pos_in_union[m.reshape(-1)]
        out[k] = GatherRows.apply(logits, sel) if sel.numel() else logits[:0]
    return out


def resolve_ce_targets(target_source: str, shifted_labels: torch.Tensor, ce_mask: torch.Tensor,
                       clean_teacher_logits: torch.Tensor | None) -> torch.Tensor:
    """CE targets (training/losses.py:38-56): the shifted labels of the CE rows ("data"), or the
    first-index argmax of the teacher's logits ("clean_argmax", the row-argmax kernel)."""
    if target_source == "data":
        return shifted_labels[ce_mask]
    if target_source != "clean_argmax":
        raise ValueError(f"Unsupported CE target source: {target_source}.")
    if clean_teacher_logits is None:
        raise RuntimeError("Teacher CE requires clean teacher logits.")
    expected = int(ce_mask.sum().item())
    if clean_teacher_logits.size(0) != expected:
        raise RuntimeError("Teacher logits do not align with noised CE positions: "
                           f"{clean_teacher_logits.size(0)} rows for {expected} positions.")
    return logits_argmax(clean_teacher_logits.detach())


def _inv_n(t: torch.Tensor, num_tokens: int) -> torch.Tensor:
    return torch.full((), 1.0 / max(num_tokens, 1), device=t.device, dtype=torch.float32)


def token_normalized_reverse_kl(student_logits, teacher_logits, num_tokens: int) -> torch.Tensor:
    """KL(student || detached teacher) summed over rows, divided by max(num_tokens, 1)."""
    if student_logits.shape[0] == 0:
        return student_logits.sum() * 0.0
    return LogitsDistributionLoss.apply(student_logits.reshape(-1, student_logits.shape[-1]),
                                        teacher_logits.detach().reshape(-1, teacher_logits.shape[-1]),
                                        _inv_n(student_logits, num_tokens), "kl")


def token_normalized_total_variation(student_logits, teacher_logits, num_tokens: int,
                                     chunk_size: int = 2048) -> torch.Tensor:
    """sum |softmax(s) - softmax(t)| / max(num_tokens, 1); exact full-vocabulary L1."""
    if student_logits.shape != teacher_logits.shape:
        raise ValueError("Student and teacher logits must have identical shapes.")
    if chunk_size <= 0:
        raise ValueError("TV chunk_size must be positive.")
    V = student_logits.size(-1)
    s = student_logits.reshape(-1, V)
    if not s.size(0):
        return s.sum()
    return LogitsDistributionLoss.apply(s, teacher_logits.detach().reshape(-1, V), _inv_n(s, num_tokens), "tv")


__all__ = ["shift_labels_for_next_token", "project_hidden_states", "resolve_ce_targets",
           "token_normalized_reverse_kl", "token_normalized_total_variation", "lm_head_logits"]
