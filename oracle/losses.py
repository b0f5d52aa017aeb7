"""Uno objectives (oracle restatement, dense fp32, autograd for gradients).

Reference: training/losses.py:21-73,163-183 and training/trainer.py:223-287. The chunked
TV forward/backward of the reference (losses.py:76-160) is the exact gradient of the dense
sum of |softmax(s) - softmax(t)| with sign(0) = 0, so the oracle states the dense formula and
lets autograd differentiate it; tests/test_oracle_losses.py checks that claim against a
line-by-line chunked restatement of the reference algorithm.
"""
from __future__ import annotations

import torch
import torch.nn.functional as F

IGNORE_INDEX = -100


def _up(x):
    """Upcast bf16/fp16 to fp32; keep fp32/fp64 as they are."""
    return x if x.dtype in (torch.float32, torch.float64) else x.float()


def project_hidden_states(lm_weight, hidden, masks: dict):
    """training/losses.py:21-35: LM head on the union of masked rows, reselected per mask."""
    union = torch.zeros_like(next(iter(masks.values())), dtype=torch.bool)
    for m in masks.values():
        union |= m
    if not union.any():
        empty = hidden.new_empty((0, lm_weight.shape[0]))
        return {k: empty for k in masks}
    logits = hidden[union] @ lm_weight.T
    idx = union.reshape(-1).long().cumsum(0) - 1
    return {k: logits[idx[m.reshape(-1)]] for k, m in masks.items()}


def resolve_ce_targets(source, shifted, ce_mask, teacher_logits):
    """training/losses.py:38-56 (argmax takes the first index on ties)."""
    if source == "data":
        return shifted[ce_mask]
    if source != "clean_argmax":
        raise ValueError(f"Unsupported CE target source: {source}.")
    return teacher_logits.detach().argmax(dim=-1)


def reverse_kl(student, teacher, n):
    """training/losses.py:59-73: sum exp(ls) (ls - lt) / max(n, 1)."""
    ls = F.log_softmax(_up(student), dim=-1)
    lt = F.log_softmax(_up(teacher.detach()), dim=-1)
    return (ls.exp() * (ls - lt)).sum() / max(n, 1)


def total_variation(student, teacher, n):
    """sum |softmax(s) - softmax(t)| / max(n, 1) (no 1/2 factor), teacher detached."""
    p = torch.softmax(_up(student), dim=-1)
    q = torch.softmax(_up(teacher.detach()), dim=-1)
    return (p - q).abs().sum() / max(n, 1)


def chunked_tv_reference_algorithm(student, teacher, n, chunk=2048):
    """Literal restatement of training/losses.py:76-160: (value, grad wrt student logits)."""
    s_max = student.amax(-1).float()
    t_max = teacher.amax(-1).float()

    def den(x, m):
        d = torch.zeros_like(m)
        for c in range(0, x.size(-1), chunk):
            d += torch.exp(x[:, c:c + chunk].float() - m[:, None]).sum(-1)
        return d.clamp_min(torch.finfo(torch.float32).tiny)

    sd, td = den(student, s_max), den(teacher, t_max)
    l1 = torch.zeros((), dtype=torch.float32)
    sps = torch.zeros_like(s_max)
    for c in range(0, student.size(-1), chunk):
        ps = torch.exp(student[:, c:c + chunk].float() - s_max[:, None]) / sd[:, None]
        pt = torch.exp(teacher[:, c:c + chunk].float() - t_max[:, None]) / td[:, None]
        l1 += (ps - pt).abs().sum()
        sps += (torch.sign(ps - pt) * ps).sum(-1)
    norm = max(n, 1)
    grad = torch.empty_like(student, dtype=torch.float32)
    for c in range(0, student.size(-1), chunk):
        ps = torch.exp(student[:, c:c + chunk].float() - s_max[:, None]) / sd[:, None]
        pt = torch.exp(teacher[:, c:c + chunk].float() - t_max[:, None]) / td[:, None]
        grad[:, c:c + chunk] = ps * (torch.sign(ps - pt) - sps[:, None]) / norm
    return l1 / norm, grad


def weighted_ce(student_logits, targets, p_sel, n):
    """training/trainer.py:275-281: sum(CE / p) / max(n, 1)."""
    per = F.cross_entropy(_up(student_logits), targets, reduction="none")
    if p_sel.numel() != per.numel():
        raise RuntimeError("Noise probabilities do not align with Uno CE rows.")
    return (per / p_sel.to(per.dtype)).sum() / max(n, 1)
