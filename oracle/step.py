"""One Uno training step on the CPU: compute_loss -> backward -> clip(1.0) -> AdamW.

Restates training/trainer.py:174-308 (loss) and the optimizer configuration of
training/train.py:282-288 (torch AdamW, betas (0.9, 0.999), eps 1e-8, weight decay 0,
max_grad_norm 1.0), with a constant learning rate (the warm-up schedule gives LR 0 at
step 0, so parity runs use a constant LR).
"""
from __future__ import annotations

from dataclasses import dataclass

import torch

from . import bd, layout, losses
from .model import Cfg, decoder

IGNORE_INDEX = -100


@dataclass
class Objective:
    ce_weight: float = 1.0
    kl_weight: float = 0.0
    tv_weight: float = 0.0
    ce_target: str = "data"          # internal: "data" | "clean_argmax"


def compute_loss(params, lora, cfg: Cfg, batch: dict, objective: Objective, *, block_size: int,
                 mask_token_id: int, seed: int, step: int, noise: str = "uniform", rnd=None):
    input_ids, labels = batch["input_ids"], batch["labels"]
    L = input_ids.shape[1]
    pos, model_pos, region = layout.prepare_uno_layout(input_ids, batch.get("position_ids"))
    shifted = layout.shift_labels_for_next_token(labels, pos)
    cids, cpos, mask, noised, _, p_mask = bd.prepare_for_bd_training(
        input_ids, model_pos, labels == IGNORE_INDEX, block_size=block_size,
        mask_token_id=mask_token_id, seed=seed, step=step, noise=noise)
    hidden = decoder(params, lora, cfg, cids, cpos, mask, region, rnd=rnd)
    noisy, clean = layout.extract_uno_regions(hidden, region, L)
    supervised = labels != IGNORE_INDEX
    valid_next = shifted != IGNORE_INDEX
    ce_mask = noised & valid_next
    dist = objective.kl_weight > 0 or objective.tv_weight > 0
    smasks, tmasks = {}, {}
    if dist:
        smasks["distribution"] = supervised
        tmasks["distribution"] = supervised
    if objective.ce_weight > 0:
        smasks["ce"] = ce_mask
        if objective.ce_target == "clean_argmax":
            tmasks["ce"] = ce_mask
    W = params["lm_head.weight"]
    slog = losses.project_hidden_states(W, noisy, smasks)
    tlog = losses.project_hidden_states(W, clean.detach(), tmasks) if tmasks else {}
    n = int(supervised.sum())
    zero = noisy.sum() * 0.0
    kl = losses.reverse_kl(slog["distribution"], tlog["distribution"], n) if objective.kl_weight > 0 else zero
    tv = losses.total_variation(slog["distribution"], tlog["distribution"], n) if objective.tv_weight > 0 else zero
    if objective.ce_weight > 0 and int(ce_mask.sum()):
        tgt = losses.resolve_ce_targets(objective.ce_target, shifted, ce_mask, tlog.get("ce"))
        ce = losses.weighted_ce(slog["ce"], tgt, p_mask[valid_next[noised]], n)
    else:
        ce = zero
    total = objective.ce_weight * ce + objective.kl_weight * kl + objective.tv_weight * tv
    return total, {"ce": ce, "kl": kl, "tv": tv, "noised": noised, "p_mask": p_mask,
                   "concat_ids": cids, "concat_pos": cpos, "mask": mask, "region": region,
                   "hidden": hidden}


def train_steps(params, lora, cfg: Cfg, batch: dict, objective: Objective, *, block_size: int,
                mask_token_id: int, seed: int, steps: int, lr: float = 1e-4, first_step: int = 0,
                max_grad_norm: float = 1.0, block_sizes: list[int] | None = None,
                micro_batches: list[dict] | None = None, grad_accum: int = 1):
    """Runs `steps` optimizer steps; returns (losses, first-step grads, final lora).

    `block_sizes[s]`, when given, is the block size of step s (a curriculum that switches block
    size between optimizer steps, training/trainer.py:182-184 with training/curriculum.py:109-112);
    otherwise every step uses `block_size`.

    With `grad_accum` > 1, optimizer step s accumulates the gradients of `grad_accum` micro-batches
    (`micro_batches[s * grad_accum + i]`, or `batch` for every one), each loss divided by
    `grad_accum` as HF's Trainer does when the model takes no loss kwargs
    (training/trainer.py:161 sets model_accepts_loss_kwargs = False); each micro-batch draws the
    next noise step. `losses` then holds every micro-batch's unscaled loss, in order."""
    leaves = {k: v.detach().clone().float().requires_grad_(True) for k, v in lora.items()}
    opt = torch.optim.AdamW(list(leaves.values()), lr=lr, betas=(0.9, 0.999), eps=1e-8,
                            weight_decay=0.0)
    hist, first_grads = [], None
    for s in range(steps):
        opt.zero_grad(set_to_none=True)
        bs = block_sizes[s] if block_sizes is not None else block_size
        for i in range(grad_accum):
            j = s * grad_accum + i
            mb = micro_batches[j] if micro_batches is not None else batch
            loss, _ = compute_loss(params, leaves, cfg, mb, objective, block_size=bs,
                                   mask_token_id=mask_token_id, seed=seed, step=first_step + j)
            (loss / grad_accum if grad_accum > 1 else loss).backward()
            if grad_accum > 1:
                hist.append(float(loss.detach()))
        if first_grads is None:
            first_grads = {k: v.grad.detach().clone() for k, v in leaves.items()}
        torch.nn.utils.clip_grad_norm_(list(leaves.values()), max_grad_norm)
        opt.step()
        if grad_accum == 1:
            hist.append(float(loss.detach()))
    return hist, first_grads, {k: v.detach() for k, v in leaves.items()}
