"""Uno training step (counterpart of training/trainer.py in the reference).

``UnoTrainer.compute_loss(model, inputs, return_outputs=False, num_items_in_batch=None)`` keeps
the reference's call surface and control flow (trainer.py:174-308): curriculum block size ->
layout -> noising/concatenation -> gated forward -> region split -> objectives -> combine ->
log. Underneath, the decoder runs the two-stream HIP path and the objectives are the fused
LM-head kernels (CE never materialises [rows x vocab] logits). The trainer is standalone: the
HF Trainer loop around compute_loss (backward, clip, AdamW, LR schedule) is provided by
``training_step`` / ``optimizer_step`` with the reference's optimizer settings.
"""
from __future__ import annotations

import json
from dataclasses import dataclass, field
from pathlib import Path

import torch

from ..layers import GatherRows
from ..objectives import distribution_loss, fused_weighted_ce, teacher_argmax
from ..optim import FusedLoraAdamW
from .config import UnoObjectiveConfig
from .constants import IGNORE_INDEX
from .curriculum import BlockCurriculumPlan, set_model_block_size
from .lora import TokenwiseLoraRouter, load_adapter, make_saved_adapter_portable, save_adapter
from .losses import shift_labels_for_next_token
from .modeling import (extract_uno_regions, prepare_uno_layout, run_prepared_uno_forward, unwrap_base_model,
                       validate_uno_model)


# AdamW moments of a curriculum-boundary checkpoint (flat fp32 buffers, safetensors).
OPTIMIZER_STATE = "uno_optimizer_state.safetensors"


def combine_objective_losses(ce_loss, kl_loss, tv_loss, objective: UnoObjectiveConfig):
    """alpha * CE + beta * KL + gamma * TV."""
    objective.validate()
    return objective.ce_weight * ce_loss + objective.kl_weight * kl_loss + objective.tv_weight * tv_loss


def validate_curriculum_resume(checkpoint, curriculum: BlockCurriculumPlan) -> None:
    state_path = Path(checkpoint) / "uno_curriculum_state.json"
    if not state_path.is_file():
        raise FileNotFoundError("Uno resumes are supported only from curriculum-boundary checkpoints; "
                                f"missing {state_path}.")
    state = json.loads(state_path.read_text())
    if state.get("curriculum_sha256") != curriculum.sha256():
        raise ValueError("Checkpoint curriculum does not match the current curriculum.")
    if state.get("global_step") not in curriculum.checkpoint_reasons:
        raise ValueError(f"Checkpoint step {state.get('global_step')} is not a curriculum boundary.")


@dataclass
class TrainerState:
    global_step: int = 0
    log_history: list = field(default_factory=list)


@dataclass
class UnoTrainingArguments:
    learning_rate: float = 1e-5
    weight_decay: float = 0.0
    adam_beta1: float = 0.9
    adam_beta2: float = 0.999
    adam_epsilon: float = 1e-8
    max_grad_norm: float = 1.0
    warmup_steps: int = 0
    output_dir: str | None = None


def _unwrap_wrappers(model):
    while hasattr(model, "module"):
        model = model.module
    return model


class UnoTrainer:
    """LoRA-only, single-forward Uno trainer on the MI355X kernels."""

    def __init__(self, *, model, objective: UnoObjectiveConfig, curriculum: BlockCurriculumPlan,
                 args: UnoTrainingArguments | None = None):
        objective.validate()
        self.model = model
        self.args = args or UnoTrainingArguments()
        self.objective = objective
        self.curriculum = curriculum
        self.state = TrainerState()
        validate_uno_model(model)
        self._lora_router = TokenwiseLoraRouter(model)
        lora_state = _unwrap_wrappers(model).state
        self.optimizer = FusedLoraAdamW(lora_state, lr=self.args.learning_rate,
                                        betas=(self.args.adam_beta1, self.args.adam_beta2),
                                        eps=self.args.adam_epsilon, weight_decay=self.args.weight_decay,
                                        max_grad_norm=self.args.max_grad_norm)

    # ---- logging ----------------------------------------------------------------------------
    def log(self, logs: dict) -> None:
        """Keeps device scalars as tensors; they are converted when the history is read."""
        self.state.log_history.append(logs)

    def logged(self) -> list[dict]:
        return [{k: (float(v) if torch.is_tensor(v) else v) for k, v in rec.items()} for rec in self.state.log_history]

    # ---- the step -----------------------------------------------------------------------------
    def learning_rate(self, step: int) -> float:
        """Warmup-stable schedule with zero decay steps (training/train.py:282-284)."""
        w = self.args.warmup_steps
        if w > 0 and step < w:
            return self.args.learning_rate * step / w
        return self.args.learning_rate

    def compute_loss(self, model, inputs, return_outputs=False, num_items_in_batch=None):
        del num_items_in_batch
        step = min(self.state.global_step, self.curriculum.max_steps - 1)
        block_size = self.curriculum.stage_for_step(step).block_size
        set_model_block_size(model, block_size)

        labels = inputs.get("labels")
        if labels is None:
            raise RuntimeError("Uno training batches must contain labels.")
        unwrapped = _unwrap_wrappers(model)
        base_model = unwrap_base_model(unwrapped)
        sequence_length = inputs["input_ids"].size(-1)
        original_positions, model_positions, noisy_region_mask = prepare_uno_layout(
            base_model, inputs["input_ids"], inputs.get("position_ids"))
        shifted_labels = shift_labels_for_next_token(labels, original_positions)
        concatenated_ids, concatenated_positions, bd_mask, noised_positions, _, p_mask = \
            base_model.prepare_for_bd_training(inputs["input_ids"], model_positions, labels == IGNORE_INDEX)
        self._lora_router.set_token_mask(noisy_region_mask)
        hidden_states = run_prepared_uno_forward(model, base_model, inputs, concatenated_ids,
                                                 concatenated_positions, bd_mask)
        noisy_hidden, clean_hidden = extract_uno_regions(hidden_states, noisy_region_mask, sequence_length)

        supervised_mask = labels != IGNORE_INDEX
        valid_next_token = shifted_labels != IGNORE_INDEX
        ce_mask = noised_positions & valid_next_token
        token_count, ce_count = (int(x) for x in torch.stack([supervised_mask.sum(), ce_mask.sum()]).tolist())
        dev = noisy_hidden.device
        inv_n = torch.full((), 1.0 / max(token_count, 1), device=dev, dtype=torch.float32)
        zero_loss = torch.zeros((), device=dev, dtype=torch.float32)
        hdim = noisy_hidden.shape[-1]
        flat_noisy = noisy_hidden.reshape(-1, hdim)
        flat_clean = clean_hidden.reshape(-1, hdim)
        lm_head = unwrapped.lm_head

        kl_loss = tv_loss = zero_loss
        if self.objective.kl_weight > 0 or self.objective.tv_weight > 0:
            rows = torch.nonzero(supervised_mask.reshape(-1)).flatten().to(torch.int32)
            h_s = GatherRows.apply(flat_noisy, rows)
            with torch.no_grad():
                h_t = GatherRows.apply(flat_clean.detach(), rows)
            if self.objective.kl_weight > 0:
                kl_loss = distribution_loss(lm_head, h_s, h_t, inv_n, "kl")
            if self.objective.tv_weight > 0:
                tv_loss = distribution_loss(lm_head, h_s, h_t, inv_n, "tv")

        if self.objective.ce_weight > 0 and ce_count:
            rows = torch.nonzero(ce_mask.reshape(-1)).flatten().to(torch.int32)
            h_ce = GatherRows.apply(flat_noisy, rows)
            if self.objective.internal_ce_target == "data":
                targets = shifted_labels.reshape(-1)[rows.long()]
            else:
                with torch.no_grad():
                    targets = teacher_argmax(lm_head, GatherRows.apply(flat_clean.detach(), rows))
            selected_probabilities = p_mask[valid_next_token[noised_positions]]
            if selected_probabilities.numel() != ce_count:
                raise RuntimeError("Noise probabilities do not align with Uno CE rows.")
            ce_loss = fused_weighted_ce(lm_head, h_ce, targets, 1.0 / selected_probabilities, inv_n)
        else:
            ce_loss = zero_loss

        combined_loss = combine_objective_losses(ce_loss, kl_loss, tv_loss, self.objective)
        self.log({
            "train/ce_loss": ce_loss.detach(), "train/reverse_kl_loss": kl_loss.detach(),
            "train/tv_loss": tv_loss.detach(), "train/combined_loss": combined_loss.detach(),
            "train/alpha": self.objective.ce_weight, "train/beta": self.objective.kl_weight,
            "train/gamma": self.objective.tv_weight, "train/block_size": block_size,
            "train/transformer_forwards": 1,
        })
        if return_outputs:
            return combined_loss, {"loss": combined_loss, "ce_loss": ce_loss, "reverse_kl_loss": kl_loss,
                                   "tv_loss": tv_loss}
        return combined_loss

    def training_step(self, model, inputs) -> torch.Tensor:
        """Forward + backward of one micro-batch (gradients accumulate into the flat buffer)."""
        loss = self.compute_loss(model, inputs)
        loss.backward()
        return loss.detach()

    def optimizer_step(self) -> None:
        """Global-norm clip + AdamW over the LoRA tensors, then zero the gradients."""
        self.optimizer.step(lr=self.learning_rate(self.state.global_step))
        self.optimizer.zero_grad()
        self.state.global_step += 1

    def train_step(self, inputs) -> torch.Tensor:
        loss = self.training_step(self.model, inputs)
        self.optimizer_step()
        return loss

    def save_checkpoint(self, output_dir) -> Path:
        """Adapter checkpoint (PEFT format); at curriculum boundaries the complete resume state
        too (training/trainer.py:89-128 saves full state there): the AdamW moments and update
        count, the position of the model's noise stream (what the reference's RNG state restores),
        then the curriculum state file, which is written last so that its presence marks a
        complete checkpoint."""
        from safetensors.torch import save_file

        ckpt = Path(output_dir) / f"checkpoint-{self.state.global_step}"
        save_adapter(_unwrap_wrappers(self.model), ckpt)
        make_saved_adapter_portable(ckpt)
        reason = self.curriculum.checkpoint_reasons.get(self.state.global_step)
        if reason:
            st = self.optimizer.state
            save_file({"exp_avg": st.exp_avg.detach().cpu(), "exp_avg_sq": st.exp_avg_sq.detach().cpu()},
                      str(ckpt / OPTIMIZER_STATE))
            base = unwrap_base_model(_unwrap_wrappers(self.model))
            payload = {"version": 1, "global_step": self.state.global_step, "reason": reason,
                       "curriculum_sha256": self.curriculum.sha256(), "adamw_updates": st.step,
                       "noise_draws": int(getattr(base, "_bd_step", 0))}
            tmp = ckpt / "uno_curriculum_state.json.tmp"
            tmp.write_text(json.dumps(payload, indent=2, sort_keys=True) + "\n")
            tmp.replace(ckpt / "uno_curriculum_state.json")
        return ckpt

    def resume_from_checkpoint(self, checkpoint) -> None:
        """Restores a curriculum-boundary checkpoint (validate_curriculum_resume, then adapters,
        AdamW moments, update count, noise-stream position and global step): the next train_step
        continues the run exactly."""
        from safetensors.torch import load_file

        checkpoint = Path(checkpoint)
        validate_curriculum_resume(checkpoint, self.curriculum)
        payload = json.loads((checkpoint / "uno_curriculum_state.json").read_text())
        moments_path = checkpoint / OPTIMIZER_STATE
        if not moments_path.is_file() or "adamw_updates" not in payload:
            raise FileNotFoundError(f"{checkpoint} holds no optimizer state ({OPTIMIZER_STATE}).")
        moments = load_file(str(moments_path))
        st = self.optimizer.state
        for name in ("exp_avg", "exp_avg_sq"):
            if tuple(moments[name].shape) != (st.numel,):
                raise ValueError(f"{name} in {moments_path} has {moments[name].numel()} values, expected {st.numel}.")
        load_adapter(_unwrap_wrappers(self.model), checkpoint)
        st.exp_avg.copy_(moments["exp_avg"])
        st.exp_avg_sq.copy_(moments["exp_avg_sq"])
        st.step = int(payload["adamw_updates"])
        base = unwrap_base_model(_unwrap_wrappers(self.model))
        if hasattr(base, "_bd_step"):
            base._bd_step = int(payload.get("noise_draws", payload["global_step"]))
        self.state.global_step = int(payload["global_step"])
