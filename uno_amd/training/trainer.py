"""Uno training step as an HF Trainer (counterpart of training/trainer.py in the reference).

``UnoTrainer(*, objective, curriculum, **trainer_kwargs)`` takes the reference's constructor
(training/trainer.py:152-168, called as in training/train.py:307-315) and is a
``transformers.Trainer``: ``train()``, callbacks, LR scheduling, clipping and checkpointing are
HF's. What it changes is underneath ``compute_loss`` (same signature and control flow,
training/trainer.py:174-308): the decoder runs the two-stream HIP path, and the objectives are the
fused LM-head kernels. Its default optimizer is ``FusedLoraAdamW`` (torch AdamW semantics over the
adapter's flat buffers); any torch optimizer over ``model.parameters()`` works too, since the
adapters follow their fp32 parameters whatever updates them.

``train_step(inputs)`` runs one optimizer step outside HF's loop (loss, backward, global-norm clip,
AdamW, LR schedule): the unit the benchmark times.
"""
from __future__ import annotations

import json
import os
import tempfile
import warnings
from dataclasses import dataclass, field
from pathlib import Path

import torch
from transformers import Trainer, TrainerCallback, TrainingArguments

from ..layers import GatherRows
from ..objectives import distribution_loss, fused_weighted_ce, teacher_argmax
from ..optim import FusedLoraAdamW
from .config import UnoObjectiveConfig
from .constants import DEFAULT_LEARNING_RATE, IGNORE_INDEX
from .curriculum import BlockCurriculumPlan, set_model_block_size
from .lora import TokenwiseLoraRouter, load_adapter, make_saved_adapter_portable, save_adapter
from .losses import shift_labels_for_next_token
from .modeling import (extract_uno_regions, prepare_uno_layout, run_prepared_uno_forward, unwrap_base_model,
                       validate_uno_model)

# AdamW moments of a curriculum-boundary checkpoint written by save_checkpoint (flat fp32 buffers).
OPTIMIZER_STATE = "uno_optimizer_state.safetensors"
CURRICULUM_STATE = "uno_curriculum_state.json"


def combine_objective_losses(ce_loss, kl_loss, tv_loss, objective: UnoObjectiveConfig):
    """alpha * CE + beta * KL + gamma * TV (training/trainer.py:34-46)."""
    objective.validate()
    return objective.ce_weight * ce_loss + objective.kl_weight * kl_loss + objective.tv_weight * tv_loss


def sync_scheduler_param_groups(lr_scheduler) -> None:
    """Re-aligns an LR scheduler with its optimizer's parameter groups when something (DeepSpeed
    consolidation in the reference, training/trainer.py:49-79) changed their number after the
    scheduler was built. Only a scheduler whose groups all share one base LR can be re-aligned."""
    opt = getattr(lr_scheduler, "optimizer", None)
    groups = getattr(opt, "param_groups", None)
    base = getattr(lr_scheduler, "base_lrs", None)
    if groups is None or base is None:
        return
    n = len(groups)
    lambdas = getattr(lr_scheduler, "lr_lambdas", None)
    if len(base) == n and (lambdas is None or len(lambdas) == n):
        return
    if len(set(map(float, base))) > 1:
        raise RuntimeError(f"Optimizer groups changed, and the scheduler's base LRs differ ({base}); "
                           "cannot re-align them.")
    lr_scheduler.base_lrs = [g.get("initial_lr", g.get("lr", 0.0)) for g in groups]
    if lambdas is not None:
        if not lambdas:
            raise RuntimeError("The scheduler has no LR lambda to extend.")
        lr_scheduler.lr_lambdas = (list(lambdas) + [lambdas[-1]] * n)[:n]
    if hasattr(lr_scheduler, "_last_lr"):
        lr_scheduler._last_lr = [g["lr"] for g in groups]


def _write_json(path: Path, payload: dict) -> None:
    tmp = path.with_name(path.name + ".tmp")
    tmp.write_text(json.dumps(payload, indent=2, sort_keys=True) + "\n")
    tmp.replace(path)


class SchedulerSyncCallback(TrainerCallback):
    """Re-aligns the scheduler before every step (training/trainer.py:82-86)."""

    def on_step_begin(self, args, state, control, **kwargs):
        sync_scheduler_param_groups(kwargs.get("lr_scheduler"))
        return control


class CurriculumCheckpointCallback(TrainerCallback):
    """Sets each step's block size and saves at every stage boundary (training/trainer.py:89-128)."""

    def __init__(self, curriculum: BlockCurriculumPlan) -> None:
        self.curriculum = curriculum

    def on_step_begin(self, args, state, control, **kwargs):
        if state.global_step < self.curriculum.max_steps:
            set_model_block_size(kwargs["model"], self.curriculum.stage_for_step(state.global_step).block_size)
        return control

    def on_step_end(self, args, state, control, **kwargs):
        if state.global_step in self.curriculum.checkpoint_reasons:
            control.should_save = True
        return control

    def on_save(self, args, state, control, **kwargs):
        if not state.is_world_process_zero:
            return control
        ckpt = Path(args.output_dir) / f"checkpoint-{state.global_step}"
        make_saved_adapter_portable(ckpt)
        reason = self.curriculum.checkpoint_reasons.get(state.global_step)
        if reason:
            _write_json(ckpt / CURRICULUM_STATE, {"version": 1, "global_step": state.global_step, "reason": reason,
                                                  "curriculum_sha256": self.curriculum.sha256()})
        return control


def validate_curriculum_resume(checkpoint, curriculum: BlockCurriculumPlan) -> None:
    """A resume must start from a boundary checkpoint of this very curriculum."""
    path = Path(checkpoint) / CURRICULUM_STATE
    if not path.is_file():
        raise FileNotFoundError(f"Uno resumes only from curriculum-boundary checkpoints; {path} is missing.")
    state = json.loads(path.read_text())
    if state.get("curriculum_sha256") != curriculum.sha256():
        raise ValueError(f"{checkpoint} was written under a different curriculum.")
    if state.get("global_step") not in curriculum.checkpoint_reasons:
        raise ValueError(f"Step {state.get('global_step')} of {checkpoint} is not a curriculum boundary.")


@dataclass
class UnoTrainingArguments(TrainingArguments):
    """TrainingArguments with the reference run's settings as defaults (training/train.py:275-305):
    torch AdamW, weight decay 0, clip 1.0, warmup-stable schedule without decay; no reporting and
    no periodic saving (the curriculum callback saves at stage boundaries)."""

    # HF creates the output directory when the Trainer is built: default to a scratch location
    output_dir: str | None = field(default=os.path.join(tempfile.gettempdir(), "uno_trainer_output"))
    learning_rate: float = field(default=DEFAULT_LEARNING_RATE)
    weight_decay: float = field(default=0.0)
    max_grad_norm: float = field(default=1.0)
    optim: str = field(default="adamw_torch")
    lr_scheduler_type: str = field(default="warmup_stable_decay")
    lr_scheduler_kwargs: dict | str | None = field(default_factory=lambda: {"num_decay_steps": 0})
    save_strategy: str = field(default="no")
    remove_unused_columns: bool = field(default=False)
    dataloader_drop_last: bool = field(default=True)
    report_to: str | list[str] | None = field(default="none")
    disable_tqdm: bool | None = field(default=True)


def _unwrap_wrappers(model):
    while getattr(model, "module", None) is not None:
        model = model.module
    return model


class UnoTrainer(Trainer):
    """LoRA-only, single-forward Uno trainer on the MI355X kernels."""

    def __init__(self, *, objective: UnoObjectiveConfig, curriculum: BlockCurriculumPlan, **kwargs) -> None:
        objective.validate()
        if kwargs.get("args") is None:
            kwargs["args"] = UnoTrainingArguments()
        super().__init__(**kwargs)
        self.model_accepts_loss_kwargs = False
        self.objective = objective
        self.curriculum = curriculum
        validate_uno_model(self.model)
        self._lora_router = TokenwiseLoraRouter(self.model)
        self.add_callback(SchedulerSyncCallback())
        self.add_callback(CurriculumCheckpointCallback(curriculum))

    # ---- optimizer and schedule ---------------------------------------------------------------
    def create_optimizer(self, model=None):
        """FusedLoraAdamW for the torch AdamW settings of the run (the Trainer clips beforehand);
        any other choice, or an optimizer passed in, is left to the Trainer."""
        if self.optimizer is None and self.args.optim in ("adamw_torch", "adamw_torch_fused") \
                and self.optimizer_cls_and_kwargs is None:
            lora = getattr(_unwrap_wrappers(model if model is not None else self.model), "state", None)
            if lora is not None:
                a = self.args
                self.optimizer = FusedLoraAdamW(lora, lr=a.learning_rate, betas=(a.adam_beta1, a.adam_beta2),
                                                eps=a.adam_epsilon, weight_decay=a.weight_decay, max_grad_norm=None)
                return self.optimizer
        return super().create_optimizer(model)

    def create_scheduler(self, num_training_steps, optimizer=None):
        scheduler = super().create_scheduler(num_training_steps, optimizer)
        sync_scheduler_param_groups(scheduler)
        return scheduler

    # ---- the step -----------------------------------------------------------------------------
    def compute_loss(self, model, inputs, return_outputs=False, num_items_in_batch=None):
        del num_items_in_batch
        step = min(self.state.global_step, self.curriculum.max_steps - 1)
        block_size = self.curriculum.stage_for_step(step).block_size
        set_model_block_size(model, block_size)

        labels = inputs.get("labels")
        if labels is None:
            raise RuntimeError("Uno training batches must contain labels.")
        unwrapped = self.accelerator.unwrap_model(model)
        base_model = unwrap_base_model(unwrapped)
        sequence_length = inputs["input_ids"].size(-1)
        original_positions, model_positions, noisy_region_mask = prepare_uno_layout(
            base_model, inputs["input_ids"], inputs.get("position_ids"))
        shifted_labels = shift_labels_for_next_token(labels, original_positions)
        concatenated_ids, concatenated_positions, bd_mask, noised_positions, _, p_mask = \
            base_model.prepare_for_bd_training(inputs["input_ids"], model_positions, labels == IGNORE_INDEX)
        self._lora_router.set_token_mask(noisy_region_mask)
        # The clean stream's final hidden states feed only the teacher side of the losses; the
        # decoder skips them for this forward when no loss reads them.
        decoder = base_model.model
        keep = getattr(decoder, "clean_final_needed", None)
        if keep is not None:
            decoder.clean_final_needed = self._needs_teacher()
        try:
            hidden_states = run_prepared_uno_forward(model, base_model, inputs, concatenated_ids,
                                                     concatenated_positions, bd_mask)
        finally:
            if keep is not None:
                decoder.clean_final_needed = keep
        noisy_hidden, clean_hidden = extract_uno_regions(hidden_states, noisy_region_mask, sequence_length)

        supervised_mask = labels != IGNORE_INDEX
        valid_next_token = shifted_labels != IGNORE_INDEX
        ce_mask = noised_positions & valid_next_token
        # one host synchronisation for both counts (the CE row count sizes the LM-head GEMM)
        token_count, ce_count = (int(x) for x in torch.stack([supervised_mask.sum(), ce_mask.sum()]).tolist())
        dev = noisy_hidden.device
        inv_n = torch.full((), 1.0 / max(token_count, 1), device=dev, dtype=torch.float32)
        # inactive or empty terms stay connected to the graph (training/trainer.py:249), so that
        # backward() works, with zero gradients, on a micro-batch that has no rows for the loss
        zero_loss = noisy_hidden.sum() * 0.0
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
        # Per-step metrics through Trainer.log (state.log_history, on_log callbacks, reporters),
        # as training/trainer.py:288-300; one device-to-host copy for the four values.
        ce_v, kl_v, tv_v, comb_v = torch.stack([t.detach().float().reshape(()) for t in
                                                (ce_loss, kl_loss, tv_loss, combined_loss)]).tolist()
        self.log({
            "train/ce_loss": ce_v, "train/reverse_kl_loss": kl_v, "train/tv_loss": tv_v,
            "train/combined_loss": comb_v, "train/alpha": self.objective.ce_weight,
            "train/beta": self.objective.kl_weight, "train/gamma": self.objective.tv_weight,
            "train/block_size": block_size, "train/transformer_forwards": 1,
        })
        if return_outputs:
            return combined_loss, {"loss": combined_loss, "ce_loss": ce_loss, "reverse_kl_loss": kl_loss,
                                   "tv_loss": tv_loss}
        return combined_loss

    def _needs_teacher(self) -> bool:
        """Whether the losses read the clean stream's hidden states (TV, KL, clean-argmax CE targets)."""
        o = self.objective
        return o.kl_weight > 0 or o.tv_weight > 0 or (o.ce_weight > 0 and o.internal_ce_target != "data")

    # ---- one optimizer step outside HF's loop ---------------------------------------------------
    def _ensure_optimizer(self) -> None:
        if self.optimizer is None:
            self.create_optimizer_and_scheduler(num_training_steps=self.curriculum.max_steps)

    def train_step(self, inputs) -> torch.Tensor:
        """compute_loss + backward + global-norm clip + AdamW + LR schedule for one micro-batch."""
        self._ensure_optimizer()
        self.model.train()
        loss = self.compute_loss(self.model, self._prepare_inputs(inputs))
        self.accelerator.backward(loss)
        self.optimizer_step()
        return loss.detach()

    def optimizer_step(self) -> None:
        """Clip to max_grad_norm, step the optimizer and the LR schedule, zero the gradients."""
        self._ensure_optimizer()
        opt = self.optimizer
        if isinstance(opt, FusedLoraAdamW):
            opt.step(max_grad_norm=self.args.max_grad_norm)
        else:
            if self.args.max_grad_norm:
                torch.nn.utils.clip_grad_norm_([p for p in self.model.parameters() if p.grad is not None],
                                               self.args.max_grad_norm)
            opt.step()
        if self.lr_scheduler is not None:
            self.lr_scheduler.step()
        opt.zero_grad(set_to_none=True)
        self.state.global_step += 1

    # ---- saving ---------------------------------------------------------------------------------
    def _save(self, output_dir: str | None = None, state_dict=None) -> None:
        """Writes the adapter in PEFT format (the frozen base is never saved) plus the Trainer's
        own files."""
        del state_dict
        out = Path(output_dir if output_dir is not None else self.args.output_dir)
        save_adapter(_unwrap_wrappers(self.model), out)
        if self.processing_class is not None:
            self.processing_class.save_pretrained(str(out))
        torch.save(self.args, out / "training_args.bin")

    def save_checkpoint(self, output_dir) -> Path:
        """Adapter checkpoint (PEFT format); at curriculum boundaries also the complete resume
        state (training/trainer.py:89-128 saves full state there): the AdamW moments and update
        count, the position of the model's noise stream (what the reference's RNG state restores),
        then the curriculum state file, written last so that its presence marks a complete
        checkpoint."""
        from safetensors.torch import save_file

        ckpt = Path(output_dir) / f"checkpoint-{self.state.global_step}"
        save_adapter(_unwrap_wrappers(self.model), ckpt)
        make_saved_adapter_portable(ckpt)
        reason = self.curriculum.checkpoint_reasons.get(self.state.global_step)
        if reason:
            self._ensure_optimizer()
            st = _unwrap_wrappers(self.model).state
            save_file({"exp_avg": st.exp_avg.detach().cpu(), "exp_avg_sq": st.exp_avg_sq.detach().cpu()},
                      str(ckpt / OPTIMIZER_STATE))
            base = unwrap_base_model(_unwrap_wrappers(self.model))
            _write_json(ckpt / CURRICULUM_STATE, {
                "version": 1, "global_step": self.state.global_step, "reason": reason,
                "curriculum_sha256": self.curriculum.sha256(), "adamw_updates": st.step,
                "noise_draws": int(getattr(base, "_bd_step", 0))})
        return ckpt

    def resume_from_checkpoint(self, checkpoint) -> None:
        """Restores a save_checkpoint boundary checkpoint (adapters, AdamW moments, update count,
        noise-stream position, global step): the next train_step continues the run exactly."""
        from safetensors.torch import load_file

        checkpoint = Path(checkpoint)
        validate_curriculum_resume(checkpoint, self.curriculum)
        payload = json.loads((checkpoint / CURRICULUM_STATE).read_text())
        moments_path = checkpoint / OPTIMIZER_STATE
        if not moments_path.is_file() or "adamw_updates" not in payload:
            raise FileNotFoundError(f"{checkpoint} holds no optimizer state ({OPTIMIZER_STATE}).")
        moments = load_file(str(moments_path))
        self._ensure_optimizer()
        st = _unwrap_wrappers(self.model).state
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
        if self.lr_scheduler is not None:
            with warnings.catch_warnings():    # replaying the schedule, no optimizer step is due
                warnings.simplefilter("ignore", UserWarning)
                for _ in range(self.state.global_step):
                    self.lr_scheduler.step()
