"""The step as a drop-in for the reference trainer: the adapters are ordinary torch parameters.

* A torch optimizer over ``lm.parameters()``: compute_loss -> backward -> clip_grad_norm_ ->
  torch.optim.AdamW -> zero_grad(set_to_none=True), three steps, against the oracle's three steps
  (training/train.py:282-288 optimizer settings). The compute copies the kernels read must follow
  torch's in-place updates, and the gradient views must survive set_to_none.
* HF ``Trainer.train()`` of ``UnoTrainer`` built with the reference's constructor arguments
  (training/train.py:307-315: model, args, train_dataset, data_collator, objective, curriculum),
  three steps through HF's own loop, against the same oracle run.
* Hand-made gradient edits (a replaced ``.grad``, ``.grad = None`` on some tensors) are adopted.
"""
import pytest
import torch

from oracle import step as ostep
from oracle.model import Cfg, init_lora, init_params
from uno_amd.model import UnoQwen3Config, UnoQwen3ForCausalLM
from uno_amd.training.config import LoraSettings, UnoObjectiveConfig
from uno_amd.training.curriculum import BlockCurriculumPlan
from uno_amd.training.data import UnoDataCollator
from uno_amd.training.lora import create_lora_model
from uno_amd.training.trainer import UnoTrainer, UnoTrainingArguments
from transformers import TrainerCallback

pytestmark = pytest.mark.gpu

SPEC = dict(vocab_size=4096, hidden_size=256, intermediate_size=768, num_hidden_layers=2, num_attention_heads=4,
            num_key_value_heads=2, head_dim=64, rank=8, alpha=16, L=256, prompt=64, block=4)
OBJ = (UnoObjectiveConfig(ce_target="ground_truth", ce_weight=1.0, kl_weight=0.0, tv_weight=0.0),
       ostep.Objective(1, 0, 0, "data"))
STEPS = 3


def _fixture(dev, B):
    s = SPEC
    ocfg = Cfg(s["vocab_size"], s["hidden_size"], s["intermediate_size"], s["num_hidden_layers"],
               s["num_attention_heads"], s["num_key_value_heads"], s["head_dim"], lora_rank=s["rank"],
               lora_alpha=s["alpha"])
    params, lora = init_params(ocfg, seed=0), init_lora(ocfg, seed=1)
    g = torch.Generator().manual_seed(2)
    ids = torch.randint(0, ocfg.vocab_size - 1, (B, s["L"]), generator=g)
    labels = ids.clone()
    labels[:, :s["prompt"]] = -100
    batch = {"input_ids": ids, "labels": labels, "attention_mask": torch.ones_like(ids)}
    ucfg = UnoQwen3Config(vocab_size=ocfg.vocab_size, hidden_size=ocfg.hidden_size,
                          intermediate_size=ocfg.intermediate_size, num_hidden_layers=ocfg.num_hidden_layers,
                          num_attention_heads=ocfg.num_attention_heads, num_key_value_heads=ocfg.num_key_value_heads,
                          head_dim=ocfg.head_dim, block_size=s["block"])
    model = UnoQwen3ForCausalLM(ucfg, device=dev, dtype=torch.float32)
    model.load_weights(params)
    lm, _ = create_lora_model(model, LoraSettings("all", s["rank"], s["alpha"], 0.0))
    lm.load_lora(lora)
    return ocfg, params, lora, batch, lm


def _oracle(ocfg, params, lora, batch):
    losses, _, final = ostep.train_steps(params, lora, ocfg, batch, OBJ[1], block_size=SPEC["block"],
                                         mask_token_id=ocfg.vocab_size - 1, seed=20260813, steps=STEPS, lr=1e-4)
    return losses, final


def _compare(lm, final, tol=1e-3):
    worst = 0.0
    for name, p in lm.lora_tensors().items():
        ref = final[name.replace("base_model.model.", "", 1)]
        rel = ((p.detach().float().cpu() - ref).norm() / ref.norm()).item()
        worst = max(worst, rel)
    print(f"   worst LoRA weight rel L2 after {STEPS} steps: {worst:.2e}", flush=True)
    assert worst < tol


STEP_KEYS = ("train/ce_loss", "train/reverse_kl_loss", "train/tv_loss", "train/combined_loss", "train/alpha",
             "train/beta", "train/gamma", "train/block_size", "train/transformer_forwards")


class _LogRecorder(TrainerCallback):
    """Records what HF hands to on_log (the path W&B and other reporters take)."""

    def __init__(self):
        self.logs = []

    def on_log(self, args, state, control, logs=None, **kwargs):
        self.logs.append(dict(logs or {}))


def _check_step_logs(trainer, seen, steps, accum):
    """compute_loss logs the reference's per-step keys through Trainer.log (training/trainer.py:288-300):
    one entry per micro-batch in state.log_history (with the global step it ran in) and in on_log."""
    hist = [r for r in trainer.state.log_history if "train/combined_loss" in r]
    cb = [r for r in seen.logs if "train/combined_loss" in r]
    assert len(hist) == len(cb) == steps * accum
    for i, r in enumerate(hist):
        assert set(STEP_KEYS) <= set(r)
        assert r["step"] == i // accum
        assert r["train/block_size"] == SPEC["block"] and r["train/transformer_forwards"] == 1
        assert (r["train/alpha"], r["train/beta"], r["train/gamma"]) == (1.0, 0.0, 0.0)
        assert r["train/ce_loss"] == r["train/combined_loss"] and r["train/tv_loss"] == 0.0
        assert all(isinstance(r[k], (int, float)) for k in STEP_KEYS)
    assert [r["train/combined_loss"] for r in cb] == [r["train/combined_loss"] for r in hist]
    return [r["train/combined_loss"] for r in hist]


def test_torch_adamw_over_lm_parameters(dev, tmp_path):
    print("[drop-in] torch.optim.AdamW over lm.parameters()", flush=True)
    ocfg, params, lora, batch, lm = _fixture(dev, B=2)
    trainer = UnoTrainer(model=lm, objective=OBJ[0],
                         curriculum=BlockCurriculumPlan.fixed(SPEC["block"], 100, SPEC["L"], 2),
                         args=UnoTrainingArguments(output_dir=str(tmp_path), learning_rate=1e-4))
    opt = torch.optim.AdamW(lm.parameters(), lr=1e-4, betas=(0.9, 0.999), eps=1e-8, weight_decay=0.0)
    gb = {k: v.to(dev) for k, v in batch.items()}
    mine = []
    for _ in range(STEPS):
        loss = trainer.compute_loss(lm, gb)
        loss.backward()
        torch.nn.utils.clip_grad_norm_(lm.parameters(), 1.0)
        opt.step()
        opt.zero_grad(set_to_none=True)
        mine.append(loss.item())
    torch.cuda.synchronize()
    losses, final = _oracle(ocfg, params, lora, batch)
    print(f"   losses {mine} vs oracle {losses}", flush=True)
    for a, b in zip(mine, losses):
        assert abs(a - b) / abs(b) < 1e-4
    _compare(lm, final)


def test_hf_trainer_train_reference_constructor(dev, tmp_path):
    print("[drop-in] UnoTrainer(model, args, train_dataset, data_collator, objective, curriculum).train()",
          flush=True)
    ocfg, params, lora, batch, lm = _fixture(dev, B=1)

    class Tok:
        pad_token_id = 0
        padding_side = "right"

    dataset = [{"input_ids": batch["input_ids"][0].tolist(), "labels": batch["labels"][0].tolist()}]
    args = UnoTrainingArguments(output_dir=str(tmp_path), max_steps=STEPS, per_device_train_batch_size=1,
                                learning_rate=1e-4, logging_strategy="no", dataloader_num_workers=0)
    seen = _LogRecorder()
    trainer = UnoTrainer(model=lm, args=args, train_dataset=dataset,
                         data_collator=UnoDataCollator(Tok(), sequence_length=SPEC["L"]), objective=OBJ[0],
                         curriculum=BlockCurriculumPlan.fixed(SPEC["block"], STEPS, SPEC["L"], 1), callbacks=[seen])
    trainer.train()
    torch.cuda.synchronize()
    assert trainer.state.global_step == STEPS
    losses, final = _oracle(ocfg, params, lora, batch)
    mine = _check_step_logs(trainer, seen, STEPS, 1)
    print(f"   losses {mine} vs oracle {losses}", flush=True)
    for a, b in zip(mine, losses):
        assert abs(a - b) / abs(b) < 1e-4
    _compare(lm, final)
    # the curriculum boundary at the last step saved a portable PEFT adapter
    ckpt = tmp_path / f"checkpoint-{STEPS}"
    assert (ckpt / "adapter_model.safetensors").is_file()
    assert (ckpt / "uno_curriculum_state.json").is_file()


def test_gradient_edits_are_adopted(dev, tmp_path):
    """A replaced .grad contributes its values; a cleared one restarts from zero."""
    print("[drop-in] replaced and cleared gradients", flush=True)
    _, _, _, batch, lm = _fixture(dev, B=2)
    trainer = UnoTrainer(model=lm, objective=OBJ[0],
                         curriculum=BlockCurriculumPlan.fixed(SPEC["block"], 100, SPEC["L"], 2),
                         args=UnoTrainingArguments(output_dir=str(tmp_path), learning_rate=1e-4))
    gb = {k: v.to(dev) for k, v in batch.items()}
    names = list(lm.lora_tensors())
    p0, p1 = lm.lora_tensors()[names[0]], lm.lora_tensors()[names[1]]
    trainer.compute_loss(lm, gb).backward()
    base = {n: p.grad.detach().clone() for n, p in lm.lora_tensors().items()}
    lm.base_model.model._bd_step = 0            # same noise draw again
    p0.grad = torch.full_like(p0, 3.0)         # replaced: accumulates onto 3.0
    p1.grad = None                             # cleared: accumulates onto 0
    trainer.compute_loss(lm, gb).backward()
    torch.cuda.synchronize()
    g = lm.lora_tensors()
    assert torch.allclose(g[names[0]].grad, base[names[0]] + 3.0, rtol=1e-5, atol=1e-6)
    assert torch.allclose(g[names[1]].grad, base[names[1]], rtol=1e-5, atol=1e-7)
    assert torch.allclose(g[names[2]].grad, 2 * base[names[2]], rtol=1e-5, atol=1e-7)


def test_hf_trainer_gradient_accumulation(dev, tmp_path):
    """HF train() with gradient_accumulation_steps=4 over four different rows: each optimizer step
    sums four micro-batch gradients, each loss divided by 4 (the reference trainer's
    model_accepts_loss_kwargs = False, training/trainer.py:161), every micro-batch draws the next
    noise step, and every micro-batch logs its losses. The rows reach compute_loss in the order of
    HF's shuffling sampler; the oracle replays that order."""
    print("[drop-in] UnoTrainer.train() with gradient_accumulation_steps=4", flush=True)
    accum = 4
    ocfg, params, lora, batch, lm = _fixture(dev, B=accum)

    class Tok:
        pad_token_id = 0
        padding_side = "right"

    class Recording(UnoTrainer):
        order = []

        def compute_loss(self, model, inputs, return_outputs=False, num_items_in_batch=None):
            self.order.append(inputs["input_ids"].detach().cpu().clone())
            return super().compute_loss(model, inputs, return_outputs, num_items_in_batch)

    dataset = [{"input_ids": batch["input_ids"][b].tolist(), "labels": batch["labels"][b].tolist()}
               for b in range(accum)]
    args = UnoTrainingArguments(output_dir=str(tmp_path), max_steps=STEPS, per_device_train_batch_size=1,
                                gradient_accumulation_steps=accum, learning_rate=1e-4, logging_strategy="no",
                                dataloader_num_workers=0)
    seen = _LogRecorder()
    trainer = Recording(model=lm, args=args, train_dataset=dataset,
                        data_collator=UnoDataCollator(Tok(), sequence_length=SPEC["L"]), objective=OBJ[0],
                        curriculum=BlockCurriculumPlan.fixed(SPEC["block"], STEPS, SPEC["L"], accum),
                        callbacks=[seen])
    trainer.train()
    torch.cuda.synchronize()
    assert trainer.state.global_step == STEPS
    assert len(trainer.order) == STEPS * accum
    rows = {tuple(batch["input_ids"][b].tolist()): b for b in range(accum)}
    micro = []
    for ids in trainer.order:
        b = rows[tuple(ids[0].tolist())]
        micro.append({"input_ids": batch["input_ids"][b:b + 1], "labels": batch["labels"][b:b + 1]})
    print(f"   row order {[rows[tuple(i[0].tolist())] for i in trainer.order]}", flush=True)
    losses, _, final = ostep.train_steps(params, lora, ocfg, batch, OBJ[1], block_size=SPEC["block"],
                                         mask_token_id=ocfg.vocab_size - 1, seed=20260813, steps=STEPS, lr=1e-4,
                                         micro_batches=micro, grad_accum=accum)
    mine = _check_step_logs(trainer, seen, STEPS, accum)
    print(f"   losses {mine} vs oracle {losses}", flush=True)
    for a, b in zip(mine, losses):
        assert abs(a - b) / abs(b) < 1e-4
    _compare(lm, final)


def test_ce_only_batch_without_ce_rows_backpropagates(dev, tmp_path):
    """A CE-only objective on a micro-batch with no CE rows (every label -100) still returns a loss
    connected to the graph, as the reference's noisy_hidden.sum() * 0.0 (training/trainer.py:249):
    backward() runs and leaves every LoRA gradient at zero."""
    print("[drop-in] CE-only step on a batch with no CE rows", flush=True)
    _, _, _, batch, lm = _fixture(dev, B=2)
    trainer = UnoTrainer(model=lm, objective=OBJ[0],
                         curriculum=BlockCurriculumPlan.fixed(SPEC["block"], 100, SPEC["L"], 2),
                         args=UnoTrainingArguments(output_dir=str(tmp_path), learning_rate=1e-4))
    gb = {k: v.to(dev) for k, v in batch.items()}
    gb["labels"] = torch.full_like(gb["labels"], -100)
    loss = trainer.compute_loss(lm, gb)
    assert loss.requires_grad and loss.grad_fn is not None
    loss.backward()
    torch.cuda.synchronize()
    assert loss.item() == 0.0
    for name, p in lm.lora_tensors().items():
        assert p.grad is not None and torch.count_nonzero(p.grad).item() == 0, name
    assert trainer.state.log_history[-1]["train/ce_loss"] == 0.0
