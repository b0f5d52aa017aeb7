"""Adapter checkpoints in the PEFT on-disk format and exact resume at a curriculum boundary.

The reference saves the PEFT adapter at every checkpoint and the complete training state at each
curriculum-stage boundary (training/trainer.py:89-128), and resumes only from such boundaries
(validate_curriculum_resume, training/trainer.py:131-146). Here: train two steps, checkpoint at the
stage boundary, train two more; a fresh model resumed from the checkpoint must reproduce those two
steps (losses and final LoRA weights) from the saved adapters, AdamW moments, step and the
position of the model's noise stream."""
import json

import pytest
import torch
from safetensors.torch import load_file

from oracle.model import Cfg, init_lora, init_params
from uno_amd.model import UnoQwen3Config, UnoQwen3ForCausalLM
from uno_amd.training.config import LoraSettings, UnoObjectiveConfig
from uno_amd.training.curriculum import BlockCurriculumPlan
from uno_amd.training.lora import create_lora_model
from uno_amd.training.trainer import OPTIMIZER_STATE, UnoTrainer, UnoTrainingArguments

pytestmark = pytest.mark.gpu

SPEC = dict(vocab_size=4096, hidden_size=256, intermediate_size=768, num_hidden_layers=2, num_attention_heads=4,
            num_key_value_heads=2, head_dim=64, rank=8, alpha=16, B=2, L=256, prompt=64)


def _plan():
    tps = SPEC["B"] * SPEC["L"]
    return BlockCurriculumPlan.from_dict({"tokens_per_step": tps, "sequence_length": SPEC["L"],
                                          "global_batch_size": SPEC["B"], "seed": 0,
                                          "stages": [{"block_size": 4, "tokens": 2 * tps},
                                                     {"block_size": 8, "tokens": 2 * tps}]})


def _trainer(dev, lora_seed):
    ocfg = Cfg(SPEC["vocab_size"], SPEC["hidden_size"], SPEC["intermediate_size"], SPEC["num_hidden_layers"],
               SPEC["num_attention_heads"], SPEC["num_key_value_heads"], SPEC["head_dim"],
               lora_rank=SPEC["rank"], lora_alpha=SPEC["alpha"])
    ucfg = UnoQwen3Config(vocab_size=ocfg.vocab_size, hidden_size=ocfg.hidden_size,
                          intermediate_size=ocfg.intermediate_size, num_hidden_layers=ocfg.num_hidden_layers,
                          num_attention_heads=ocfg.num_attention_heads, num_key_value_heads=ocfg.num_key_value_heads,
                          head_dim=ocfg.head_dim, block_size=4)
    model = UnoQwen3ForCausalLM(ucfg, device=dev, dtype=torch.float32)
    model.load_weights(init_params(ocfg, seed=0))
    lm, _ = create_lora_model(model, LoraSettings("all", SPEC["rank"], SPEC["alpha"], 0.0))
    lm.load_lora(init_lora(ocfg, seed=lora_seed))
    trainer = UnoTrainer(model=lm, objective=UnoObjectiveConfig(ce_target="ground_truth", ce_weight=1.0,
                                                                kl_weight=0.0, tv_weight=0.0),
                         curriculum=_plan(), args=UnoTrainingArguments(learning_rate=1e-3))
    g = torch.Generator().manual_seed(7)
    ids = torch.randint(0, ocfg.vocab_size - 1, (SPEC["B"], SPEC["L"]), generator=g)
    labels = ids.clone()
    labels[:, :SPEC["prompt"]] = -100
    batch = {k: v.to(dev) for k, v in {"input_ids": ids, "labels": labels,
                                        "attention_mask": torch.ones_like(ids)}.items()}
    return lm, trainer, batch


def _weights(lm):
    return {n: p.detach().cpu().clone() for n, p in lm.lora_tensors().items()}


def test_peft_checkpoint_and_exact_resume(dev, tmp_path):
    lm, trainer, batch = _trainer(dev, lora_seed=1)
    print("[checkpoint] run A: 2 steps, checkpoint, 2 steps", flush=True)
    for _ in range(2):
        trainer.train_step(batch)
    ckpt = trainer.save_checkpoint(tmp_path)
    saved = _weights(lm)
    losses_a = [trainer.train_step(batch).item() for _ in range(2)]
    final_a = _weights(lm)
    torch.cuda.synchronize()

    # PEFT on-disk format: tensor names and shapes the inference loader reads, fp32 values equal to
    # the weights at the checkpoint, adapter_config.json, and the boundary's resume state.
    assert ckpt.name == "checkpoint-2"
    tensors = load_file(str(ckpt / "adapter_model.safetensors"))
    r, H = SPEC["rank"], SPEC["hidden_size"]
    q_out = SPEC["num_attention_heads"] * SPEC["head_dim"]
    shapes = {"self_attn.q_proj.lora_A.weight": (r, H), "self_attn.q_proj.lora_B.weight": (q_out, r),
              "self_attn.o_proj.lora_A.weight": (r, q_out), "mlp.down_proj.lora_A.weight": (r, SPEC["intermediate_size"]),
              "mlp.down_proj.lora_B.weight": (H, r), "mlp.gate_proj.lora_B.weight": (SPEC["intermediate_size"], r)}
    for li in range(SPEC["num_hidden_layers"]):
        for suffix, shape in shapes.items():
            name = f"base_model.model.model.layers.{li}.{suffix}"
            assert tuple(tensors[name].shape) == shape and tensors[name].dtype == torch.float32, name
    assert len(tensors) == 14 * SPEC["num_hidden_layers"]
    for n, v in tensors.items():
        assert torch.equal(v, saved[n]), n
    cfg = json.loads((ckpt / "adapter_config.json").read_text())
    assert cfg["peft_type"] == "LORA" and cfg["r"] == r and cfg["lora_alpha"] == SPEC["alpha"]
    assert sorted(cfg["target_modules"]) == sorted(["q_proj", "k_proj", "v_proj", "o_proj", "gate_proj", "up_proj",
                                                    "down_proj"])
    state = json.loads((ckpt / "uno_curriculum_state.json").read_text())
    assert state["global_step"] == 2 and state["reason"] == "completed_block_size_4" and state["adamw_updates"] == 2
    assert state["noise_draws"] == 2
    assert (ckpt / OPTIMIZER_STATE).is_file()

    print("[checkpoint] run B: fresh adapters, resume, 2 steps", flush=True)
    lm_b, trainer_b, batch_b = _trainer(dev, lora_seed=5)
    trainer_b.resume_from_checkpoint(ckpt)
    assert trainer_b.state.global_step == 2
    losses_b = [trainer_b.train_step(batch_b).item() for _ in range(2)]
    final_b = _weights(lm_b)
    torch.cuda.synchronize()
    for a, b in zip(losses_a, losses_b):
        assert abs(a - b) <= 1e-6 * abs(a), (losses_a, losses_b)
    for n, v in final_a.items():
        assert ((final_b[n] - v).norm() / v.norm()).item() <= 1e-6, n


def test_resume_requires_a_boundary_checkpoint(dev, tmp_path):
    lm, trainer, batch = _trainer(dev, lora_seed=1)
    trainer.train_step(batch)
    ckpt = trainer.save_checkpoint(tmp_path)      # step 1 is inside the first stage
    assert not (ckpt / OPTIMIZER_STATE).exists()
    with pytest.raises(FileNotFoundError, match="curriculum-boundary"):
        trainer.resume_from_checkpoint(ckpt)


def test_incomplete_or_mismatched_adapter_is_rejected(dev, tmp_path):
    """load_adapter refuses a partial or misshaped adapter file before writing anything."""
    from safetensors.torch import save_file

    from uno_amd.training.lora import load_adapter, save_adapter

    lm, _, _ = _trainer(dev, lora_seed=1)
    before = _weights(lm)
    save_adapter(lm, tmp_path / "full")
    tensors = load_file(str(tmp_path / "full" / "adapter_model.safetensors"))
    names = sorted(tensors)
    partial = dict(tensors)
    del partial[names[3]]
    (tmp_path / "partial").mkdir()
    save_file(partial, str(tmp_path / "partial" / "adapter_model.safetensors"))
    with pytest.raises(ValueError, match="incomplete"):
        load_adapter(lm, tmp_path / "partial")
    wrong = dict(tensors)
    wrong[names[0]] = torch.zeros(wrong[names[0]].shape[0] + 1, wrong[names[0]].shape[1])
    (tmp_path / "wrong").mkdir()
    save_file(wrong, str(tmp_path / "wrong" / "adapter_model.safetensors"))
    with pytest.raises(ValueError, match="shape"):
        load_adapter(lm, tmp_path / "wrong")
    for n, v in _weights(lm).items():
        assert torch.equal(v, before[n]), n
