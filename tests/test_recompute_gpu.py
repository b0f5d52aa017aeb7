"""Activation recompute of the noisy stream (training/checkpointing.py:12-52 checkpoints every
LoRA layer): a layer that recomputes keeps only its input and reruns the same deterministic
kernels in the backward, so loss and every LoRA gradient are bit-identical with recompute off,
on for every layer, and on for the layers an HBM budget leaves out ("auto")."""
import pytest
import torch

from oracle.model import Cfg, init_lora, init_params
from uno_amd.layers import saved_bytes_per_row
from uno_amd.model import UnoQwen3Config, UnoQwen3ForCausalLM
from uno_amd.training.checkpointing import configure_gradient_checkpointing
from uno_amd.training.config import LoraSettings, UnoObjectiveConfig
from uno_amd.training.curriculum import BlockCurriculumPlan
from uno_amd.training.lora import create_lora_model
from uno_amd.training.trainer import UnoTrainer, UnoTrainingArguments

pytestmark = pytest.mark.gpu

SPEC = dict(vocab_size=8192, hidden_size=512, intermediate_size=1536, num_hidden_layers=4, num_attention_heads=4,
            num_key_value_heads=2, head_dim=128, rank=64, alpha=128, B=2, L=1024, block=16)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_recompute_is_bit_identical(dev, dtype):
    s = SPEC
    ocfg = Cfg(s["vocab_size"], s["hidden_size"], s["intermediate_size"], s["num_hidden_layers"],
               s["num_attention_heads"], s["num_key_value_heads"], s["head_dim"], lora_rank=s["rank"],
               lora_alpha=s["alpha"])
    ucfg = UnoQwen3Config(vocab_size=ocfg.vocab_size, hidden_size=ocfg.hidden_size,
                          intermediate_size=ocfg.intermediate_size, num_hidden_layers=ocfg.num_hidden_layers,
                          num_attention_heads=ocfg.num_attention_heads, num_key_value_heads=ocfg.num_key_value_heads,
                          head_dim=ocfg.head_dim, block_size=s["block"])
    model = UnoQwen3ForCausalLM(ucfg, device=dev, dtype=dtype)
    model.load_weights(init_params(ocfg, seed=0))
    lm, _ = create_lora_model(model, LoraSettings("all", s["rank"], s["alpha"], 0.0))
    lm.load_lora(init_lora(ocfg, seed=1))
    trainer = UnoTrainer(model=lm, objective=UnoObjectiveConfig(ce_target="ground_truth", ce_weight=1.0,
                                                                kl_weight=0.0, tv_weight=0.0),
                         curriculum=BlockCurriculumPlan.fixed(s["block"], 100, s["L"], s["B"]),
                         args=UnoTrainingArguments(learning_rate=1e-4))
    g = torch.Generator().manual_seed(2)
    ids = torch.randint(0, s["vocab_size"] - 1, (s["B"], s["L"]), generator=g)
    labels = ids.clone()
    labels[:, :128] = -100
    batch = {"input_ids": ids.to(dev), "labels": labels.to(dev), "attention_mask": torch.ones_like(ids).to(dev)}
    rows = s["B"] * s["L"]
    per_layer = saved_bytes_per_row(model.model.geo, s["rank"], torch.tensor([], dtype=dtype).element_size()) * rows
    results = {}
    for name, policy, budget in (("off", False, None), ("all", True, None), ("auto-half", "auto", 2 * per_layer + 1),
                                 ("auto-fits", "auto", 100 * per_layer)):
        print(f"[recompute] {dtype} policy {name}", flush=True)
        configure_gradient_checkpointing(lm, policy, hbm_budget_bytes=budget)
        model._bd_step = 0
        for p in lm.parameters():
            p.grad = None
        loss = trainer.compute_loss(lm, batch)
        loss.backward()
        torch.cuda.synchronize()
        plan = list(model.model.last_recompute_plan)
        results[name] = (loss.detach().clone(), {n: p.grad.clone() for n, p in lm.lora_tensors().items()}, plan)
    assert results["off"][2] == [False] * 4
    assert results["all"][2] == [True] * 4
    assert results["auto-fits"][2] == [False] * 4
    assert 0 < sum(results["auto-half"][2]) < 4, results["auto-half"][2]
    ref_loss, ref_grads, _ = results["off"]
    for name in ("all", "auto-half", "auto-fits"):
        loss, grads, _ = results[name]
        assert torch.equal(loss, ref_loss), name
        for n, v in ref_grads.items():
            assert torch.equal(grads[n], v), (name, n)
