"""LoRA target subsets (training/lora.py:14-43 resolves them, :66-92 attaches PEFT adapters to
those projections only): the step with adapters on "qv", "qkvo" or a list of MLP projections,
against the oracle with the same targets (fp32: loss 1e-5, gradients 2e-4; bf16 at a width that
takes the fused 256x256 and SwiGLU kernels), plus what a caller observes: only the targeted
lora_A / lora_B tensors exist, train and are saved, and ten AdamW steps follow the oracle's."""
import json

import pytest
import torch

from oracle import step as ostep
from oracle.model import Cfg, init_lora, init_params
from uno_amd.model import UnoQwen3Config, UnoQwen3ForCausalLM
from uno_amd.training.config import LoraSettings, UnoObjectiveConfig
from uno_amd.training.curriculum import BlockCurriculumPlan
from uno_amd.training.lora import create_lora_model, resolve_lora_targets, save_adapter
from uno_amd.training.trainer import UnoTrainer, UnoTrainingArguments

pytestmark = pytest.mark.gpu

TINY = dict(vocab_size=4096, hidden_size=256, intermediate_size=768, num_hidden_layers=2, num_attention_heads=4,
            num_key_value_heads=2, head_dim=64, rank=8, alpha=16, B=2, L=256, prompt=64, block=4)
WIDE = dict(vocab_size=8192, hidden_size=1024, intermediate_size=2048, num_hidden_layers=2, num_attention_heads=8,
            num_key_value_heads=2, head_dim=128, rank=32, alpha=64, B=2, L=512, prompt=64, block=16)
OBJ = (UnoObjectiveConfig(ce_target="ground_truth", ce_weight=1.0, kl_weight=0.0, tv_weight=0.0),
       ostep.Objective(1, 0, 0, "data"))
TARGETS = ["qv", "qkvo", "gate_proj,down_proj", "k_proj,up_proj"]


def _setup(spec, target, dtype, dev):
    targets = resolve_lora_targets(target)
    ocfg = Cfg(spec["vocab_size"], spec["hidden_size"], spec["intermediate_size"], spec["num_hidden_layers"],
               spec["num_attention_heads"], spec["num_key_value_heads"], spec["head_dim"],
               lora_rank=spec["rank"], lora_alpha=spec["alpha"], lora_targets=targets)
    params = init_params(ocfg, seed=0)
    if dtype == torch.bfloat16:
        params = {k: v.bfloat16().float() for k, v in params.items()}
    lora = init_lora(ocfg, seed=1)
    ucfg = UnoQwen3Config(vocab_size=ocfg.vocab_size, hidden_size=ocfg.hidden_size,
                          intermediate_size=ocfg.intermediate_size, num_hidden_layers=ocfg.num_hidden_layers,
                          num_attention_heads=ocfg.num_attention_heads, num_key_value_heads=ocfg.num_key_value_heads,
                          head_dim=ocfg.head_dim, block_size=spec["block"])
    model = UnoQwen3ForCausalLM(ucfg, device=dev, dtype=dtype)
    model.load_weights(params)
    lm, got = create_lora_model(model, LoraSettings(target, spec["rank"], spec["alpha"], 0.0))
    assert got == targets
    lm.load_lora(lora)
    trainer = UnoTrainer(model=lm, objective=OBJ[0],
                         curriculum=BlockCurriculumPlan.fixed(spec["block"], 1000, spec["L"], spec["B"]),
                         args=UnoTrainingArguments(learning_rate=1e-4))
    g = torch.Generator().manual_seed(2)
    ids = torch.randint(0, ocfg.vocab_size - 1, (spec["B"], spec["L"]), generator=g)
    labels = ids.clone()
    labels[:, :spec["prompt"]] = -100
    batch = {"input_ids": ids, "labels": labels, "attention_mask": torch.ones_like(ids)}
    return ocfg, params, lora, lm, trainer, batch, targets


def _grads(lm):
    return {n.replace("base_model.model.", "", 1): p.grad for n, p in lm.lora_tensors().items()}


@pytest.mark.parametrize("target", TARGETS)
def test_subset_step_fp32(dev, target, tmp_path):
    print(f"[lora targets] fp32 step, target={target!r}", flush=True)
    ocfg, params, lora, lm, trainer, batch, targets = _setup(TINY, target, torch.float32, dev)
    names = set(_grads(lm))
    assert names == set(lora), sorted(names ^ set(lora))
    assert all(n.rsplit(".", 3)[-3] in targets for n in names)
    leaves = {k: v.clone().requires_grad_(True) for k, v in lora.items()}
    ref_loss, _ = ostep.compute_loss(params, leaves, ocfg, batch, OBJ[1], block_size=TINY["block"],
                                     mask_token_id=ocfg.vocab_size - 1, seed=20260813, step=0)
    ref_loss.backward()
    loss = trainer.compute_loss(lm, {k: v.to(dev) for k, v in batch.items()})
    loss.backward()
    torch.cuda.synchronize()
    assert abs(loss.item() - ref_loss.item()) / abs(ref_loss.item()) < 1e-5, (loss.item(), ref_loss.item())
    mine = _grads(lm)
    for k, v in leaves.items():
        r = ((mine[k].cpu() - v.grad).norm() / v.grad.norm().clamp_min(1e-30)).item()
        assert r < 2e-4, (k, r)
    # untargeted slots of the flat storage stay exactly zero (weights and gradients)
    st = lm.state
    for li in range(ocfg.num_hidden_layers):
        for name in ("q_proj", "k_proj", "v_proj", "o_proj", "gate_proj", "up_proj", "down_proj"):
            if name in targets:
                continue
            for buf in (st.master, st.grad):
                assert torch.count_nonzero(st.a_view(buf, li, name)).item() == 0
                assert torch.count_nonzero(st.b_view(buf, li, name)).item() == 0
    out = save_adapter(lm, tmp_path / "adapter")
    cfg = json.loads((out / "adapter_config.json").read_text())
    assert cfg["target_modules"] == list(targets)
    from safetensors.torch import load_file
    saved = load_file(str(out / "adapter_model.safetensors"))
    assert {k.replace("base_model.model.", "", 1) for k in saved} == set(lora)


@pytest.mark.parametrize("target", ["qv", "gate_proj,down_proj"])
def test_subset_ten_adamw_steps_fp32(dev, target):
    print(f"[lora targets] ten AdamW steps, target={target!r}", flush=True)
    ocfg, params, lora, lm, trainer, batch, targets = _setup(TINY, target, torch.float32, dev)
    hist, _, final = ostep.train_steps(params, lora, ocfg, batch, OBJ[1], block_size=TINY["block"],
                                       mask_token_id=ocfg.vocab_size - 1, seed=20260813, steps=10, lr=1e-4)
    gb = {k: v.to(dev) for k, v in batch.items()}
    losses = [trainer.train_step(gb).item() for _ in range(10)]
    torch.cuda.synchronize()
    for a, b in zip(losses, hist):
        assert abs(a - b) / abs(b) < 1e-4, (losses, hist)
    mine = {n.replace("base_model.model.", "", 1): p.detach().cpu() for n, p in lm.lora_tensors().items()}
    worst = max(((mine[k] - v).norm() / v.norm()).item() for k, v in final.items())
    print(f"   worst LoRA weight rel L2 after 10 steps: {worst:.2e}", flush=True)
    assert worst < 1e-3
    st = lm.state
    untargeted = [n for n in ("q_proj", "k_proj", "v_proj", "o_proj", "gate_proj", "up_proj", "down_proj")
                  if n not in targets]
    for li in range(ocfg.num_hidden_layers):
        for name in untargeted:
            assert torch.count_nonzero(st.a_view(st.master, li, name)).item() == 0
            assert torch.count_nonzero(st.b_view(st.master, li, name)).item() == 0


@pytest.mark.parametrize("target", ["qv", "qkvo", "k_proj,up_proj"])
def test_subset_step_bf16(dev, target):
    """bf16 at a width that takes the fused 256x256 and SwiGLU kernels: against the fp32 oracle with
    the bars of the other bf16 step tests (cosine >= 0.999; rel L2 within 1e-2 or 1.3x the reference's
    own bf16 arithmetic), and equal to the all-projection step whose untargeted adapters are zero
    (the skipped LoRA products would add exact zeros)."""
    print(f"[lora targets] bf16 step, target={target!r}", flush=True)
    ocfg, params, lora, lm, trainer, batch, targets = _setup(WIDE, target, torch.bfloat16, dev)
    kw = dict(block_size=WIDE["block"], mask_token_id=ocfg.vocab_size - 1, seed=20260813, step=0)
    leaves = {k: v.clone().requires_grad_(True) for k, v in lora.items()}
    ref_loss, _ = ostep.compute_loss(params, leaves, ocfg, batch, OBJ[1], **kw)
    ref_loss.backward()
    leaves16 = {k: v.clone().requires_grad_(True) for k, v in lora.items()}
    loss16, _ = ostep.compute_loss({k: v.bfloat16() for k, v in params.items()}, leaves16, ocfg, batch, OBJ[1], **kw)
    loss16.backward()
    gb = {k: v.to(dev) for k, v in batch.items()}
    loss = trainer.compute_loss(lm, gb)
    loss.backward()
    torch.cuda.synchronize()
    lrel = abs(loss.item() - ref_loss.item()) / abs(ref_loss.item())
    mine = {k: v.float().cpu() for k, v in _grads(lm).items()}
    worst = 0.0
    for k, v in leaves.items():
        cos = torch.nn.functional.cosine_similarity(mine[k].flatten(), v.grad.flatten(), dim=0).item()
        r = ((mine[k] - v.grad).norm() / v.grad.norm()).item()
        r16 = ((leaves16[k].grad - v.grad).norm() / v.grad.norm()).item()
        worst = max(worst, r)
        assert cos >= 0.999, (k, cos)
        assert r <= max(1e-2, 1.3 * r16), (k, r, r16)
    print(f"   loss rel {lrel:.2e}, worst LoRA gradient rel L2 {worst:.3e}", flush=True)
    assert lrel < 1e-3

    # the same step on every projection, untargeted adapters zero
    full_cfg = UnoQwen3Config(vocab_size=ocfg.vocab_size, hidden_size=ocfg.hidden_size,
                              intermediate_size=ocfg.intermediate_size, num_hidden_layers=ocfg.num_hidden_layers,
                              num_attention_heads=ocfg.num_attention_heads,
                              num_key_value_heads=ocfg.num_key_value_heads, head_dim=ocfg.head_dim,
                              block_size=WIDE["block"])
    model = UnoQwen3ForCausalLM(full_cfg, device=dev, dtype=torch.bfloat16)
    model.load_weights(params)
    lm_all, _ = create_lora_model(model, LoraSettings("all", WIDE["rank"], WIDE["alpha"], 0.0))
    zeros = {n.replace("base_model.model.", "", 1): torch.zeros_like(p).cpu() for n, p in lm_all.lora_tensors().items()}
    zeros.update(lora)
    lm_all.load_lora(zeros)
    trainer_all = UnoTrainer(model=lm_all, objective=OBJ[0],
                             curriculum=BlockCurriculumPlan.fixed(WIDE["block"], 1000, WIDE["L"], WIDE["B"]),
                             args=UnoTrainingArguments(learning_rate=1e-4))
    loss_all = trainer_all.compute_loss(lm_all, gb)
    loss_all.backward()
    torch.cuda.synchronize()
    assert loss_all.item() == loss.item()
    got = _grads(lm_all)
    for k in lora:
        assert torch.equal(got[k].cpu().float(), mine[k]), k
