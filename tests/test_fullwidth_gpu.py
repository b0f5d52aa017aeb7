"""Step parity at the full Qwen3-8B widths (hidden 4096, 32 q / 8 kv heads of 128, FFN 12288,
vocab 151936, LoRA r=64 / alpha=128 on all seven projections, block 16) on one 4096-token
sequence with one decoder layer: the widths, tile paths and LM head of the benchmarked step.

The GPU step (bf16 weights, adapters and activations) is compared with the fp32 oracle on the
same bf16-rounded weights; the yardstick for the LoRA gradients is the reference's own bf16
arithmetic (the oracle run with bf16 weights, adapters and activations) on the same inputs, as in
the reduced-width step tests: loss within 1e-3 relative, gradient cosine >= 0.999, relative L2
error no more than 1.1x the bf16 reference's over all tensors (RMS) and 1.3x per tensor (or 1e-2)."""
import pytest
import torch
import torch.nn.functional as F

from oracle import step as ostep
from oracle.model import Cfg, init_lora, init_params
from uno_amd.model import UnoQwen3Config, UnoQwen3ForCausalLM
from uno_amd.training.config import LoraSettings, UnoObjectiveConfig
from uno_amd.training.curriculum import BlockCurriculumPlan
from uno_amd.training.lora import create_lora_model
from uno_amd.training.trainer import UnoTrainer, UnoTrainingArguments

pytestmark = pytest.mark.gpu

L, PROMPT, BLOCK, RANK, ALPHA = 4096, 512, 16, 64, 128


def _errors(grads, ref):
    return {k: (F.cosine_similarity(grads[k].float().cpu().flatten(), v.flatten(), dim=0).item(),
                ((grads[k].float().cpu() - v).norm() / v.norm()).item()) for k, v in ref.items()}


def test_step_bf16_qwen3_8b_widths_one_layer(dev):
    torch.set_num_threads(min(16, torch.get_num_threads()))
    cfg = Cfg(151936, 4096, 12288, 1, 32, 8, 128, lora_rank=RANK, lora_alpha=ALPHA)
    params = {k: v.bfloat16().float() for k, v in init_params(cfg, seed=0).items()}
    lora = init_lora(cfg, seed=1)
    g = torch.Generator().manual_seed(2)
    ids = torch.randint(0, cfg.vocab_size - 1, (1, L), generator=g)
    labels = ids.clone()
    labels[:, :PROMPT] = -100
    batch = {"input_ids": ids, "labels": labels, "attention_mask": torch.ones_like(ids)}
    kw = dict(block_size=BLOCK, mask_token_id=cfg.vocab_size - 1, seed=20260813, step=0)
    obj = ostep.Objective(1, 0, 0, "data")

    print("[full width] GPU step", flush=True)
    ucfg = UnoQwen3Config(vocab_size=cfg.vocab_size, hidden_size=cfg.hidden_size,
                          intermediate_size=cfg.intermediate_size, num_hidden_layers=1,
                          num_attention_heads=cfg.num_attention_heads, num_key_value_heads=cfg.num_key_value_heads,
                          head_dim=cfg.head_dim, block_size=BLOCK)
    model = UnoQwen3ForCausalLM(ucfg, device=dev, dtype=torch.bfloat16)
    model.load_weights(params)
    lm, _ = create_lora_model(model, LoraSettings("all", RANK, ALPHA, 0.0))
    lm.load_lora(lora)
    trainer = UnoTrainer(model=lm, objective=UnoObjectiveConfig(ce_target="ground_truth", ce_weight=1.0,
                                                                kl_weight=0.0, tv_weight=0.0),
                         curriculum=BlockCurriculumPlan.fixed(BLOCK, 10, L, 1),
                         args=UnoTrainingArguments(learning_rate=1e-4))
    loss = trainer.compute_loss(lm, {k: v.to(dev) for k, v in batch.items()})
    loss.backward()
    torch.cuda.synchronize()
    mine_grads = {n.replace("base_model.model.", "", 1): p.grad.float().cpu() for n, p in lm.lora_tensors().items()}
    mine_loss = loss.item()
    del trainer, lm, model, loss
    torch.cuda.empty_cache()

    print("[full width] fp32 oracle", flush=True)
    leaves = {k: v.clone().requires_grad_(True) for k, v in lora.items()}
    ref_loss, _ = ostep.compute_loss(params, leaves, cfg, batch, obj, **kw)
    ref_loss.backward()
    ref = {k: v.grad for k, v in leaves.items()}
    print("[full width] bf16 oracle", flush=True)
    leaves16 = {k: v.clone().requires_grad_(True) for k, v in lora.items()}
    loss16, _ = ostep.compute_loss({k: v.bfloat16() for k, v in params.items()}, leaves16, cfg, batch, obj, **kw)
    loss16.backward()

    lrel = abs(mine_loss - ref_loss.item()) / abs(ref_loss.item())
    mine = _errors(mine_grads, ref)
    theirs = _errors({k: v.grad for k, v in leaves16.items()}, ref)
    rms = lambda d: (sum(r * r for _, r in d.values()) / len(d)) ** 0.5
    worst = sorted(mine, key=lambda k: -mine[k][1])[:4]
    for k in worst:
        print(f"   {k:50s} mine cos {mine[k][0]:.5f} rel {mine[k][1]:.3e} | bf16-ref rel {theirs[k][1]:.3e}")
    print(f"[full width] loss {mine_loss:.6f} vs {ref_loss.item():.6f} (rel {lrel:.2e}, bf16 reference "
          f"{abs(loss16.item() - ref_loss.item()) / abs(ref_loss.item()):.2e}); grad rel L2 RMS {rms(mine):.3e} "
          f"(bf16 reference {rms(theirs):.3e})", flush=True)
    assert lrel < 1e-3
    assert min(c for c, _ in mine.values()) >= 0.999
    assert rms(mine) <= max(1e-2, 1.1 * rms(theirs))
    for k, (c, r) in mine.items():
        assert r <= max(1e-2, 1.3 * theirs[k][1]), (k, r, theirs[k][1])
