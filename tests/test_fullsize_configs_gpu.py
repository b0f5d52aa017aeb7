"""Step parity at the real widths and row counts of every benchmarked configuration, one decoder
layer each, against the fp32 oracle on the same bf16-rounded weights:

* qwen3_8b  hidden 4096, 32 q / 8 kv heads of 128, FFN 12288, vocab 151936, q/k-norm, r 64 / alpha 128,
            block 16, one 4096-token row;
* dense_1b  hidden 2048, 16 q / 8 kv heads of 128, FFN 5632, vocab 151936, r 32 / alpha 64, block 8,
            four 2048-token rows (8192 rows per stream, so every product of the layer takes the
            kernels the full 8 x 2048 batch takes: the 256 x 256 MFMA GEMM, the fused SwiGLU forward,
            the skinny LoRA products);
* qwen3_8b_r128  the Qwen3-8B widths with the released recipe's adapter, r 128 / alpha 2048 (16 r):
            the 3r = 384- and 2r = 256-wide LoRA products and weight gradients;
* mha_7b    hidden 4096, 32 q = 32 kv heads, no q/k-norm, FFN 11008, vocab 32000, r 64 / alpha 1024
            (16 r), one 4096-token row, at block 16 and at every block size of the 4 -> 32 curriculum.

The GPU step keeps bf16 weights, adapters and activations. Bars: loss within
1e-3 relative, LoRA gradient cosine >= 0.999 and relative L2 error <= 1e-2 per tensor against the
fp32 oracle. The configurations with alpha = 16 r (7B MHA, rank 128) are held to max(1e-2, 1.3 x
the reference's own bf16 arithmetic on the same inputs) instead: there the error that bf16 storage
of the forward activations alone causes (no gradient rounding, every op in fp32) is above 1e-2 at
these widths (asserted), so no bf16 step can meet the literal bar. The per-tensor errors are printed with the reference's.
"""
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

SEED = 20260813
CONFIGS = {
    "qwen3_8b": dict(cfg=dict(vocab_size=151936, hidden_size=4096, intermediate_size=12288, num_attention_heads=32,
                              num_key_value_heads=8, head_dim=128, qk_norm=True),
                     rank=64, alpha=128, B=1, L=4096, prompt=512, blocks=[16], literal=True),
    "dense_1b": dict(cfg=dict(vocab_size=151936, hidden_size=2048, intermediate_size=5632, num_attention_heads=16,
                              num_key_value_heads=8, head_dim=128, qk_norm=True),
                     rank=32, alpha=64, B=4, L=2048, prompt=256, blocks=[8], literal=True),
    "qwen3_8b_r128": dict(cfg=dict(vocab_size=151936, hidden_size=4096, intermediate_size=12288,
                                   num_attention_heads=32, num_key_value_heads=8, head_dim=128, qk_norm=True),
                          rank=128, alpha=2048, B=1, L=4096, prompt=512, blocks=[16]),
    "mha_7b": dict(cfg=dict(vocab_size=32000, hidden_size=4096, intermediate_size=11008, num_attention_heads=32,
                            num_key_value_heads=32, head_dim=128, qk_norm=False),
                   rank=64, alpha=1024, B=1, L=4096, prompt=512, blocks=[16]),
    "mha_7b_curriculum": dict(cfg=dict(vocab_size=32000, hidden_size=4096, intermediate_size=11008,
                                       num_attention_heads=32, num_key_value_heads=32, head_dim=128, qk_norm=False),
                              rank=64, alpha=1024, B=1, L=4096, prompt=512, blocks=[4, 8, 32]),
}


STORED = {"x1", "qkv", "qk", "o", "resid", "x2", "gu", "sw", "final", "lora_w", "lora_h"}


def _stored_bf16(x, point):
    """Rounds the forward value stored at a named oracle point to bf16 and passes the gradient through
    unrounded: the error of bf16 activation storage alone, with every op and gradient in fp32."""
    return x + (x.bfloat16().float() - x).detach() if point in STORED else x


def _errors(grads, ref):
    return {k: (F.cosine_similarity(grads[k].float().flatten(), v.flatten(), dim=0).item(),
                ((grads[k].float() - v).norm() / v.norm()).item()) for k, v in ref.items()}


@pytest.mark.parametrize("name", list(CONFIGS))
def test_bf16_step_full_width(dev, name):
    spec = CONFIGS[name]
    torch.set_num_threads(min(16, torch.get_num_threads()))
    c = spec["cfg"]
    cfg = Cfg(c["vocab_size"], c["hidden_size"], c["intermediate_size"], 1, c["num_attention_heads"],
              c["num_key_value_heads"], c["head_dim"], qk_norm=c["qk_norm"], lora_rank=spec["rank"],
              lora_alpha=spec["alpha"])
    params = {k: v.bfloat16().float() for k, v in init_params(cfg, seed=0).items()}
    lora = init_lora(cfg, seed=1)
    g = torch.Generator().manual_seed(2)
    B, L = spec["B"], spec["L"]
    ids = torch.randint(0, cfg.vocab_size - 1, (B, L), generator=g)
    labels = ids.clone()
    labels[:, :spec["prompt"]] = -100
    batch = {"input_ids": ids, "labels": labels, "attention_mask": torch.ones_like(ids)}
    obj = ostep.Objective(1, 0, 0, "data")

    ucfg = UnoQwen3Config(num_hidden_layers=1, block_size=spec["blocks"][0], **c)
    model = UnoQwen3ForCausalLM(ucfg, device=dev, dtype=torch.bfloat16)
    model.load_weights(params)
    lm, _ = create_lora_model(model, LoraSettings("all", spec["rank"], spec["alpha"], 0.0))
    lm.load_lora(lora)
    blocks = spec["blocks"]
    tps = B * L
    plan = BlockCurriculumPlan.from_dict({"tokens_per_step": tps, "sequence_length": L, "global_batch_size": B,
                                          "seed": 0, "stages": [{"block_size": b, "tokens": tps} for b in blocks]})
    trainer = UnoTrainer(model=lm, objective=UnoObjectiveConfig(ce_target="ground_truth", ce_weight=1.0,
                                                                kl_weight=0.0, tv_weight=0.0),
                         curriculum=plan, args=UnoTrainingArguments(learning_rate=1e-4))
    gb = {k: v.to(dev) for k, v in batch.items()}
    for step, block in enumerate(blocks):
        print(f"[full size] {name}: GPU step at block {block}", flush=True)
        trainer.state.global_step = step            # the curriculum picks this step's block size
        lm.get_base_model()._bd_step = 0            # the same noise draw as the oracle's step 0
        for p in lm.parameters():
            p.grad = None
        loss = trainer.compute_loss(lm, gb)
        assert lm.get_base_model().config.block_size == block
        loss.backward()
        torch.cuda.synchronize()
        mine = {n.replace("base_model.model.", "", 1): p.grad.float().cpu() for n, p in lm.lora_tensors().items()}
        mine_loss = loss.item()
        del loss

        print(f"[full size] {name}: fp32 oracle", flush=True)
        kw = dict(block_size=block, mask_token_id=cfg.vocab_size - 1, seed=SEED, step=0)
        leaves = {k: v.clone().requires_grad_(True) for k, v in lora.items()}
        ref_loss, _ = ostep.compute_loss(params, leaves, cfg, batch, obj, **kw)
        ref_loss.backward()
        ref = {k: v.grad for k, v in leaves.items()}
        print(f"[full size] {name}: bf16 oracle", flush=True)
        leaves16 = {k: v.clone().requires_grad_(True) for k, v in lora.items()}
        loss16, _ = ostep.compute_loss({k: v.bfloat16() for k, v in params.items()}, leaves16, cfg, batch, obj, **kw)
        loss16.backward()

        floor = None
        if step == 0:
            print(f"[full size] {name}: fp32 oracle with bf16-stored activations", flush=True)
            leaves_f = {k: v.clone().requires_grad_(True) for k, v in lora.items()}
            loss_f, _ = ostep.compute_loss(params, leaves_f, cfg, batch, obj, rnd=_stored_bf16, **kw)
            loss_f.backward()
            floor = _errors({k: v.grad for k, v in leaves_f.items()}, ref)

        lrel = abs(mine_loss - ref_loss.item()) / abs(ref_loss.item())
        err = _errors(mine, ref)
        theirs = _errors({k: v.grad for k, v in leaves16.items()}, ref)
        rms = lambda d: (sum(r * r for _, r in d.values()) / len(d)) ** 0.5
        print(f"[full size] {name} block {block}: loss rel {lrel:.2e}; rel L2 per tensor (mine | bf16 reference):",
              flush=True)
        for k in sorted(err, key=lambda k: -err[k][1]):
            print(f"   {k:50s} cos {err[k][0]:.6f} rel {err[k][1]:.3e} | {theirs[k][1]:.3e}", flush=True)
        print(f"[full size] {name} block {block}: worst rel L2 {max(r for _, r in err.values()):.3e}, RMS "
              f"{rms(err):.3e} (bf16 reference {max(r for _, r in theirs.values()):.3e}, RMS {rms(theirs):.3e})",
              flush=True)
        if floor is not None:
            worst_floor = max(r for _, r in floor.values())
            print(f"[full size] {name}: bf16 activation storage alone: worst rel L2 {worst_floor:.3e}, RMS "
                  f"{rms(floor):.3e}", flush=True)
            # the relative bar is kept only where that floor itself is above the literal one
            assert spec.get("literal") or worst_floor > 1e-2
        assert lrel < 1e-3
        assert min(cc for cc, _ in err.values()) >= 0.999
        for k, (_, r) in err.items():
            bar = 1e-2 if spec.get("literal") else max(1e-2, 1.3 * theirs[k][1])
            assert r <= bar, (k, r, theirs[k][1])
