"""End-to-end parity of the Uno step (compute_loss -> backward -> clip -> AdamW) with the oracle.

fp32 mode: loss and LoRA gradients tight; LoRA weights after 10 optimizer steps within 1e-3
relative (per-tensor L2). bf16 mode (weights rounded to bf16 on both sides): loss within 1e-3
relative, LoRA gradients with cosine >= 0.999 and per-tensor relative L2 <= 1e-2 of the fp32
oracle or, where bf16 rounding alone exceeds that, no worse than the reference's own bf16
arithmetic (the oracle run with bf16 weights, adapters and activations) on the same inputs."""
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

TINY = dict(vocab_size=4096, hidden_size=256, intermediate_size=768, num_hidden_layers=2, num_attention_heads=4,
            num_key_value_heads=2, head_dim=64, rank=8, alpha=16, B=2, L=256, prompt=64, block=4)
MID = dict(vocab_size=8192, hidden_size=512, intermediate_size=1024, num_hidden_layers=2, num_attention_heads=4,
           num_key_value_heads=2, head_dim=128, rank=16, alpha=32, B=2, L=512, prompt=64, block=16)

OBJECTIVES = {
    "ce_data": (UnoObjectiveConfig(ce_target="ground_truth", ce_weight=1.0, kl_weight=0.0, tv_weight=0.0),
                ostep.Objective(1, 0, 0, "data")),
    "tv": (UnoObjectiveConfig(ce_weight=0.0, kl_weight=0.0, tv_weight=1.0), ostep.Objective(0, 0, 1)),
    "kl": (UnoObjectiveConfig(ce_weight=0.0, kl_weight=1.0, tv_weight=0.0), ostep.Objective(0, 1, 0)),
    "ce_teacher_mix": (UnoObjectiveConfig(ce_target="teacher", ce_weight=0.5, kl_weight=0.0, tv_weight=1.0),
                       ostep.Objective(0.5, 0, 1, "clean_argmax")),
}


def _setup(spec, dtype, dev, objective, seed=0):
    ocfg = Cfg(spec["vocab_size"], spec["hidden_size"], spec["intermediate_size"], spec["num_hidden_layers"],
               spec["num_attention_heads"], spec["num_key_value_heads"], spec["head_dim"],
               lora_rank=spec["rank"], lora_alpha=spec["alpha"])
    params = init_params(ocfg, seed=seed)
    if dtype == torch.bfloat16:
        params = {k: v.bfloat16().float() for k, v in params.items()}
    lora = init_lora(ocfg, seed=seed + 1)
    ucfg = UnoQwen3Config(vocab_size=ocfg.vocab_size, hidden_size=ocfg.hidden_size,
                          intermediate_size=ocfg.intermediate_size, num_hidden_layers=ocfg.num_hidden_layers,
                          num_attention_heads=ocfg.num_attention_heads, num_key_value_heads=ocfg.num_key_value_heads,
                          head_dim=ocfg.head_dim, block_size=spec["block"])
    model = UnoQwen3ForCausalLM(ucfg, device=dev, dtype=dtype)
    model.load_weights(params)
    lm, _ = create_lora_model(model, LoraSettings("all", spec["rank"], spec["alpha"], 0.0))
    lm.load_lora(lora)
    trainer = UnoTrainer(model=lm, objective=objective,
                         curriculum=BlockCurriculumPlan.fixed(spec["block"], 1000, spec["L"], spec["B"]),
                         args=UnoTrainingArguments(learning_rate=1e-4))
    g = torch.Generator().manual_seed(seed + 2)
    ids = torch.randint(0, ocfg.vocab_size - 1, (spec["B"], spec["L"]), generator=g)
    labels = ids.clone()
    labels[:, :spec["prompt"]] = -100
    batch = {"input_ids": ids, "labels": labels, "attention_mask": torch.ones_like(ids)}
    return ocfg, params, lora, model, lm, trainer, batch


def _to(batch, dev):
    return {k: v.to(dev) for k, v in batch.items()}


def _my_grads(lm):
    return {n.replace("base_model.model.", "", 1): p.grad for n, p in lm.lora_tensors().items()}


@pytest.mark.parametrize("obj", list(OBJECTIVES))
def test_step_fp32_loss_and_grads(dev, obj):
    mine_obj, ref_obj = OBJECTIVES[obj]
    ocfg, params, lora, model, lm, trainer, batch = _setup(TINY, torch.float32, dev, mine_obj)
    print(f"[step fp32] objective={obj}", flush=True)
    leaves = {k: v.clone().requires_grad_(True) for k, v in lora.items()}
    ref_loss, _ = ostep.compute_loss(params, leaves, ocfg, batch, ref_obj, block_size=TINY["block"],
                                     mask_token_id=ocfg.vocab_size - 1, seed=20260813, step=0)
    ref_loss.backward()
    loss = trainer.compute_loss(lm, _to(batch, dev))
    loss.backward()
    torch.cuda.synchronize()
    assert abs(loss.item() - ref_loss.item()) / abs(ref_loss.item()) < 1e-5, (loss.item(), ref_loss.item())
    mine = _my_grads(lm)
    # TV's gradient has sign(p - q): entries where p and q agree to rounding can flip sign
    # between two correct fp32 implementations, so its bound is looser.
    tol = 2e-3 if obj == "tv" else 2e-4
    for k, v in leaves.items():
        r = ((mine[k].cpu() - v.grad).norm() / v.grad.norm().clamp_min(1e-30)).item()
        assert r < tol, (k, r)


def test_ten_adamw_steps_fp32(dev):
    mine_obj, ref_obj = OBJECTIVES["ce_data"]
    ocfg, params, lora, model, lm, trainer, batch = _setup(TINY, torch.float32, dev, mine_obj)
    hist, _, final = ostep.train_steps(params, lora, ocfg, batch, ref_obj, block_size=TINY["block"],
                                       mask_token_id=ocfg.vocab_size - 1, seed=20260813, steps=10, lr=1e-4)
    gb = _to(batch, dev)
    losses = [trainer.train_step(gb).item() for _ in range(10)]
    torch.cuda.synchronize()
    for a, b in zip(losses, hist):
        assert abs(a - b) / abs(b) < 1e-4, (losses, hist)
    mine = {n.replace("base_model.model.", "", 1): p.detach().cpu() for n, p in lm.lora_tensors().items()}
    worst_w, worst_u = 0.0, 0.0
    for k, v in final.items():
        worst_w = max(worst_w, ((mine[k] - v).norm() / v.norm()).item())
        upd_ref = v - lora[k]
        worst_u = max(worst_u, ((mine[k] - lora[k] - upd_ref).norm() / upd_ref.norm()).item())
    print(f"[10 steps fp32] worst weight rel err {worst_w:.3e}, worst update rel err {worst_u:.3e}")
    assert worst_w < 1e-3
    assert worst_u < 5e-2


def _grad_errors(grads, ref):
    out = {}
    for k, v in ref.items():
        a = grads[k].float().cpu()
        out[k] = (F.cosine_similarity(a.flatten(), v.flatten(), dim=0).item(), ((a - v).norm() / v.norm()).item())
    return out


@pytest.mark.parametrize("spec_name", ["TINY", "MID"])
@pytest.mark.parametrize("obj", ["ce_data", "tv"])
def test_step_bf16_tolerances(dev, spec_name, obj):
    spec = TINY if spec_name == "TINY" else MID
    mine_obj, ref_obj = OBJECTIVES[obj]
    ocfg, params, lora, model, lm, trainer, batch = _setup(spec, torch.bfloat16, dev, mine_obj)
    print(f"[step bf16] spec={spec_name} objective={obj}", flush=True)
    kw = dict(block_size=spec["block"], mask_token_id=ocfg.vocab_size - 1, seed=20260813, step=0)
    leaves = {k: v.clone().requires_grad_(True) for k, v in lora.items()}
    ref_loss, _ = ostep.compute_loss(params, leaves, ocfg, batch, ref_obj, **kw)
    ref_loss.backward()
    ref = {k: v.grad for k, v in leaves.items()}
    # the reference's own arithmetic: bf16 weights, adapters and activations
    leaves16 = {k: v.clone().requires_grad_(True) for k, v in lora.items()}
    loss16, _ = ostep.compute_loss({k: v.bfloat16() for k, v in params.items()}, leaves16, ocfg, batch, ref_obj, **kw)
    loss16.backward()
    loss = trainer.compute_loss(lm, _to(batch, dev))
    loss.backward()
    torch.cuda.synchronize()
    lrel = abs(loss.item() - ref_loss.item()) / abs(ref_loss.item())
    lrel16 = abs(loss16.item() - ref_loss.item()) / abs(ref_loss.item())
    mine = _grad_errors(_my_grads(lm), ref)
    theirs = _grad_errors({k: v.grad for k, v in leaves16.items()}, ref)
    worst = sorted(mine, key=lambda k: -mine[k][1])[:6]
    for k in worst:
        print(f"   {k:60s} mine cos {mine[k][0]:.5f} rel {mine[k][1]:.3e} | bf16-ref cos {theirs[k][0]:.5f} "
              f"rel {theirs[k][1]:.3e}")
    worst_cos = min(c for c, _ in mine.values())
    worst_rel = max(r for _, r in mine.values())
    ref_rel = max(r for _, r in theirs.values())
    print(f"[step bf16] loss rel {lrel:.2e} (bf16 reference arithmetic {lrel16:.2e}); worst grad cos "
          f"{worst_cos:.5f}; worst grad rel L2 {worst_rel:.3e} (bf16 reference arithmetic {ref_rel:.3e})")
    assert lrel < 1e-3
    assert worst_cos >= 0.999
    # Within 1e-2 of fp32, or no further from fp32 than the reference's own bf16 arithmetic is
    # (bf16 rounding alone puts that at 1.5-4e-2 at these shapes): 1.1x over the RMS of all
    # tensors, 1.3x per tensor (per-tensor errors of two differently rounded bf16 computations
    # scatter by +-15%; a real fault on one tensor costs far more).
    rms = lambda d: (sum(r * r for _, r in d.values()) / len(d)) ** 0.5
    print(f"[step bf16] rel L2 RMS over tensors {rms(mine):.3e} (bf16 reference arithmetic {rms(theirs):.3e})")
    assert rms(mine) <= max(1e-2, 1.1 * rms(theirs))
    for k, (c, r) in mine.items():
        assert r <= max(1e-2, 1.3 * theirs[k][1]), (k, r, theirs[k][1])


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_clean_tail_skipped_only_when_no_teacher(dev, dtype):
    """A CE step on data targets skips the clean stream's last-layer output (only that layer's K/V
    feed the noisy stream): loss and LoRA gradients are bit-identical to the step that computes it,
    the decoder's setting is restored afterwards, and a TV step keeps computing it."""
    obj, _ = OBJECTIVES["ce_data"]
    _, _, _, model, lm, trainer, batch = _setup(MID, dtype, dev, obj)
    decoder = model.model
    assert trainer._needs_teacher() is False

    seen = []
    full = decoder.forward

    def spy(*a, **k):
        seen.append(decoder.clean_final_needed)
        return full(*a, **k)

    decoder.forward = spy
    results = {}
    draws = model._bd_step          # both steps draw the same noise
    for forced in (None, True):
        if forced:
            trainer._needs_teacher = lambda: True
        model._bd_step = draws
        lm.zero_grad(set_to_none=True)
        loss = trainer.compute_loss(lm, _to(batch, dev))
        loss.backward()
        torch.cuda.synchronize()
        results[forced] = (loss.detach().clone(), {k: v.detach().clone() for k, v in _my_grads(lm).items()})
        assert decoder.clean_final_needed is True
    assert seen == [False, True]
    (l0, g0), (l1, g1) = results[None], results[True]
    assert torch.equal(l0, l1)
    for k in g0:
        assert torch.equal(g0[k], g1[k]), k

    del trainer._needs_teacher
    trainer.objective = OBJECTIVES["tv"][0]
    assert trainer._needs_teacher() is True
    seen.clear()
    trainer.compute_loss(lm, _to(batch, dev))
    assert seen == [True]
    decoder.forward = full
