"""How close to the fp32 step can any bf16 step get? (CPU, the oracle only.)

A bf16 training step stores its activations in bf16. This test runs the oracle step in fp32 twice:
exactly, and with every stored activation of the forward (x1, qkv, q/k after RoPE, the attention
output, residual stream, x2, gate/up, SwiGLU output, final norm, LoRA weights and inner product)
rounded to bf16 while its gradient passes through unrounded, and compares the LoRA gradients. That
error is a floor for every bf16 implementation: it leaves out the rounding of gradients and of every
intermediate inside an op. At these reduced widths it is about 0.8e-2 at Qwen3-like proportions
(alpha/r = 2) and about 2.1e-2 with the 7B configuration's alpha = 16 r. The same measurement at
the real widths runs with the full-width GPU parity tests (tests/test_fullsize_configs_gpu.py),
which hold the Qwen3-8B and 1B steps to the literal 1e-2 and the 7B step, whose floor is above it,
to the reference's own bf16 arithmetic. A second run also rounds the gradients at the same points:
the floor is what bf16 storage costs, not a bound on the error gradient rounding adds.
"""
import pytest
import torch

from oracle import step as ostep
from oracle.model import Cfg, init_lora, init_params

STORED = {"x1", "qkv", "qk", "o", "resid", "x2", "gu", "sw", "final", "lora_w", "lora_h"}


def _stored_only(x, point):
    """bf16 forward value at a stored point; the gradient passes through unrounded."""
    return x + (x.bfloat16().float() - x).detach() if point in STORED else x


def _stored_and_grad(x, point):
    """bf16 at a stored point in both directions (the cast's backward rounds the gradient)."""
    return x.bfloat16().float() if point in STORED else x


def _grad_errors(spec):
    torch.set_num_threads(min(8, torch.get_num_threads()))
    cfg = Cfg(spec["V"], spec["H"], spec["F"], 1, spec["nq"], spec["nk"], 128, qk_norm=spec["qkn"],
              lora_rank=64, lora_alpha=spec["alpha"])
    params = {k: v.bfloat16().float() for k, v in init_params(cfg, seed=0).items()}
    lora = init_lora(cfg, seed=1)
    g = torch.Generator().manual_seed(2)
    ids = torch.randint(0, cfg.vocab_size - 1, (1, spec["L"]), generator=g)
    labels = ids.clone()
    labels[:, :spec["L"] // 8] = -100
    batch = {"input_ids": ids, "labels": labels}
    grads = []
    for rnd in (None, _stored_only, _stored_and_grad):
        leaves = {k: v.clone().requires_grad_(True) for k, v in lora.items()}
        loss, _ = ostep.compute_loss(params, leaves, cfg, batch, ostep.Objective(1, 0, 0, "data"), block_size=16,
                                     mask_token_id=cfg.vocab_size - 1, seed=20260813, step=0, rnd=rnd)
        loss.backward()
        grads.append({k: v.grad for k, v in leaves.items()})
    exact = grads[0]
    return [max(((gr[k] - v).norm() / v.norm()).item() for k, v in exact.items()) for gr in grads[1:]]


@pytest.mark.parametrize("name,spec,lo,hi", [
    ("qwen3-like: GQA 4:1, q/k-norm, alpha 2r",
     dict(V=8000, H=1024, F=3072, nq=8, nk=2, qkn=True, alpha=128, L=1024), 0.5e-2, 1e-2),
    ("7B-like: MHA, no q/k-norm, alpha 16r",
     dict(V=8000, H=1024, F=2816, nq=8, nk=8, qkn=False, alpha=1024, L=1024), 1.2e-2, 3e-2),
])
def test_bf16_activation_floor(name, spec, lo, hi):
    floor, with_grads = _grad_errors(spec)
    print(f"[bf16 floor] {name}: worst LoRA-gradient rel L2 from bf16 activation storage {floor:.3e}; "
          f"with the gradients rounded at the same points {with_grads:.3e}")
    assert lo < floor < hi
    assert with_grads > floor
