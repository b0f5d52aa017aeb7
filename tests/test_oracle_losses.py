"""Pins the oracle objectives: closed forms, the reference's chunked TV algorithm, KL via
torch's kl_div, CE weighting by hand, and the full-step wiring by finite differences."""
import math

import pytest
import torch
import torch.nn.functional as F

from oracle import losses, step
from oracle.model import Cfg, init_lora, init_params


def test_project_hidden_states_union_reselection():
    torch.manual_seed(0)
    W = torch.randn(11, 5)
    h = torch.randn(2, 4, 5)
    m1 = torch.tensor([[1, 0, 1, 0], [0, 0, 1, 1]], dtype=torch.bool)
    m2 = torch.tensor([[0, 0, 1, 1], [1, 0, 0, 1]], dtype=torch.bool)
    out = losses.project_hidden_states(W, h, {"a": m1, "b": m2})
    assert torch.allclose(out["a"], h[m1] @ W.T) and torch.allclose(out["b"], h[m2] @ W.T)
    empty = losses.project_hidden_states(W, h, {"a": torch.zeros_like(m1)})
    assert empty["a"].shape == (0, 11)


def test_weighted_ce_hand_case():
    logits = torch.tensor([[0.0, math.log(3.0)], [math.log(2.0), 0.0]])
    targets = torch.tensor([1, 1])
    p = torch.tensor([0.5, 0.25])
    # CE row0 = -log(3/4), row1 = -log(1/3)
    expect = (-math.log(0.75) / 0.5 + -math.log(1 / 3) / 0.25) / 5
    assert abs(losses.weighted_ce(logits, targets, p, 5).item() - expect) < 1e-6
    with pytest.raises(RuntimeError):
        losses.weighted_ce(logits, targets, p[:1], 5)


def test_ce_targets_argmax_first_index_on_ties():
    t = torch.tensor([[1.0, 3.0, 3.0], [2.0, 2.0, 0.0]])
    out = losses.resolve_ce_targets("clean_argmax", None, None, t)
    assert out.tolist() == [1, 0]
    with pytest.raises(ValueError):
        losses.resolve_ce_targets("bogus", None, None, t)


def test_kl_matches_torch_kl_div():
    torch.manual_seed(1)
    s, t = torch.randn(7, 33), torch.randn(7, 33)
    ref = F.kl_div(F.log_softmax(t, -1), F.log_softmax(s, -1), log_target=True, reduction="sum") / 4
    assert abs(losses.reverse_kl(s, t, 4).item() - ref.item()) < 1e-5


@pytest.mark.parametrize("chunk", [5, 2048])
def test_tv_dense_equals_reference_chunked_algorithm(chunk):
    torch.manual_seed(2)
    s, t = torch.randn(6, 37), torch.randn(6, 37)
    t[2] = s[2]            # identical row: sign(0) = 0 everywhere -> zero gradient there
    sv = s.clone().requires_grad_(True)
    dense = losses.total_variation(sv, t, 3)
    dense.backward()
    val, grad = losses.chunked_tv_reference_algorithm(s, t, 3, chunk=chunk)
    assert abs(dense.item() - val.item()) < 1e-6
    assert torch.allclose(sv.grad, grad, atol=1e-7)
    assert grad[2].abs().max().item() == 0.0
    # closed form for two-way softmax: |p-q|_1 = 2|sigmoid(a)-sigmoid(b)|
    a, b = torch.tensor([[0.3, -0.2]]), torch.tensor([[1.0, 0.0]])
    expect = 2 * abs(torch.sigmoid(torch.tensor(0.5)) - torch.sigmoid(torch.tensor(1.0))).item()
    assert abs(losses.total_variation(a, b, 1).item() - expect) < 1e-6


TINY = Cfg(vocab_size=64, hidden_size=32, intermediate_size=48, num_hidden_layers=1,
           num_attention_heads=2, num_key_value_heads=1, head_dim=16, lora_rank=2, lora_alpha=4)


def _tiny_batch(L=16, prompt=4):
    g = torch.Generator().manual_seed(9)
    ids = torch.randint(0, 63, (1, L), generator=g)
    labels = ids.clone()
    labels[:, :prompt] = -100
    return {"input_ids": ids, "labels": labels}


@pytest.mark.parametrize("obj", [step.Objective(1, 0, 0), step.Objective(0, 0, 1), step.Objective(0, 1, 0),
                                 step.Objective(1, 0, 0, "clean_argmax")])
def test_full_step_gradient_finite_differences(obj):
    """fp64 central differences on a few LoRA entries pin the wiring of the whole step."""
    params = {k: v.double() for k, v in init_params(TINY, seed=0, std=0.2).items()}
    lora = {k: v.double().requires_grad_(True) for k, v in init_lora(TINY, seed=1, b_std=0.2).items()}
    batch = _tiny_batch()
    kw = dict(block_size=4, mask_token_id=63, seed=5, step=0)
    loss, _ = step.compute_loss(params, lora, TINY, batch, obj, **kw)
    loss.backward()
    g = torch.Generator().manual_seed(0)
    for name in list(lora)[:4]:
        t = lora[name]
        flat = t.detach().view(-1)
        for idx in torch.randint(0, flat.numel(), (3,), generator=g).tolist():
            eps = 1e-6
            orig = flat[idx].item()
            with torch.no_grad():
                flat[idx] = orig + eps
                lp, _ = step.compute_loss(params, lora, TINY, batch, obj, **kw)
                flat[idx] = orig - eps
                lm, _ = step.compute_loss(params, lora, TINY, batch, obj, **kw)
                flat[idx] = orig
            fd = (lp.item() - lm.item()) / (2 * eps)
            an = t.grad.view(-1)[idx].item()
            assert abs(fd - an) <= 1e-6 + 1e-4 * abs(fd), (name, idx, fd, an)


def test_first_adamw_step_closed_form():
    """Step 1 of AdamW: m_hat = g, v_hat = g^2 -> p1 = p0 - lr * g_c / (|g_c| + eps),
    with g_c = g * min(1, 1 / (||g|| + 1e-6)) (global-norm clip at 1.0)."""
    params = init_params(TINY, seed=0, std=0.2)
    lora = init_lora(TINY, seed=1, b_std=0.2)
    batch = _tiny_batch()
    _, grads, final = step.train_steps(params, lora, TINY, batch, step.Objective(1, 0, 0), block_size=4,
                                       mask_token_id=63, seed=5, steps=1, lr=1e-3)
    norm = math.sqrt(sum(float((g.double() ** 2).sum()) for g in grads.values()))
    coef = min(1.0, 1.0 / (norm + 1e-6))
    for k in lora:
        gc = grads[k].double() * coef
        expect = lora[k].double() - 1e-3 * gc / (gc.abs() + 1e-8)
        assert torch.allclose(final[k].double(), expect, atol=1e-7), k
