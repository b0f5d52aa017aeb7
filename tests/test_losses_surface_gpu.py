"""The logits-level call surface of training/losses.py on the GPU kernels.

* ``project_hidden_states`` (training/losses.py:21-35): the LM head over the union of the masks,
  re-selected per mask, against ``hidden[mask] @ W^T`` in fp32, forward and backward.
* ``resolve_ce_targets`` (training/losses.py:38-56): "data" targets are the shifted labels of the
  CE rows, bit-exact; "clean_argmax" is torch.argmax's first-index rule, bit-exact on logits built
  with ties (within a row chunk, across chunk boundaries, all-equal rows, -inf rows, NaN).
* ``teacher_argmax`` (the chunked LM-head argmax of the step) on an LM head with duplicated rows,
  whose logits tie exactly: the lower vocabulary index wins, as torch.argmax picks it.
"""
import pytest
import torch

from uno_amd import _native as N
from uno_amd import kernels as K
from uno_amd.objectives import logits_argmax, teacher_argmax
from uno_amd.training.losses import project_hidden_states, resolve_ce_targets, shift_labels_for_next_token

pytestmark = pytest.mark.gpu


class _Head(torch.nn.Module):
    def __init__(self, w):
        super().__init__()
        self.weight = w
        self.weight_t = w.t().contiguous()

    def forward(self, x):
        from uno_amd.objectives import lm_head_logits
        return lm_head_logits(self, x)


def _tied_logits(R, V, dtype, dev):
    g = torch.Generator(device=dev).manual_seed(3)
    z = torch.randn(R, V, device=dev, generator=g).to(dtype)
    top = z.float().max() + 1
    for r in range(R):
        kind = r % 6
        if kind == 0:      # tie inside one 256-column stride of a thread
            z[r, 10] = z[r, 266] = top
        elif kind == 1:    # tie across the chunk boundary used below
            z[r, 999] = z[r, 1000] = z[r, V - 1] = top
        elif kind == 2:    # every value equal
            z[r] = 0.5
        elif kind == 3:    # all -inf
            z[r] = float("-inf")
        elif kind == 4:    # a NaN beats every number; the first NaN wins
            z[r, 7] = top
            z[r, 4000] = float("nan")
            z[r, 4500] = float("nan")
        else:              # plain row
            pass
    return z


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("V", [5003, 8192])   # rows at odd offsets (mostly element-wise) / all 16-byte walks
def test_argmax_ties_bit_exact(dev, dtype, V):
    R = 60
    z = _tied_logits(R, V, dtype, dev)
    ref = torch.argmax(z.float().cpu(), dim=-1)
    assert torch.equal(logits_argmax(z).cpu(), ref)
    # the chunked merge of the step: chunks of 1000 columns, ties straddling chunk edges
    best_val = torch.empty(R, device=dev)
    best_idx = torch.empty(R, device=dev, dtype=torch.int64)
    for i, c0 in enumerate(range(0, V, 1000)):
        c1 = min(V, c0 + 1000)
        zc = z[:, c0:c1]
        N.call("unok_row_argmax_update", N.dtype_code(dtype), R, c1 - c0, N.ptr(zc), z.stride(0), c0,
               N.ptr(best_val), N.ptr(best_idx), int(i == 0), N.stream())
    assert torch.equal(best_idx.cpu(), ref)


def test_teacher_argmax_duplicated_head_rows(dev):
    """Rows j and j + V/2 of the LM head are equal, so their logits tie bit for bit; the lower
    index must win in every row, through the chunked GEMM + argmax path."""
    torch.manual_seed(8)
    R, H, V = 257, 256, 8192
    half = (torch.randn(V // 2, H, device=dev) * 0.05).bfloat16()
    w = torch.cat([half, half])
    h = torch.randn(R, H, device=dev).bfloat16()
    am = teacher_argmax(_Head(w), h, chunk=3000)
    z = K.gemm_nt(h, w)
    assert torch.equal(am, torch.argmax(z.float(), dim=-1))
    assert bool((am < V // 2).all())


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_project_hidden_states(dev, dtype):
    torch.manual_seed(9)
    B, L, H, V = 2, 96, 128, 3000
    hidden = torch.randn(B, L, H, device=dev).to(dtype)
    w = (torch.randn(V, H, device=dev) * 0.05).to(dtype)
    m1 = torch.rand(B, L, device=dev) < 0.5
    m2 = torch.rand(B, L, device=dev) < 0.3
    head = _Head(w)
    hr = hidden.clone().requires_grad_(True)
    out = project_hidden_states(head, hr, {"a": m1, "b": m2, "none": torch.zeros_like(m1)})
    ref_h = hidden.float().clone().requires_grad_(True)
    refs = {k: ref_h[m] @ w.float().T for k, m in (("a", m1), ("b", m2))}
    tol = 1e-5 if dtype == torch.float32 else 8e-3
    for k in ("a", "b"):
        assert out[k].shape == refs[k].shape
        assert ((out[k].float() - refs[k]).norm() / refs[k].norm()).item() < tol
    assert out["none"].shape == (0, V)
    g1 = torch.randn_like(refs["a"])
    g2 = torch.randn_like(refs["b"])
    ((out["a"].float() * g1).sum() + (out["b"].float() * g2).sum()).backward()
    ((refs["a"] * g1).sum() + (refs["b"] * g2).sum()).backward()
    assert ((hr.grad.float() - ref_h.grad).norm() / ref_h.grad.norm()).item() < (1e-5 if dtype == torch.float32
                                                                                   else 1e-2)


def test_resolve_ce_targets(dev):
    torch.manual_seed(10)
    B, L, V = 2, 64, 5003
    labels = torch.randint(0, V, (B, L), device=dev)
    labels[:, :8] = -100
    pos = torch.arange(L, device=dev).expand(B, L)
    shifted = shift_labels_for_next_token(labels, pos)
    ce_mask = (torch.rand(B, L, device=dev) < 0.4) & (shifted != -100)
    data = resolve_ce_targets("data", shifted, ce_mask, None)
    assert torch.equal(data, shifted[ce_mask])
    n = int(ce_mask.sum())
    z = _tied_logits(n, V, torch.bfloat16, dev)
    tgt = resolve_ce_targets("clean_argmax", shifted, ce_mask, z)
    assert torch.equal(tgt.cpu(), torch.argmax(z.float().cpu(), dim=-1))
    with pytest.raises(ValueError):
        resolve_ce_targets("teacher", shifted, ce_mask, z)
    with pytest.raises(RuntimeError):
        resolve_ce_targets("clean_argmax", shifted, ce_mask, None)
    with pytest.raises(RuntimeError):
        resolve_ce_targets("clean_argmax", shifted, ce_mask, z[:-1])
