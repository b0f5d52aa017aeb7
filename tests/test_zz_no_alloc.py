"""unok_gemm_tn_noalloc (split-K partials in the library's per-device scratch array, nothing
allocated) against unok_gemm_tn with a caller workspace: same kernels and split counts, so the
results are bit-identical. Two calls in a row, the second smaller, so a stale scratch content
would show; then a problem beyond the 64 MiB scratch is rejected on the host."""
import ctypes

import pytest
import torch

from uno_amd import _native as N
from uno_amd import kernels as K

pytestmark = pytest.mark.gpu

# (rows, P, Q): the LoRA weight-gradient shapes of a 4096-hidden layer (dB = s dY^T h,
# dA = g^T x with g = [g_q | g_k | g_v]) and a smaller one.
CASES = [(16384, 4096, 64), (16384, 192, 4096), (4096, 64, 1024), (1000, 1408, 32)]


def _operands(rows, P, Q, seed, dev):
    g = torch.Generator(device=dev).manual_seed(seed)
    a = torch.randn(rows, P, device=dev, generator=g).bfloat16()
    b = torch.randn(rows, Q, device=dev, generator=g).bfloat16()
    c0 = torch.randn(P, Q, device=dev, generator=g)
    return a, b, c0


@pytest.mark.parametrize("order", [(0, 2), (1, 3), (0, 1, 2, 3)])
def test_noalloc_matches_workspace_entry(dev, order):
    for i, ci in enumerate(order):
        rows, P, Q = CASES[ci]
        print(f"[no-alloc] call {i}: rows={rows} P={P} Q={Q}", flush=True)
        a, b, c0 = _operands(rows, P, Q, 10 + ci, dev)
        ref = K.gemm_tn(a, b, out=c0.clone(), alpha=0.5, beta=1.0)
        mine = K.gemm_tn_noalloc(a, b, c0.clone(), alpha=0.5, beta=1.0)
        torch.cuda.synchronize()
        assert torch.equal(mine, ref), (rows, P, Q, (mine - ref).abs().max().item())
        # beta = 0 overwrites whatever the output held
        mine0 = K.gemm_tn_noalloc(a, b, torch.full_like(c0, float("nan")), beta=0.0)
        ref0 = K.gemm_tn(a, b)
        torch.cuda.synchronize()
        assert torch.equal(mine0, ref0)


def test_noalloc_rejects_oversized_problem(dev):
    rows, P, Q = 64, 256, 100000   # partials of 256 x 100000 fp32 = 102 MB > 64 MiB
    assert N.lib().unok_gemm_tn_workspace(rows, P, Q) > (64 << 20)
    a = torch.zeros(rows, P, device=dev, dtype=torch.bfloat16)
    b = torch.zeros(rows, Q, device=dev, dtype=torch.bfloat16)
    out = torch.zeros(P, Q, device=dev)
    with pytest.raises(ValueError, match="scratch"):
        K.gemm_tn_noalloc(a, b, out)
