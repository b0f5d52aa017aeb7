"""GPU parity of the GEMM kernels against plain fp32 torch products of the same operands."""
import pytest
import torch

from uno_amd import kernels as K

pytestmark = pytest.mark.gpu


def _rel(a, b):
    return ((a.float() - b.float()).norm() / b.float().norm().clamp_min(1e-30)).item()


@pytest.mark.parametrize("M,N,Kd", [(256, 256, 64), (300, 200, 136), (1024, 1024, 512),
                                    (4096, 6144, 4096), (17, 640, 8), (2048, 64, 256)])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_gemm_nt_plain(dev, M, N, Kd, dtype):
    torch.manual_seed(M * 7 + N)
    a = torch.randn(M, Kd, device=dev).to(dtype)
    b = torch.randn(N, Kd, device=dev).to(dtype)
    ref = a.float() @ b.float().T
    out = K.gemm_nt(a, b, out_dtype=torch.float32)
    torch.cuda.synchronize()
    assert _rel(out, ref) < (1e-6 if dtype == torch.float32 else 1e-5), (M, N, Kd)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_gemm_nt_lora_segments_gate_residual(dev, dtype):
    """Fused q|k|v-style product: per-segment LoRA extension, row gate, residual, alpha."""
    torch.manual_seed(1)
    M, Kd, r = 640, 512, 64
    ends = [256, 384, 512]          # q | k | v output columns
    a = torch.randn(M, Kd, device=dev).to(dtype)
    w = torch.randn(512, Kd, device=dev).to(dtype)
    h = torch.randn(M, 3 * r, device=dev).to(dtype)
    bl = torch.randn(512, r, device=dev).to(dtype)
    res = torch.randn(M, 512, device=dev).to(dtype)
    gate = torch.rand(M, device=dev) > 0.5
    out = K.gemm_nt(a, w, a2=h, b2=bl, segments=[(256, 0), (384, r), (512, 2 * r)],
                    residual=res, gate=gate, alpha=0.5)
    ref = a.float() @ w.float().T
    start = 0
    for j, e in enumerate(ends):
        ref[:, start:e] += h[:, j * r:(j + 1) * r].float() @ bl[start:e].float().T
        start = e
    ref = 0.5 * ref * gate[:, None].float() + res.float()
    torch.cuda.synchronize()
    assert _rel(out, ref) < (1e-6 if dtype == torch.float32 else 8e-3)


@pytest.mark.parametrize("Mr,P,Q", [(4096, 64, 1024), (1000, 128, 64), (16384, 64, 4096), (64, 8, 16)])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_gemm_tn(dev, Mr, P, Q, dtype):
    torch.manual_seed(Mr + P)
    a = torch.randn(Mr, P, device=dev).to(dtype)
    b = torch.randn(Mr, Q, device=dev).to(dtype)
    c0 = torch.randn(P, Q, device=dev)
    out = K.gemm_tn(a, b, out=c0.clone(), alpha=2.0, beta=1.0)
    ref = c0 + 2.0 * a.float().T @ b.float()
    torch.cuda.synchronize()
    assert _rel(out, ref) < (1e-5 if dtype == torch.float32 else 1e-5)


def test_gemm_strided_views(dev):
    """Column-sliced operands (row stride > width), as used for fused projections."""
    torch.manual_seed(3)
    big = torch.randn(512, 1024, device=dev).bfloat16()
    a = big[:, 256:768]
    b = torch.randn(320, 512, device=dev).bfloat16()
    out_big = torch.zeros(512, 640, device=dev, dtype=torch.bfloat16)
    out = out_big[:, 64:384]
    K.gemm_nt(a, b, out=out)
    torch.cuda.synchronize()
    assert _rel(out, a.float() @ b.float().T) < 8e-3
    assert out_big[:, :64].abs().sum().item() == 0 and out_big[:, 384:].abs().sum().item() == 0
