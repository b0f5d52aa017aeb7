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


def test_gemm_nt_operand_beyond_4gib(dev):
    """An operand whose rows lie 2^20 elements apart spans more than 4 GiB (the shape of the TV / KL
    logit-gradient product, dz [rows, vocab] times the LM head): the 256x256 kernel addresses each
    256-row strip from its own base, so its 32-bit buffer offsets still reach every row. Checked
    against fp32 and, bit for bit, against the same rows as a compact operand."""
    torch.manual_seed(11)
    M, Kd, N, lda = 2304, 4096, 512, 1 << 20
    big = torch.empty(M, lda, device=dev, dtype=torch.bfloat16)     # 4.8 GB
    a = big[:, :Kd]
    a.copy_(torch.randn(M, Kd, device=dev))
    b = torch.randn(N, Kd, device=dev).bfloat16()
    out = K.gemm_nt(a, b)
    compact = K.gemm_nt(a.contiguous(), b)
    ref = a.float() @ b.float().T
    torch.cuda.synchronize()
    assert _rel(out, ref) < 1e-2
    assert torch.equal(out, compact)
    del big


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


@pytest.mark.parametrize("M,N,Kd", [(8192, 8192, 512), (8200, 8448, 576), (16384, 4096, 320), (32768, 384, 4096)])
def test_gemm_nt_direct_to_lds_path(dev, M, N, Kd):
    """Shapes large enough (>= 512 tiles of 256x256, K a multiple of 64) for the direct-to-LDS
    kernel, including ragged M/N edges, with fp32 output."""
    assert K.nt_uses_256_tiles(M, N, [N])
    torch.manual_seed(M + N)
    a = torch.randn(M, Kd, device=dev).bfloat16()
    b = torch.randn(N, Kd, device=dev).bfloat16()
    out = K.gemm_nt(a, b, out_dtype=torch.float32)
    torch.cuda.synchronize()
    assert _rel(out, a.float() @ b.float().T) < 1e-5


@pytest.mark.parametrize("M,N,Kd", [(16384, 64, 4096), (16384, 128, 1024), (16384, 192, 4096),
                                    (8237, 64, 12288), (4096, 100, 512), (5000, 160, 640),
                                    (32768, 128, 12288), (32800, 120, 8192)])
@pytest.mark.parametrize("out_dtype", [torch.bfloat16, torch.float32])
def test_gemm_nt_skinny_path(dev, M, N, Kd, out_dtype):
    """Skinny products (N <= 192, M >= 4096, K a multiple of 64): one 64-row tile spans all N
    columns (128-row tiles of 8 waves for N <= 128 at >= 32768 rows and K >= 8192). Ragged M and N,
    a row gate and alpha, bf16 and fp32 outputs."""
    torch.manual_seed(M + N + Kd)
    a = torch.randn(M, Kd, device=dev).bfloat16()
    b = torch.randn(N, Kd, device=dev).bfloat16()
    gate = torch.rand(M, device=dev) > 0.3
    out = K.gemm_nt(a, b, gate=gate, alpha=0.75, out_dtype=out_dtype)
    torch.cuda.synchronize()
    ref = 0.75 * (a.float() @ b.float().T) * gate.float()[:, None]
    assert _rel(out, ref) < (1e-5 if out_dtype == torch.float32 else 5e-3)


def test_gemm_nt_direct_to_lds_lora_residual(dev):
    """q|k|v-shaped fused product on the direct-to-LDS kernel: three 256-aligned segments with
    their LoRA K-extension (K2 = 64), residual, alpha, bf16 output."""
    torch.manual_seed(2)
    M, Kd, r = 8192, 1024, 64
    ends = [4096, 5120, 6144]
    assert K.nt_uses_256_tiles(M, ends[-1], ends)
    a = torch.randn(M, Kd, device=dev).bfloat16()
    w = torch.randn(ends[-1], Kd, device=dev).bfloat16() * 0.05
    h = torch.randn(M, 3 * r, device=dev).bfloat16()
    bl = torch.randn(ends[-1], r, device=dev).bfloat16() * 0.05
    res = torch.randn(M, ends[-1], device=dev).bfloat16()
    out = K.gemm_nt(a, w, a2=h, b2=bl, segments=[(ends[0], 0), (ends[1], r), (ends[2], 2 * r)],
                    residual=res, alpha=0.5)
    ref = a.float() @ w.float().T
    start = 0
    for j, e in enumerate(ends):
        ref[:, start:e] += h[:, j * r:(j + 1) * r].float() @ bl[start:e].float().T
        start = e
    ref = 0.5 * ref + res.float()
    torch.cuda.synchronize()
    # bf16 output: the only error beyond fp32 accumulation is the final rounding (2^-9 relative)
    assert _rel(out, ref) < 4e-3


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


@pytest.mark.parametrize("Mr,P,Q", [(1000, 192, 4096), (16384, 4096, 64), (777, 1000, 96), (4100, 64, 12288),
                                     (300, 1032, 256), (16384, 128, 4096), (2000, 64, 1000), (2000, 1000, 64),
                                     (2000, 1000, 128), (16384, 192, 4096), (3000, 4104, 192),
                                     (4096, 32, 2048), (3000, 5640, 32), (16384, 5632, 32), (3000, 96, 5640),
                                     (16384, 96, 2048), (1000, 160, 4104), (2000, 4104, 160),
                                     (4100, 384, 4096), (3000, 4104, 384), (2000, 256, 1000), (16384, 4096, 256),
                                     (777, 384, 12288), (32768, 384, 4096), (2000, 224, 1024), (1000, 4096, 288)])
def test_gemm_tn_skinny_bf16(dev, Mr, P, Q):
    """LoRA weight-gradient shapes (rank side <= 256 columns, or 384 = 3r at rank 128; 32, 96 and 160
    are r, 3r and 5r at rank 32): dA = g^T x and dB = dY^T h, with ragged row counts and wide sides
    that are not a multiple of the 128- or 256-column strips; 224 and 288 take the general kernel."""
    torch.manual_seed(Mr + Q)
    a = torch.randn(Mr, P, device=dev).bfloat16()
    b = torch.randn(Mr, Q, device=dev).bfloat16()
    c0 = torch.randn(P, Q, device=dev)
    out = K.gemm_tn(a, b, out=c0.clone(), alpha=0.5, beta=1.0)
    ref = c0 + 0.5 * a.float().T @ b.float()
    fresh = K.gemm_tn(a, b, alpha=1.0)
    torch.cuda.synchronize()
    assert _rel(out, ref) < 1e-5
    assert _rel(fresh, a.float().T @ b.float()) < 1e-5


@pytest.mark.parametrize("r", [64, 32])
def test_gemm_tn_skinny_column_slices(dev, r):
    """Operands that are column slices of wider buffers (g_gu[:, r:2r], dgu[:, F:2F]) and an
    output that is a row slice of the flat gradient buffer."""
    torch.manual_seed(5)
    Mr, F = 2048, 1536
    dgu = torch.randn(Mr, 2 * F, device=dev).bfloat16()
    h = torch.randn(Mr, 2 * r, device=dev).bfloat16()
    flat = torch.randn(3 * F * r, device=dev)
    out = flat[F * r:2 * F * r].view(F, r)
    before = flat.clone()
    K.gemm_tn(dgu[:, F:], h[:, r:], out=out, alpha=2.0, beta=1.0)
    torch.cuda.synchronize()
    ref = before[F * r:2 * F * r].view(F, r) + 2.0 * dgu[:, F:].float().T @ h[:, r:].float()
    assert _rel(out, ref) < 1e-5
    assert torch.equal(flat[:F * r], before[:F * r]) and torch.equal(flat[2 * F * r:], before[2 * F * r:])


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


@pytest.mark.parametrize("M,F,Kd", [(512, 512, 256), (1024, 1536, 512), (256, 128, 64)])
def test_gemm_nt_swiglu_matches_unfused(dev, M, F, Kd):
    """Gate/up product with SwiGLU in the GEMM epilogue (64-row interleaved weights) equals the
    plain product on the [gate; up] layout followed by the SwiGLU kernel, bit for bit."""
    torch.manual_seed(M + F)
    x = (torch.randn(M, Kd, device=dev) * 0.5).bfloat16()
    w = (torch.randn(2 * F, Kd, device=dev) * 0.1).bfloat16()
    ref = K.swiglu_fwd(K.gemm_nt(x, w), F)
    fused = K.gemm_nt_swiglu(x, K.interleave_gate_up(w, F))
    torch.cuda.synchronize()
    assert fused.shape == (M, F)
    assert torch.equal(fused, ref)


def _interleave_lora_b(sb_gu, F, r):
    """[sB_gate; sB_up] [2F, r] -> [2F, 2r] in the interleaved row order, zero off-diagonal halves."""
    out = torch.zeros(F // 64, 2, 64, 2 * r, device=sb_gu.device, dtype=sb_gu.dtype)
    out[:, 0, :, :r] = sb_gu[:F].view(F // 64, 64, r)
    out[:, 1, :, r:] = sb_gu[F:].view(F // 64, 64, r)
    return out.view(2 * F, 2 * r)


@pytest.mark.parametrize("M,F,Kd,r", [(512, 512, 256, 32), (1024, 1536, 512, 64), (256, 256, 128, 64)])
def test_gemm_nt_swiglu_lora_and_gate_up_store(dev, M, F, Kd, r):
    """With the gate/up LoRA terms as one K = 2r extension on interleaved rows, and the [gate | up]
    product stored for the backward: both outputs equal the segmented LoRA product followed by the
    SwiGLU kernel, bit for bit."""
    torch.manual_seed(M + F + r)
    x = (torch.randn(M, Kd, device=dev) * 0.5).bfloat16()
    w = (torch.randn(2 * F, Kd, device=dev) * 0.1).bfloat16()
    h = (torch.randn(M, 2 * r, device=dev) * 0.5).bfloat16()
    sb = (torch.randn(2 * F, r, device=dev) * 0.1).bfloat16()
    gu_ref = K.gemm_nt(x, w, a2=h, b2=sb, segments=[(F, 0), (2 * F, r)])
    ref = K.swiglu_fwd(gu_ref, F)
    gu = torch.full((M, 2 * F), float("nan"), device=dev, dtype=torch.bfloat16)
    fused = K.gemm_nt_swiglu(x, K.interleave_gate_up(w, F), a2=h, b2_interleaved=_interleave_lora_b(sb, F, r), gu=gu)
    torch.cuda.synchronize()
    assert torch.equal(gu, gu_ref)
    assert torch.equal(fused, ref)


def test_lora_state_keeps_interleaved_gate_up_b(dev):
    """The LoRA state's interleaved gate/up sB follows the compute copy after every refresh."""
    from types import SimpleNamespace
    from uno_amd.adapter import LoraState
    cfg = SimpleNamespace(hidden_size=128, head_dim=64, num_attention_heads=2, num_key_value_heads=1,
                          intermediate_size=256, num_hidden_layers=3)
    st = LoraState(cfg, 32, 64.0, dev, torch.bfloat16)
    for it in range(2):
        st.master.normal_()
        st.refresh_copies()
        torch.cuda.synchronize()
        for li in range(3):
            assert torch.equal(st.sb_gu_i(li), _interleave_lora_b(st.sb_c(li, "gu"), 256, 32)), (it, li)


def test_gemm_nt_swiglu_rejects_unaligned_shapes(dev):
    x = torch.randn(300, 64, device=dev).bfloat16()
    w = torch.randn(256, 64, device=dev).bfloat16()
    with pytest.raises(ValueError, match="multiples of 256"):
        K.gemm_nt_swiglu(x, w)


@pytest.mark.parametrize("M,F,Kd,K2", [(512, 512, 256, 64), (1024, 1536, 512, 64), (256, 256, 128, 0)])
def test_gemm_nt_swiglu_bwd_matches_unfused(dev, M, F, Kd, K2):
    """SwiGLU backward in the epilogue of the down-projection data-gradient GEMM (with the LoRA
    K-extension) equals the product followed by the SwiGLU backward kernel, bit for bit."""
    torch.manual_seed(M + F + K2)
    dy = (torch.randn(M, Kd, device=dev) * 0.5).bfloat16()
    wt = (torch.randn(F, Kd, device=dev) * 0.1).bfloat16()
    gu = (torch.randn(M, 2 * F, device=dev) * 2.0).bfloat16()
    a2 = (torch.randn(M, K2, device=dev) * 0.5).bfloat16() if K2 else None
    b2 = (torch.randn(F, K2, device=dev) * 0.1).bfloat16() if K2 else None
    ds = K.gemm_nt(dy, wt, a2=a2, b2=b2)
    ref = K.swiglu_bwd(ds, gu, F)
    fused = K.gemm_nt_swiglu_bwd(dy, wt, a2, b2, gu)
    torch.cuda.synchronize()
    assert torch.equal(fused, ref)


@pytest.mark.parametrize("r", [32, 96])
def test_gemm_nt_lora_rank_not_multiple_of_64(dev, r):
    """LoRA extension of K2 = 32 (mod 64) on the 256x256 kernel (rank 32 of the 1B configuration):
    the last extension tile is half full. Against fp32 torch, and bit for bit against the same
    product with the extension zero-padded to the next multiple of 64."""
    torch.manual_seed(r)
    M, N, Kd = 4096, 6144, 512
    ends = [4096, 5120, 6144]
    assert K.nt_uses_256_tiles(M, N, ends)
    a = torch.randn(M, Kd, device=dev).bfloat16()
    w = (torch.randn(N, Kd, device=dev) * 0.1).bfloat16()
    h = torch.randn(M, 3 * r, device=dev).bfloat16()
    bl = (torch.randn(N, r, device=dev) * 0.1).bfloat16()
    res = torch.randn(M, N, device=dev).bfloat16()
    segs = [(4096, 0), (5120, r), (6144, 2 * r)]
    out = K.gemm_nt(a, w, a2=h, b2=bl, segments=segs, residual=res)
    ref = a.float() @ w.float().T
    start = 0
    for j, e in enumerate(ends):
        ref[:, start:e] += h[:, j * r:(j + 1) * r].float() @ bl[start:e].float().T
        start = e
    ref += res.float()
    rp = (r + 63) // 64 * 64
    hp = torch.zeros(M, 3 * rp, device=dev, dtype=torch.bfloat16)
    for j in range(3):
        hp[:, j * rp:j * rp + r] = h[:, j * r:(j + 1) * r]
    bp = torch.zeros(N, rp, device=dev, dtype=torch.bfloat16)
    bp[:, :r] = bl
    padded = K.gemm_nt(a, w, a2=hp, b2=bp, segments=[(4096, 0), (5120, rp), (6144, 2 * rp)], residual=res)
    torch.cuda.synchronize()
    assert _rel(out, ref) < 8e-3
    assert torch.equal(out, padded)


def test_gemm_nt_swiglu_bwd_rank_32(dev):
    """The SwiGLU-backward product with a rank-32 LoRA extension equals the product with the
    extension zero-padded to 64, bit for bit, and the unfused path within bf16 rounding."""
    torch.manual_seed(5)
    M, F, Kd, r = 1024, 1536, 512, 32
    dy = (torch.randn(M, Kd, device=dev) * 0.5).bfloat16()
    wt = (torch.randn(F, Kd, device=dev) * 0.1).bfloat16()
    gu = (torch.randn(M, 2 * F, device=dev) * 2.0).bfloat16()
    a2 = (torch.randn(M, r, device=dev) * 0.5).bfloat16()
    b2 = (torch.randn(F, r, device=dev) * 0.1).bfloat16()
    a2p = torch.zeros(M, 64, device=dev, dtype=torch.bfloat16)
    a2p[:, :r] = a2
    b2p = torch.zeros(F, 64, device=dev, dtype=torch.bfloat16)
    b2p[:, :r] = b2
    fused = K.gemm_nt_swiglu_bwd(dy, wt, a2, b2, gu)
    padded = K.gemm_nt_swiglu_bwd(dy, wt, a2p, b2p, gu)
    ds = (dy.float() @ wt.float().T + a2.float() @ b2.float().T).bfloat16()
    ref = K.swiglu_bwd(ds, gu, F)
    torch.cuda.synchronize()
    assert torch.equal(fused, padded)
    assert _rel(fused, ref) < 1e-2
