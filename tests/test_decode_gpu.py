"""GPU parity of the few-row gated LoRA linears of draft blocks (unok_gemm_nt_rows) against fp32
torch products of the same bf16 operands: row counts from one row to past one 128-row tile, LoRA
A rows as extra product columns with per-segment hidden columns, ranks 16 to 128, the row gate on
the LoRA hidden, residual, the SwiGLU epilogue, forced and automatic K-range counts, and
determinism across calls."""
import pytest
import torch

from uno_amd import kernels as K

pytestmark = pytest.mark.gpu


def _rel(a, b):
    return ((a.float() - b.float()).norm() / b.float().norm().clamp_min(1e-30)).item()


def _ref(a, w, la=None, lb=None, segments=None, residual=None, gate=None):
    """fp32 value of a w^T + h[:, seg] lb^T + residual with h = bf16(gate (.) a la^T)."""
    y = a.float() @ w.float().T
    if la is not None:
        h = a.float() @ la.float().T
        if gate is not None:
            h = h * gate.float()[:, None]
        h = h.bfloat16().float()
        r = lb.shape[1]
        lo = 0
        for end, col in (segments or [(w.shape[0], 0)]):
            y[:, lo:end] += h[:, col:col + r] @ lb[lo:end].float().T
            lo = end
    if residual is not None:
        y = y + residual.float()
    return y


@pytest.mark.parametrize("M", [1, 16, 100, 128, 200])
@pytest.mark.parametrize("N,Kd,splits", [(64, 4096, 0), (192, 512, 3), (1024, 1024, 1), (640, 3072, 0)])
def test_rows_plain(dev, M, N, Kd, splits):
    print(f"[rows] M={M} N={N} K={Kd} splits={splits}", flush=True)
    torch.manual_seed(M * 31 + N)
    a = torch.randn(M, Kd, device=dev).bfloat16()
    w = torch.randn(N, Kd, device=dev).bfloat16()
    out = K.gemm_nt_rows(a, w, splits=splits)
    again = K.gemm_nt_rows(a, w, splits=splits)
    torch.cuda.synchronize()
    assert _rel(out, _ref(a, w)) < 5e-3, (M, N, Kd, splits)
    assert torch.equal(out, again)


@pytest.mark.parametrize("r", [16, 64, 128])
@pytest.mark.parametrize("splits", [0, 1, 5])
@pytest.mark.parametrize("M", [40, 128])
def test_rows_lora_segments_gate_residual(dev, r, splits, M):
    """q|k|v-style linear: three segments reading their own r columns of the LoRA hidden, row gate
    on the hidden, residual. Gated-off rows equal the product without LoRA plus the residual, bit
    for bit (same K ranges)."""
    print(f"[rows lora] M={M} r={r} splits={splits}", flush=True)
    torch.manual_seed(r + splits + M)
    Kd = 1024
    segs = [(512, 0), (640, r), (768, 2 * r)]
    a = torch.randn(M, Kd, device=dev).bfloat16()
    w = (torch.randn(768, Kd, device=dev) * 0.05).bfloat16()
    la = (torch.randn(3 * r, Kd, device=dev) * 0.05).bfloat16()
    lb = torch.randn(768, r, device=dev).bfloat16()
    res = torch.randn(M, 768, device=dev).bfloat16()
    gate = torch.rand(M, device=dev) > 0.3
    out = K.gemm_nt_rows(a, w, lora_a=la, lora_b=lb, segments=segs, residual=res, gate=gate, splits=splits)
    torch.cuda.synchronize()
    ref = _ref(a, w, la, lb, segs, res, gate)
    assert _rel(out, ref) < 5e-3
    if splits > 0:
        base = K.gemm_nt_rows(a, w, residual=res, splits=splits)
        off = ~gate
        assert torch.equal(out[off], base[off])


@pytest.mark.parametrize("M,F,Kd,r", [(128, 1536, 1024, 64), (48, 768, 512, 32)])
@pytest.mark.parametrize("splits", [1, 4])
def test_rows_swiglu_epilogue(dev, M, F, Kd, r, splits):
    """The SwiGLU reduction equals the plain reduction (same K ranges) stored in bf16 followed by
    unok_swiglu_fwd, bit for bit, and the fp32 SwiGLU of the fp32 value to bf16 tolerance."""
    print(f"[rows swiglu] M={M} F={F} K={Kd} r={r} splits={splits}", flush=True)
    torch.manual_seed(F + splits)
    a = torch.randn(M, Kd, device=dev).bfloat16()
    w = (torch.randn(2 * F, Kd, device=dev) * 0.05).bfloat16()
    la = (torch.randn(2 * r, Kd, device=dev) * 0.05).bfloat16()
    lb = (torch.randn(2 * F, r, device=dev) * 0.05).bfloat16()
    gate = torch.rand(M, device=dev) > 0.5
    segs = [(F, 0), (2 * F, r)]
    s = K.gemm_nt_rows(a, w, lora_a=la, lora_b=lb, segments=segs, gate=gate, swiglu=True, splits=splits)
    gu = K.gemm_nt_rows(a, w, lora_a=la, lora_b=lb, segments=segs, gate=gate, splits=splits)
    unfused = K.swiglu_fwd(gu, F)
    torch.cuda.synchronize()
    assert torch.equal(s, unfused)
    y = _ref(a, w, la, lb, segs, gate=gate)
    ref = torch.nn.functional.silu(y[:, :F]) * y[:, F:]
    assert _rel(s, ref) < 1e-2


def test_rows_matches_unfused_lora_path(dev):
    """The fused linear against the two-product path of the training kernels (h = gate (.) x A^T
    by gemm_nt, then x W^T + h (s B)^T by the K-extended gemm_nt) on a q|k|v shape."""
    torch.manual_seed(7)
    M, Kd, r = 128, 2048, 64
    segs = [(1024, 0), (1280, r), (1536, 2 * r)]
    a = torch.randn(M, Kd, device=dev).bfloat16()
    w = (torch.randn(1536, Kd, device=dev) * 0.02).bfloat16()
    la = (torch.randn(3 * r, Kd, device=dev) * 0.02).bfloat16()
    lb = (torch.randn(1536, r, device=dev) * 0.02).bfloat16()
    gate = torch.ones(M, device=dev, dtype=torch.bool)
    gate[::16] = False
    fused = K.gemm_nt_rows(a, w, lora_a=la, lora_b=lb, segments=segs, gate=gate)
    h = K.gemm_nt(a, la, gate=gate)
    two = K.gemm_nt(a, w, a2=h, b2=lb, segments=segs)
    torch.cuda.synchronize()
    assert _rel(fused, two) < 5e-3


def test_rows_rejects_bad_shapes(dev):
    a = torch.randn(16, 192, device=dev).bfloat16()         # K not a multiple of 128
    w = torch.randn(64, 192, device=dev).bfloat16()
    with pytest.raises(ValueError, match="multiple of 128"):
        K.gemm_nt_rows(a, w)
    a = torch.randn(16, 256, device=dev).bfloat16()
    w = torch.randn(64, 256, device=dev).bfloat16()
    with pytest.raises(ValueError, match="K ranges"):
        K.gemm_nt_rows(a, w, splits=3)                       # 2 K tiles cannot make 3 ranges
    la = torch.randn(16, 256, device=dev).bfloat16()
    lb = torch.randn(64, 16, device=dev).bfloat16()
    with pytest.raises(ValueError, match="LoRA hidden columns"):
        K.gemm_nt_rows(a, w, lora_a=la, lora_b=lb, segments=[(32, 0), (64, 8)])


def _bf16_close(a, b):
    """Elementwise within one bf16 rounding step of the reference value."""
    a, b = a.float(), b.float()
    return bool(((a - b).abs() <= b.abs() * 2.0 ** -7 + 1e-6).all())


@pytest.mark.parametrize("D,nq,nk,L,norm", [(128, 8, 2, 16, True), (64, 4, 2, 8, True), (128, 4, 1, 32, False)])
def test_decode_prep_matches_training_kernels(dev, D, nq, nk, L, norm):
    """unok_decode_prep against unok_qknorm_rope_fwd at the same positions (lengths_b + t) plus the
    cache-store and query-layout row copies: K / V rows land at the committed lengths, the queries
    at row 128 (b nk + kv) + L (h % rep) + t, the other rows of each 128 are zeroed and no other
    cache row is written."""
    print(f"[decode prep] D={D} nq={nq} nk={nk} L={L} norm={norm}", flush=True)
    torch.manual_seed(D + L)
    B, max_len, rep = 3, 96, nq // nk
    lengths = torch.tensor([5, 17, 96 - L], device=dev, dtype=torch.int64)
    M = B * L
    qkv = torch.randn(M, (nq + 2 * nk) * D, device=dev).bfloat16()
    wq = (torch.rand(D, device=dev) + 0.5).bfloat16() if norm else None
    wk = (torch.rand(D, device=dev) + 0.5).bfloat16() if norm else None
    inv_freq = 1.0 / (1e6 ** (torch.arange(0, D, 2, device=dev, dtype=torch.float32) / D))
    kc = torch.zeros(B, nk, max_len, D, device=dev, dtype=torch.bfloat16)
    vc = torch.zeros_like(kc)
    qd = torch.full((B * nk * 128, D), 7.0, device=dev, dtype=torch.bfloat16)
    K.decode_prep(qkv, wq, wk, lengths, inv_freq, 1e-6, kc, vc, qd, B, L, nq, nk, D)
    pos = (lengths[:, None] + torch.arange(L, device=dev)[None]).reshape(-1).contiguous()
    q, k, _ = K.qknorm_rope_fwd(qkv, nq, nk, D, wq, wk, pos, inv_freq, 1e-6)
    v = qkv[:, (nq + nk) * D:]
    torch.cuda.synchronize()
    q = q.view(B, L, nq, D)
    k = k.view(B, L, nk, D)
    v = v.reshape(B, L, nk, D)
    written = torch.zeros(B, nk, max_len, dtype=torch.bool)
    for b in range(B):
        n = int(lengths[b])
        assert _bf16_close(kc[b, :, n:n + L].transpose(0, 1), k[b]), b
        assert torch.equal(vc[b, :, n:n + L].transpose(0, 1), v[b]), b
        written[b, :, n:n + L] = True
        for kv in range(nk):
            blk = qd[(b * nk + kv) * 128:(b * nk + kv + 1) * 128]
            for rr in range(rep):
                assert _bf16_close(blk[rr * L:(rr + 1) * L], q[b, :, kv * rep + rr]), (b, kv, rr)
            assert not blk[rep * L:].any()
    assert not kc.cpu()[~written].any() and not vc.cpu()[~written].any()


def test_attn_split_matches_unsplit(dev):
    """Split-key attention plus the log-sum-exp merge against the single-range kernel over the same
    causal cache prefix, including a sequence shorter than the number of ranges (ranges without
    keys) and padding rows, which the merge skips."""
    torch.manual_seed(11)
    D, L, rep, S, max_len = 128, 16, 2, 4, 160
    lengths = [3, 40, 137]
    pairs = len(lengths)
    QR = pairs * 128
    kc = torch.randn(pairs * max_len, D, device=dev).bfloat16()
    vc = torch.randn(pairs * max_len, D, device=dev).bfloat16()
    qd = torch.randn(QR, D, device=dev).bfloat16()
    iv = torch.zeros(QR, 8, dtype=torch.int32)
    ivs = torch.zeros(S * QR, 8, dtype=torch.int32)
    dst = torch.full((QR,), -1, dtype=torch.int32)
    for p, n in enumerate(lengths):
        start = p * max_len
        c = n // S
        for slot in range(128):
            row = p * 128 + slot
            if slot >= rep * L:
                continue
            t = slot % L
            seen = n + t + 1
            iv[row, 0], iv[row, 1] = start, start + seen
            dst[row] = row
            for s in range(S):
                lo = s * c
                hi = seen if s == S - 1 else min((s + 1) * c, seen)
                ivs[s * QR + row, 0], ivs[s * QR + row, 1] = start + lo, start + max(hi, lo)
    ref, _ = K.attn_fwd(qd, kc, vc, iv.to(dev), 1, 1, D)
    od, lse = K.attn_fwd_split(qd, kc, vc, ivs.to(dev), QR, S, D)
    out = torch.zeros(QR, D, device=dev, dtype=torch.bfloat16)
    K.attn_split_combine(od, lse, dst.to(dev), QR, S, D, out)
    torch.cuda.synchronize()
    valid = (dst >= 0).to(dev)
    assert _rel(out[valid], ref[valid]) < 1e-2
    assert not out[~valid].any()
