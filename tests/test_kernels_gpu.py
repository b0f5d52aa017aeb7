"""GPU parity of the row-wise, attention, loss, optimizer and batch-preparation kernels.

Each HIP kernel is compared with a plain fp32 PyTorch restatement of the same op (or with the
CPU oracle for the bit-exact integer work)."""
import math

import pytest
import torch
import torch.nn.functional as F

from oracle import bd as obd
from oracle import layout as olay
from oracle import losses as olosses
from uno_amd import kernels as K
from uno_amd.model import bd_prepare

pytestmark = pytest.mark.gpu


def rel(a, b):
    return ((a.float() - b.float()).norm() / b.float().norm().clamp_min(1e-30)).item()


def cos(a, b):
    return F.cosine_similarity(a.float().flatten(), b.float().flatten(), dim=0).item()


# ------------------------------------------------------------------------------------------
# RMSNorm / qk-norm + RoPE / SwiGLU
# ------------------------------------------------------------------------------------------
def ref_rmsnorm(x, w, eps):
    xf = x.float()
    return w.float() * (xf * torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + eps))


@pytest.mark.parametrize("dtype,M,H", [(torch.float32, 37, 256), (torch.bfloat16, 300, 4096), (torch.bfloat16, 5, 2048)])
def test_rmsnorm_fwd_bwd(dev, dtype, M, H):
    torch.manual_seed(0)
    x = torch.randn(M, H, device=dev).to(dtype)
    w = (1 + 0.1 * torch.randn(H, device=dev)).to(dtype)
    y, rstd = K.rmsnorm_fwd(x, w, 1e-6)
    xr = x.float().clone().requires_grad_(True)
    yr = ref_rmsnorm(xr, w, 1e-6)
    tol = 1e-6 if dtype == torch.float32 else 8e-3
    assert rel(y, yr) < tol
    dy = torch.randn(M, H, device=dev).to(dtype)
    dres = torch.randn(M, H, device=dev).to(dtype)
    yr.backward(dy.float())
    dx = K.rmsnorm_bwd(dy, x, w, rstd, dres=dres)
    assert rel(dx, xr.grad + dres.float()) < (1e-5 if dtype == torch.float32 else 8e-3)


def ref_qknorm_rope(qkv, nq, nk, d, wq, wk, pos, theta, eps):
    M = qkv.shape[0]
    q = qkv[:, :nq * d].float().view(M, nq, d)
    k = qkv[:, nq * d:(nq + nk) * d].float().view(M, nk, d)
    if wq is not None:
        q = ref_rmsnorm(q, wq, eps)
        k = ref_rmsnorm(k, wk, eps)
    inv = 1.0 / (theta ** (torch.arange(0, d, 2, dtype=torch.int64).float() / d))
    fr = pos.float().cpu()[:, None] * inv
    emb = torch.cat([fr, fr], -1).to(qkv.device)
    c, s = emb.cos()[:, None], emb.sin()[:, None]

    def rot(x):
        return torch.cat([-x[..., d // 2:], x[..., :d // 2]], -1)
    return (q * c + rot(q) * s).reshape(M, -1), (k * c + rot(k) * s).reshape(M, -1)


@pytest.mark.parametrize("dtype,d,norm,nq,nk", [(torch.float32, 64, True, 4, 2), (torch.bfloat16, 128, True, 4, 2),
                                                (torch.bfloat16, 128, False, 4, 2),
                                                # several groups of head passes, whole and partial
                                                (torch.bfloat16, 128, True, 32, 8), (torch.bfloat16, 128, False, 32, 32),
                                                (torch.float32, 64, True, 12, 4)])
def test_qknorm_rope_fwd_bwd(dev, dtype, d, norm, nq, nk):
    torch.manual_seed(1)
    M, theta = 96, 1e6
    qkv = torch.randn(M, (nq + 2 * nk) * d, device=dev).to(dtype)
    wq = (1 + 0.1 * torch.randn(d, device=dev)).to(dtype) if norm else None
    wk = (1 + 0.1 * torch.randn(d, device=dev)).to(dtype) if norm else None
    pos = torch.randint(0, 16384, (M,), device=dev)
    inv = (1.0 / (theta ** (torch.arange(0, d, 2, dtype=torch.int64).float() / d))).to(dev)
    q, k, rstd = K.qknorm_rope_fwd(qkv, nq, nk, d, wq, wk, pos, inv, 1e-6)
    x = qkv.float().clone().requires_grad_(True)
    qr, kr = ref_qknorm_rope(x, nq, nk, d, wq, wk, pos, theta, 1e-6)
    tol = 2e-5 if dtype == torch.float32 else 1e-2
    assert rel(q, qr) < tol and rel(k, kr) < tol
    dq = torch.randn_like(q)
    dk = torch.randn_like(k)
    (qr * dq.float()).sum().add_((kr * dk.float()).sum()).backward()
    dqkv = torch.zeros_like(qkv)
    K.qknorm_rope_bwd(dq, dk, qkv, nq, nk, d, wq, wk, pos, inv, rstd, dqkv)
    e = (nq + nk) * d
    assert rel(dqkv[:, :e], x.grad[:, :e]) < (5e-5 if dtype == torch.float32 else 1e-2)


@pytest.mark.parametrize("nq,nk", [(4, 2), (32, 8)])
def test_qknorm_rope_fp32_in_bf16_out(dev, nq, nk):
    """The bf16 step's q/k path: an fp32 q/k/v projection normalised and rotated in fp32 and rounded
    once (q, k and the copied v heads in bf16, v bit-identical to rounding the input), and the
    backward from fp32 dq/dk and the fp32 projection into a bf16 dqkv. Against fp32 torch, and at
    least as close as the all-bf16 path that rounds the projection first."""
    torch.manual_seed(11)
    M, d, theta = 96, 128, 1e6
    qkv = torch.randn(M, (nq + 2 * nk) * d, device=dev)
    wq = (1 + 0.1 * torch.randn(d, device=dev)).bfloat16()
    wk = (1 + 0.1 * torch.randn(d, device=dev)).bfloat16()
    pos = torch.randint(0, 16384, (M,), device=dev)
    inv = (1.0 / (theta ** (torch.arange(0, d, 2, dtype=torch.int64).float() / d))).to(dev)
    q, k, v, rstd = K.qknorm_rope_fwd(qkv, nq, nk, d, wq, wk, pos, inv, 1e-6, out_dtype=torch.bfloat16, with_v=True)
    assert q.dtype == k.dtype == v.dtype == torch.bfloat16
    assert torch.equal(v, qkv[:, (nq + nk) * d:].bfloat16())
    x = qkv.clone().requires_grad_(True)
    qr, kr = ref_qknorm_rope(x, nq, nk, d, wq, wk, pos, theta, 1e-6)
    q16, k16, _ = K.qknorm_rope_fwd(qkv.bfloat16(), nq, nk, d, wq, wk, pos, inv, 1e-6)
    assert rel(q, qr) < 4e-3 and rel(k, kr) < 4e-3
    assert rel(q, qr) <= rel(q16, qr) and rel(k, kr) <= rel(k16, kr)
    dq = torch.randn_like(qr)
    dk = torch.randn_like(kr)
    (qr * dq).sum().add_((kr * dk).sum()).backward()
    dqkv = torch.zeros(M, (nq + 2 * nk) * d, device=dev, dtype=torch.bfloat16)
    K.qknorm_rope_bwd(dq.contiguous(), dk.contiguous(), qkv, nq, nk, d, wq, wk, pos, inv, rstd, dqkv)
    e = (nq + nk) * d
    assert rel(dqkv[:, :e], x.grad[:, :e]) < 4e-3
    with pytest.raises(RuntimeError):
        K.qknorm_rope_bwd(dq.bfloat16().contiguous(), dk.contiguous(), qkv, nq, nk, d, wq, wk, pos, inv, rstd, dqkv)


@pytest.mark.parametrize("nq,nk,norm,lora", [(32, 8, True, True), (16, 8, True, False), (8, 8, False, True)])
def test_qkv_projection_rope_epilogue(dev, nq, nk, norm, lora):
    """The q|k|v GEMM with q/k norm + RoPE in its epilogue against the same GEMM into fp32 followed by
    the stand-alone q/k-norm kernel: v and the bf16 pre-norm q/k bit-identical to rounding the fp32
    product, q and k within one bf16 step of the two-kernel path, rstd to fp32 rounding; the q/k-norm
    backward from those bf16 pre-norm columns close to the one from the fp32 product."""
    torch.manual_seed(12)
    M, H, r, d = 8192, 1024, 32, 128     # both paths on the 256 x 256 kernel (the same accumulation)
    q_end, k_end, N = nq * d, (nq + nk) * d, (nq + 2 * nk) * d
    x = (torch.randn(M, H, device=dev) * 0.5).bfloat16()
    w = (torch.randn(N, H, device=dev) * 0.03).bfloat16()
    kw = {}
    if lora:
        kw = dict(a2=(torch.randn(M, 3 * r, device=dev) * 0.3).bfloat16(),
                  b2=(torch.randn(N, r, device=dev) * 0.05).bfloat16(), segments=[(q_end, 0), (k_end, r), (N, 2 * r)])
    wq = (1 + 0.1 * torch.randn(d, device=dev)).bfloat16() if norm else None
    wk = (1 + 0.1 * torch.randn(d, device=dev)).bfloat16() if norm else None
    pos = (torch.arange(M, device=dev) % 3000) + 7      # segment-like resets, largest position 3006
    inv = (1.0 / (1e6 ** (torch.arange(0, d, 2, dtype=torch.int64).float() / d))).to(dev)
    cos, sin = K.rope_table(int(pos.max()) + 1, inv)
    qf, kf, vf, rf, pre = K.gemm_nt_qkv_rope(x, w, nq, nk, wq, wk, pos, cos, sin, 1e-6, want_pre=True, **kw)
    qkv = K.gemm_nt(x, w, out_dtype=torch.float32, **kw)
    q2, k2, v2, r2 = K.qknorm_rope_fwd(qkv, nq, nk, d, wq, wk, pos, inv, 1e-6, out_dtype=torch.bfloat16, with_v=True)
    assert torch.equal(vf, v2) and torch.equal(vf, qkv[:, k_end:].bfloat16())
    assert torch.equal(pre, qkv[:, :k_end].bfloat16())

    # the two paths contract the rotation's multiply-adds differently: the same values up to fp32
    # rounding before the one bf16 rounding (a bf16 step apart where that rounding tips, more steps
    # only where the rotated value cancels to near zero)
    for a, b in ((qf, q2), (kf, k2)):
        diff = (a.float() - b.float()).abs()
        step = b.float().abs().clamp_min(b.float().abs().max() * 2 ** -8) * 2 ** -7
        print(f"[qkv epilogue] rel L2 {rel(a, b):.2e}; elements more than one bf16 step apart at their "
              f"magnitude: {int((diff > step).sum())} of {diff.numel()}", flush=True)
        assert rel(a, b) < 2e-3 and bool((diff <= step).all())
    if norm:
        assert torch.allclose(rf, r2, rtol=1e-6, atol=0)
    dq = torch.randn(M, q_end, device=dev)
    dk = torch.randn(M, k_end - q_end, device=dev)
    d1 = torch.zeros(M, N, device=dev, dtype=torch.bfloat16)
    d2 = torch.zeros_like(d1)
    K.qknorm_rope_bwd(dq, dk, pre, nq, nk, d, wq, wk, pos, inv, rf, d1)
    K.qknorm_rope_bwd(dq, dk, qkv, nq, nk, d, wq, wk, pos, inv, r2, d2)
    assert rel(d1[:, :k_end], d2[:, :k_end]) < 5e-3


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_swiglu_fwd_bwd(dev, dtype):
    torch.manual_seed(2)
    M, Fd = 77, 768
    gu = torch.randn(M, 2 * Fd, device=dev).to(dtype)
    x = gu.float().clone().requires_grad_(True)
    ref = F.silu(x[:, :Fd]) * x[:, Fd:]
    out = K.swiglu_fwd(gu, Fd)
    assert rel(out, ref) < (1e-6 if dtype == torch.float32 else 8e-3)
    d = torch.randn(M, Fd, device=dev).to(dtype)
    ref.backward(d.float())
    dgu = K.swiglu_bwd(d, gu, Fd)
    assert rel(dgu, x.grad) < (1e-5 if dtype == torch.float32 else 1e-2)


def test_embedding_and_rows_copy(dev):
    torch.manual_seed(3)
    table = torch.randn(1000, 256, device=dev).bfloat16()
    ids = torch.randint(0, 1000, (333,), device=dev)
    assert torch.equal(K.embedding(ids, table), table[ids])
    src = torch.randn(50, 128, device=dev)
    perm = torch.randperm(50, device=dev).to(torch.int32)
    dst = torch.zeros(50, 128, device=dev)
    K.rows_copy(src, dst, 50, dmap=perm)
    assert torch.equal(dst[perm.long()], src)
    out = torch.zeros(50, 128, device=dev)
    K.rows_copy(src, out, 50, smap=perm)
    assert torch.equal(out, src[perm.long()])


# ------------------------------------------------------------------------------------------
# Batch preparation: bit-exact against the oracle contract
# ------------------------------------------------------------------------------------------
def _batch(B, L, V, prompt, seed, packed=False):
    g = torch.Generator().manual_seed(seed)
    ids = torch.randint(0, V - 1, (B, L), generator=g)
    labels = ids.clone()
    labels[:, :prompt] = -100
    pos = torch.arange(L)[None].repeat(B, 1)
    if packed:
        cuts = [0, L // 3, L // 3 + L // 5, L]
        for b in range(1, B):
            for a, c in zip(cuts[:-1], cuts[1:]):
                pos[b, a:c] = torch.arange(c - a)
                labels[b, a:a + max(1, (c - a) // 10)] = -100
    return ids, labels, pos


@pytest.mark.parametrize("L,bs,packed,noise", [(64, 4, False, "uniform"), (96, 6, True, "uniform"),
                                               (256, 16, True, "mask"), (4096, 16, False, "uniform")])
def test_bd_prepare_bit_exact(dev, L, bs, packed, noise):
    B, V = 3, 4096
    ids, labels, pos = _batch(B, L, V, L // 8, seed=L + bs, packed=packed)
    prompt = labels == -100
    out = bd_prepare(ids.to(dev), pos.to(dev), prompt.to(dev), block_size=bs, mask_token_id=V - 1, noise=noise,
                     seed=20260813, step=5)
    cids, cpos, mask, noised, tfull, p_mask = out
    ref = obd.prepare_for_bd_training(ids, pos, prompt, block_size=bs, mask_token_id=V - 1, seed=20260813,
                                      step=5, noise=noise)
    assert torch.equal(cids.cpu(), ref[0])
    assert torch.equal(cpos.cpu(), ref[1])
    assert torch.equal(noised.cpu(), ref[3])
    assert torch.equal(tfull.cpu().view(torch.int32), ref[4].view(torch.int32))       # bit-exact floats
    assert torch.equal(p_mask.cpu().view(torch.int32), ref[5].view(torch.int32))
    _, _, region = olay.prepare_uno_layout(ids, pos)
    assert torch.equal(mask.region.cpu(), region)
    if L <= 256:
        assert torch.equal(mask.to_dense(), ref[2])


def _lognormal_row(total, seed, median=3000, sigma=0.6, lo=512):
    """Segment lengths of one packed row: log-normal (median, sigma) clipped to [lo, total]."""
    g = torch.Generator().manual_seed(seed)
    out, left = [], total
    while left > 0:
        n = int(math.exp(math.log(median) + sigma * torch.randn((), generator=g).item()))
        n = min(max(n, lo), left)
        out.append(n)
        left -= n
    return out


@pytest.mark.parametrize("B,L,kind", [(3, 64, "single"), (2, 96, "packed"), (4, 4096, "single"),
                                      (1, 16384, "lognormal"), (2, 3000, "ones")])
def test_region_kernel_matches_oracle(dev, B, L, kind):
    """prepare_uno_layout's region mask (one device kernel) against the oracle's per-segment loop
    (training/modeling.py:65-81): single rows, packed rows, 16384-token rows of log-normal
    segments, and rows of length-1 segments (the position never increases)."""
    if kind == "packed":
        _, _, pos = _batch(B, L, 512, 8, seed=3, packed=True)
    elif kind == "lognormal":
        segs = _lognormal_row(L, seed=11)
        pos = torch.cat([torch.arange(n) for n in segs]).view(1, L).repeat(B, 1)
    elif kind == "ones":
        pos = torch.zeros(B, L, dtype=torch.int64)
    else:
        pos = torch.arange(L).view(1, L).repeat(B, 1)
    from uno_amd.model import noisy_region_mask
    mine = noisy_region_mask(pos.to(dev)).cpu()
    ids = torch.zeros(B, L, dtype=torch.int64)
    _, _, ref = olay.prepare_uno_layout(ids, pos)
    assert torch.equal(mine, ref)


def test_extract_regions_split_any_tensor(dev):
    """extract_uno_regions on a tensor the decoder did not produce: the device row split equals
    the reference's boolean indexing (training/modeling.py:101-113)."""
    from uno_amd.model import noisy_region_mask
    from uno_amd.training.modeling import extract_uno_regions
    B, L, H = 2, 96, 64
    _, _, pos = _batch(B, L, 512, 8, seed=5, packed=True)
    region = noisy_region_mask(pos.to(dev))
    hidden = torch.randn(B, 2 * L, H, device=dev).bfloat16()
    noisy, clean = extract_uno_regions(hidden, region, L)
    assert torch.equal(noisy, hidden[region].reshape(B, L, H))
    assert torch.equal(clean, hidden[~region].reshape(B, L, H))


# ------------------------------------------------------------------------------------------
# Attention: two-stream kernels against dense attention over the oracle's mask
# ------------------------------------------------------------------------------------------
def _dense_attn(q, k, v, allow, D):
    """q [Mq,Hq,D], k/v [Mk,Hkv,D] fp32, allow [Mq,Mk] bool -> O [Mq,Hq,D], lse2 [Mq,Hq]."""
    rep = q.shape[1] // k.shape[1]
    k = k.repeat_interleave(rep, 1).permute(1, 2, 0).contiguous()     # [Hq, D, Mk]
    v = v.repeat_interleave(rep, 1).permute(1, 0, 2).contiguous()     # [Hq, Mk, D]
    qh = q.permute(1, 0, 2).contiguous()                              # [Hq, Mq, D]
    s = torch.matmul(qh, k) * D ** -0.5
    s = s.masked_fill(~allow[None], float("-inf"))
    o = torch.matmul(torch.softmax(s, -1), v).permute(1, 0, 2)
    lse2 = torch.logsumexp(s, -1).T / math.log(2.0)
    return o, lse2


@pytest.mark.parametrize("dtype,D,L,bs,packed,intra", [(torch.bfloat16, 128, 256, 16, False, "bidirectional"),
                                                       (torch.bfloat16, 128, 320, 6, True, "bidirectional"),
                                                       (torch.bfloat16, 64, 192, 12, True, "bidirectional"),
                                                       (torch.float32, 64, 128, 4, True, "bidirectional"),
                                                       (torch.bfloat16, 128, 320, 16, True, "causal"),
                                                       (torch.float32, 64, 128, 6, True, "causal")])
def test_block_diffusion_attention(dev, dtype, D, L, bs, packed, intra):
    """Both streams' forward and the noisy stream's dQ/dK/dV against dense attention over the
    oracle's mask. ``causal`` is the in-block variant the inference draft uses
    (nano_vllm_uno/layers/attention.py:658-666): noisy token j sees noisy tokens <= j of its block."""
    torch.manual_seed(4)
    B, Hq, Hkv = 2, 4, 2
    ids, labels, pos = _batch(B, L, 512, 8, seed=7, packed=packed)
    _, _, mask, _, _, _ = bd_prepare(ids.to(dev), pos.to(dev), (labels == -100).to(dev), block_size=bs,
                                     mask_token_id=511, intra_block=intra)
    M = B * L
    dense = obd.dense_mask(pos, bs, intra)                # oracle mask over the concat layout
    if L <= 256:
        assert torch.equal(mask.to_dense(), dense)
    ns, cs = mask.noisy_src.long().cpu(), mask.clean_src.long().cpu()
    full = torch.zeros(B * 2 * L, B * 2 * L, dtype=torch.bool)
    for b in range(B):
        full[b * 2 * L:(b + 1) * 2 * L, b * 2 * L:(b + 1) * 2 * L] = dense[b]
    allow_c = full[cs[:, None], cs[None, :]].to(dev)                                  # clean q -> clean k
    allow_n = torch.cat([full[ns[:, None], cs[None, :]], full[ns[:, None], ns[None, :]]], 1).to(dev)
    qc, qn = (torch.randn(M, Hq, D, device=dev).to(dtype) for _ in range(2))
    kc, vc, kn, vn = (torch.randn(M, Hkv, D, device=dev).to(dtype) for _ in range(4))
    flat = lambda t: t.reshape(M, -1)
    oc, lc = K.attn_fwd(flat(qc), flat(kc), flat(vc), mask.iv_clean, Hq, Hkv, D)
    on, ln = K.attn_fwd(flat(qn), flat(kc), flat(vc), mask.iv_noisy, Hq, Hkv, D, k2=flat(kn), v2=flat(vn))
    ref_oc, ref_lc = _dense_attn(qc.float(), kc.float(), vc.float(), allow_c, D)
    qn_r, kn_r, vn_r = (t.float().clone().requires_grad_(True) for t in (qn, kn, vn))
    ref_on, ref_ln = _dense_attn(qn_r, torch.cat([kc.float(), kn_r]), torch.cat([vc.float(), vn_r]), allow_n, D)
    tol = 1e-5 if dtype == torch.float32 else 1.2e-2
    assert rel(oc, flat(ref_oc)) < tol and rel(on, flat(ref_on)) < tol
    assert (lc - ref_lc).abs().max().item() < (1e-4 if dtype == torch.float32 else 2e-2)
    assert (ln - ref_ln).abs().max().item() < (1e-4 if dtype == torch.float32 else 2e-2)
    do = torch.randn(M, Hq * D, device=dev).to(dtype)
    (flat(ref_on) * do.float()).sum().backward()
    dk = torch.empty(M, Hkv * D, device=dev, dtype=dtype)
    dv = torch.empty(M, Hkv * D, device=dev, dtype=dtype)
    dq = K.attn_bwd(flat(qn), flat(kc), flat(vc), mask.iv_noisy, on, ln, do, Hq, Hkv, D, k2=flat(kn), v2=flat(vn),
                    ivk=mask.iv_noisy, dk=dk, dv=dv)
    gtol = 1e-4 if dtype == torch.float32 else 2e-2
    assert rel(dq, flat(qn_r.grad)) < gtol
    assert rel(dk, flat(kn_r.grad)) < gtol
    assert rel(dv, flat(vn_r.grad)) < gtol
    if dtype == torch.bfloat16:
        # dQ and dK in fp32 from the same kernels: the same values before their final rounding
        dk32 = torch.empty(M, Hkv * D, device=dev, dtype=torch.float32)
        dv2 = torch.empty_like(dv)
        dq32 = K.attn_bwd(flat(qn), flat(kc), flat(vc), mask.iv_noisy, on, ln, do, Hq, Hkv, D, k2=flat(kn),
                          v2=flat(vn), ivk=mask.iv_noisy, dk=dk32, dv=dv2, grad_dtype=torch.float32)
        assert dq32.dtype == torch.float32
        assert torch.equal(dq32.bfloat16(), dq) and torch.equal(dk32.bfloat16(), dk) and torch.equal(dv2, dv)


@pytest.mark.parametrize("D,Hq,Hkv,norm", [(128, 8, 2, True), (128, 4, 4, False), (64, 4, 2, True)])
def test_attention_backward_with_qknorm_epilogue(dev, D, Hq, Hkv, norm):
    """The noisy stream's backward with the q/k-norm + RoPE backward in the dQ and dK/dV epilogues
    against the two-kernel path (fp32 dQ / dK, then the stand-alone q/k-norm backward from the same
    bf16 pre-norm columns): dV bit-identical, the q and k gradient blocks within a bf16 step."""
    torch.manual_seed(13)
    B, L, bs = 2, 320, 16
    ids, labels, pos = _batch(B, L, 512, 8, seed=7, packed=True)
    _, _, mask, _, _, _ = bd_prepare(ids.to(dev), pos.to(dev), (labels == -100).to(dev), block_size=bs,
                                     mask_token_id=511)
    M = B * L
    bf = torch.bfloat16
    qn = torch.randn(M, Hq * D, device=dev).to(bf)
    kc, vc, kn, vn = (torch.randn(M, Hkv * D, device=dev).to(bf) for _ in range(4))
    on, ln = K.attn_fwd(qn, kc, vc, mask.iv_noisy, Hq, Hkv, D, k2=kn, v2=vn)
    do = torch.randn(M, Hq * D, device=dev).to(bf)
    pre = torch.randn(M, (Hq + Hkv) * D, device=dev).to(bf)
    wq = (1 + 0.1 * torch.randn(D, device=dev)).to(bf) if norm else None
    wk = (1 + 0.1 * torch.randn(D, device=dev)).to(bf) if norm else None
    rstd = torch.rsqrt(pre.float().view(M, Hq + Hkv, D).pow(2).mean(-1) + 1e-6).contiguous()
    inv = (1.0 / (1e6 ** (torch.arange(0, D, 2, dtype=torch.int64).float() / D))).to(dev)
    pos_s = mask.pos_stream
    cos, sin = K.rope_table(int(pos_s.max()) + 1, inv)
    n_all = (Hq + 2 * Hkv) * D
    fused = torch.zeros(M, n_all, device=dev, dtype=bf)
    K.attn_bwd_qknorm(qn, kc, vc, mask.iv_noisy, on, ln, do, Hq, Hkv, D, kn, vn, pre, rstd, wq, wk, pos_s, cos, sin,
                      fused)
    ref = torch.zeros_like(fused)
    dk = torch.empty(M, Hkv * D, device=dev, dtype=torch.float32)
    dq = K.attn_bwd(qn, kc, vc, mask.iv_noisy, on, ln, do, Hq, Hkv, D, k2=kn, v2=vn, ivk=mask.iv_noisy, dk=dk,
                    dv=ref[:, (Hq + Hkv) * D:], grad_dtype=torch.float32)
    K.qknorm_rope_bwd(dq, dk, pre, Hq, Hkv, D, wq, wk, pos_s, inv, rstd, ref)
    e = (Hq + Hkv) * D
    assert torch.equal(fused[:, e:], ref[:, e:])
    diff = (fused[:, :e].float() - ref[:, :e].float()).abs()
    mag = ref[:, :e].float().abs()
    step = mag.clamp_min(mag.max() * 2 ** -8) * 2 ** -7
    print(f"[attn bwd + qk-norm] rel L2 {rel(fused[:, :e], ref[:, :e]):.2e}; beyond one bf16 step: "
          f"{int((diff > step).sum())} of {diff.numel()}", flush=True)
    assert rel(fused[:, :e], ref[:, :e]) < 2e-3 and bool((diff <= step).all())


# ------------------------------------------------------------------------------------------
# Objectives
# ------------------------------------------------------------------------------------------
class _Head:
    def __init__(self, w):
        self.weight = w
        self.weight_t = w.t().contiguous()


@pytest.mark.parametrize("path", ["gemm_epilogue", "chunk_buffer"])
@pytest.mark.parametrize("dtype,R,H,V,chunk", [(torch.float32, 50, 64, 5000, 2048),
                                               (torch.float32, 50, 64, 5003, 2048),
                                               (torch.bfloat16, 300, 256, 8192, 3000),
                                               (torch.bfloat16, 300, 256, 8200, 4096),
                                               (torch.bfloat16, 1000, 512, 151936, 16384),
                                               (torch.bfloat16, 777, 4096, 151936, 32768)])
def test_chunked_weighted_ce(dev, dtype, R, H, V, chunk, path, monkeypatch):
    """Weighted CE against fp32 torch: bf16 through the LM-head GEMM epilogues (softmax statistics
    forward, recomputed-logit gradient backward; no [rows x vocab] buffer) and through the chunk
    buffer with the row kernels (fp32 mode, and bf16 forced onto it)."""
    from uno_amd import objectives
    from uno_amd.objectives import fused_weighted_ce, teacher_argmax
    if path == "chunk_buffer":
        monkeypatch.setattr(objectives, "_fused_ce_ok", lambda h, w: False)
    elif dtype == torch.float32:
        pytest.skip("the GEMM-epilogue path is bf16 only")
    torch.manual_seed(5)
    h = (torch.randn(R, H, device=dev) * 0.5).to(dtype)
    w = (torch.randn(V, H, device=dev) * 0.05).to(dtype)
    y = torch.randint(0, V, (R,), device=dev)
    p = torch.rand(R, device=dev) * 0.95 + 0.05
    inv_n = torch.tensor(1.0 / 777, device=dev)
    hr = h.float().clone().requires_grad_(True)
    logits = hr @ w.float().T
    ref = (F.cross_entropy(logits, y, reduction="none") / p).sum() / 777
    ref.backward()
    hh = h.clone().requires_grad_(True)
    loss = fused_weighted_ce(_Head(w), hh, y, 1.0 / p, inv_n, chunk=chunk)
    loss.backward()
    assert abs(loss.item() - ref.item()) / abs(ref.item()) < (1e-5 if dtype == torch.float32 else 1e-3)
    assert rel(hh.grad, hr.grad) < (1e-4 if dtype == torch.float32 else 1e-2)
    am = teacher_argmax(_Head(w), h, chunk=chunk)
    lg = (h.float() @ w.float().T) if dtype == torch.float32 else (h.float() @ w.float().T).bfloat16().float()
    assert (am == lg.argmax(-1)).float().mean().item() > (0.999 if dtype == torch.float32 else 0.98)


@pytest.mark.parametrize("R,H,V,chunk", [(300, 256, 8192, 3000), (777, 4096, 151936, 32768), (260, 512, 8200, 8200)])
def test_ce_stored_logits_match_recompute(dev, R, H, V, chunk, monkeypatch):
    """bf16 CE: the backward that forms dz from the logits the forward stored gives the same loss
    and data gradient, bit for bit, as the one that recomputes the logits in its GEMM epilogue
    (ragged row and vocabulary edges, a chunk that does not divide V)."""
    from uno_amd import objectives
    from uno_amd.objectives import fused_weighted_ce
    torch.manual_seed(7)
    h = (torch.randn(R, H, device=dev) * 0.5).bfloat16()
    w = (torch.randn(V, H, device=dev) * 0.05).bfloat16()
    y = torch.randint(0, V, (R,), device=dev)
    y[:3] = torch.tensor([0, V - 1, chunk], device=dev)       # targets on the vocabulary and chunk edges
    wts = torch.rand(R, device=dev) * 2 + 0.5
    inv_n = torch.tensor(1.0 / R, device=dev)
    out = {}
    for name, cap in (("stored", objectives.CE_STORED_LOGITS_MAX_BYTES), ("recompute", 0)):
        monkeypatch.setattr(objectives, "CE_STORED_LOGITS_MAX_BYTES", cap)
        hh = h.clone().requires_grad_(True)
        loss = fused_weighted_ce(_Head(w), hh, y, wts, inv_n, chunk=chunk)
        loss.backward()
        out[name] = (loss.detach().clone(), hh.grad.clone())
    torch.cuda.synchronize()
    assert torch.equal(out["stored"][0], out["recompute"][0])
    assert torch.equal(out["stored"][1], out["recompute"][1])


@pytest.mark.parametrize("kind", ["tv", "kl"])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("V", [4099, 8200])   # element-wise rows; 16-byte row walks with a partial last step
def test_distribution_losses_match_oracle(dev, kind, dtype, V):
    from uno_amd.training.losses import token_normalized_reverse_kl, token_normalized_total_variation
    torch.manual_seed(6)
    R = 40
    s = (torch.randn(R, V, device=dev) * 2).to(dtype)
    t = (torch.randn(R, V, device=dev) * 2).to(dtype)
    t[3] = s[3]
    sv = s.clone().requires_grad_(True)
    fn = token_normalized_total_variation if kind == "tv" else token_normalized_reverse_kl
    val = fn(sv, t, 17)
    val.backward()
    so = s.float().cpu().requires_grad_(True)
    ref = (olosses.total_variation if kind == "tv" else olosses.reverse_kl)(so, t.float().cpu(), 17)
    ref.backward()
    assert abs(val.item() - ref.item()) / abs(ref.item()) < (1e-5 if dtype == torch.float32 else 1e-4)
    assert rel(sv.grad.cpu(), so.grad) < (1e-4 if dtype == torch.float32 else 1e-2)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_distribution_losses_rows_with_neg_inf(dev, dtype):
    """Rows holding -inf logits, where a thread's first 16-byte groups are all -inf (the first 2048
    columns), scattered -inf columns, and -inf at the same column on both sides (p = q = 0, sign 0):
    TV stays finite and matches the reference's chunked algorithm, which takes the row max before any
    exponential (training/losses.py:76-160); reverse KL is NaN exactly where the reference's
    F.kl_div(log_target=True) is (0 * -inf at a -inf student column)."""
    from uno_amd.training.losses import token_normalized_reverse_kl, token_normalized_total_variation
    torch.manual_seed(7)
    R, V = 24, 8200
    s = torch.randn(R, V) * 2
    t = torch.randn(R, V) * 2
    s[0, :2048] = -float("inf")
    t[1, :2048] = -float("inf")
    s[2, :2048] = t[2, :2048] = -float("inf")
    s[3, 5000:5100] = -float("inf")
    s[4, ::7] = -float("inf")
    t[4, ::7] = -float("inf")
    s, t = s.to(dtype), t.to(dtype)
    sv = s.to(dev).requires_grad_(True)
    val = token_normalized_total_variation(sv, t.to(dev), 11)
    val.backward()
    ref, ref_grad = olosses.chunked_tv_reference_algorithm(s.float(), t.float(), 11)
    print(f"[-inf rows] TV {val.item():.6f} vs reference algorithm {ref.item():.6f}", flush=True)
    assert torch.isfinite(val).item() and torch.isfinite(sv.grad).all().item()
    assert abs(val.item() - ref.item()) / abs(ref.item()) < (1e-5 if dtype == torch.float32 else 1e-4)
    assert rel(sv.grad.float().cpu(), ref_grad) < (1e-4 if dtype == torch.float32 else 1e-2)
    # reverse KL per row: the reference's value is NaN on rows 0, 2, 3, 4 (student -inf columns)
    for r in range(6):
        kv = token_normalized_reverse_kl(s[r:r + 1].to(dev), t[r:r + 1].to(dev), 1).item()
        kr = torch.nn.functional.kl_div(torch.log_softmax(t[r:r + 1].float(), -1),
                                        torch.log_softmax(s[r:r + 1].float(), -1), log_target=True,
                                        reduction="sum").item()
        assert (kv != kv) == (kr != kr), (r, kv, kr)
        if math.isfinite(kr):
            assert abs(kv - kr) <= 1e-4 * max(1.0, abs(kr)), (r, kv, kr)
        elif kr == kr:
            assert kv == kr, (r, kv, kr)     # +inf: a -inf teacher column under a live student one


# ------------------------------------------------------------------------------------------
# Optimizer
# ------------------------------------------------------------------------------------------
@pytest.mark.parametrize("n", [100_003, 20_000_003])
def test_fused_adamw_matches_torch(dev, n):
    """Clip + AdamW + compute copy against torch; the larger size makes every thread of the grid
    take several passes (both the two-group body and the single-group tail)."""
    from uno_amd import _native as N
    torch.manual_seed(7)
    p0 = torch.randn(n, device=dev)
    parts = [slice(0, 40_000), slice(40_000, n)]
    ref = [p0[s].clone().requires_grad_(True) for s in parts]
    opt = torch.optim.AdamW(ref, lr=1e-3, betas=(0.9, 0.999), eps=1e-8, weight_decay=0.01)
    p, m, v = p0.clone(), torch.zeros(n, device=dev), torch.zeros(n, device=dev)
    partial = torch.empty(256, device=dev)
    clip = torch.empty(2, device=dev)
    copy = torch.empty(n, device=dev, dtype=torch.bfloat16)
    for step in range(1, 4):
        g = torch.randn(n, device=dev) * (0.02 if step < 3 else 3.0)
        for t, s in zip(ref, parts):
            t.grad = g[s].clone()
        torch.nn.utils.clip_grad_norm_(ref, 1.0)
        opt.step()
        gg = g.clone()
        N.call("unok_grad_clip_coef", n, N.ptr(gg), N.ptr(partial), 256, 1.0, N.ptr(clip), N.stream())
        N.call("unok_adamw_step", n, N.ptr(p), N.ptr(gg), N.ptr(m), N.ptr(v), N.ptr(clip), 1e-3, 0.9, 0.999, 1e-8,
               0.01, step, N.BF16, N.ptr(copy), 40_000, 2.0, N.stream())
        assert abs(clip[0].item() - g.norm().item()) / g.norm().item() < 1e-5
        assert torch.equal(gg, g * clip[1])
    mine = torch.cat([p[s] for s in parts])
    theirs = torch.cat([t.detach() for t in ref])
    assert (mine - theirs).abs().max().item() < 1e-6
    assert torch.equal(copy[:40_000], p[:40_000].bfloat16())
    assert torch.equal(copy[40_000:], (p[40_000:] * 2.0).bfloat16())


def test_bf16_rounding_matches_torch(dev):
    """The kernels' float->bf16 conversion is round-to-nearest-even like torch's, bit for bit."""
    from uno_amd import _native as N
    torch.manual_seed(8)
    x = torch.randn(1 << 16, device=dev) * torch.exp2(torch.randint(-140, 120, (1 << 16,), device=dev).float())
    specials = torch.tensor([0.0, -0.0, float("inf"), float("-inf"), 1.0 + 2 ** -8, 1.0 + 3 * 2 ** -8,
                             -(1.0 + 2 ** -8), 3.4e38, 1e-45, -1e-40], device=dev)
    # exact ties: mantissa ending in 0x8000 rounds to even
    ties = (torch.randint(0, 1 << 15, (4096,), device=dev, dtype=torch.int32) * 65536 + 0x3F808000).view(torch.float32)
    x = torch.cat([x, specials, ties]).contiguous()
    out = torch.empty(x.numel(), device=dev, dtype=torch.bfloat16)
    N.call("unok_cast_copy", N.BF16, x.numel(), x.numel(), 1.0, N.ptr(x), N.ptr(out), N.stream())
    mine, ref = out.view(torch.int16), x.bfloat16().view(torch.int16)
    # NaN payloads are not specified by either conversion: any NaN output counts as a match
    diff = (mine != ref) & ~(torch.isnan(x) & torch.isnan(out.float()))
    denormal = (x != 0) & (x.abs() < 2.0 ** -126)
    bad = diff & ~denormal
    print(f"[bf16 rounding] {int(diff.sum())} of {x.numel()} differ; {int(denormal.sum())} fp32-denormal inputs; "
          f"non-denormal mismatches {int(bad.sum())}: {x[bad][:8].tolist()}")
    assert not bad.any()
    # fp32-denormal inputs may be flushed to a signed zero by the hardware conversion
    flushed = diff & denormal
    assert ((mine[flushed] & 0x7FFF) == 0).all()


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_transpose_jobs(dev, dtype):
    """Batched transposes over one flat buffer: sides that are multiples of 8 at 16-byte-aligned
    offsets (the 16-byte path for bf16) next to ragged sides and odd offsets (the element path)."""
    from uno_amd import _native as N
    shapes = [(64, 64), (4096, 32), (32, 4104), (100, 37), (8, 8), (200, 136), (13, 8), (136, 40)]
    offs, off = [], 0
    for i, (r, c) in enumerate(shapes):
        off += 3 if i % 3 == 2 else 0          # every third job starts at an odd element offset
        offs.append(off)
        off += r * c
        off = (off + 7) // 8 * 8
    src = torch.randn(off, device=dev).to(dtype)
    dst = torch.full((off,), float("nan"), device=dev, dtype=dtype)
    jobs, tile = [], 0
    for (r, c), o in zip(shapes, offs):
        jobs.append([o, r, c, o, tile, 0, 0, 0])
        tile += ((r + 63) // 64) * ((c + 63) // 64)
    jt = torch.tensor(jobs, dtype=torch.int64, device=dev)
    N.call("unok_transpose_jobs", N.dtype_code(dtype), N.ptr(jt), len(jobs), tile, N.ptr(src), N.ptr(dst), N.stream())
    torch.cuda.synchronize()
    for (r, c), o in zip(shapes, offs):
        want = src[o:o + r * c].view(r, c).t()
        assert torch.equal(dst[o:o + r * c].view(c, r), want), (r, c, o)
