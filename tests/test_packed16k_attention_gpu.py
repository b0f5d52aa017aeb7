"""Block-diffusion attention on one 16384-token row of packed log-normal segments (the long-context
configuration: median 3000, sigma 0.6, clipped to [512, 16384], block 32, 32 q / 8 kv heads of
128), forward of both streams and the noisy stream's dQ / dK / dV, against fp32 dense attention
over the oracle's mask, computed segment by segment (segments never attend across each other)."""
import math

import pytest
import torch

from oracle import bd as obd
from uno_amd import kernels as K
from uno_amd.model import bd_prepare

pytestmark = pytest.mark.gpu

L, BLOCK, HQ, HKV, D = 16384, 32, 32, 8, 128


def _segments(seed):
    g = torch.Generator().manual_seed(seed)
    out, left = [], L
    while left > 0:
        n = int(math.exp(math.log(3000.0) + 0.6 * torch.randn((), generator=g).item()))
        n = min(max(n, 512), left)
        out.append(n)
        left -= n
    return out


def _rel(a, b):
    return ((a.float() - b.float()).norm() / b.float().norm()).item()


@pytest.mark.parametrize("seed", [3])
def test_packed_16k_row_attention(dev, seed):
    segs = _segments(seed)
    print(f"[packed 16k] segments {segs}", flush=True)
    pos = torch.cat([torch.arange(n) for n in segs]).view(1, L)
    ids = torch.zeros(1, L, dtype=torch.int64)
    prompt = torch.zeros(1, L, dtype=torch.bool)
    _, _, mask, _, _, _ = bd_prepare(ids.to(dev), pos.to(dev), prompt.to(dev), block_size=BLOCK, mask_token_id=511)
    torch.manual_seed(seed)
    bf = torch.bfloat16
    qc, qn = (torch.randn(L, HQ * D, device=dev).to(bf) for _ in range(2))
    kc, vc, kn, vn = (torch.randn(L, HKV * D, device=dev).to(bf) for _ in range(4))
    do = torch.randn(L, HQ * D, device=dev).to(bf)
    oc, lc = K.attn_fwd(qc, kc, vc, mask.iv_clean, HQ, HKV, D)
    on, ln = K.attn_fwd(qn, kc, vc, mask.iv_noisy, HQ, HKV, D, k2=kn, v2=vn)
    dk = torch.empty(L, HKV * D, device=dev, dtype=bf)
    dv = torch.empty(L, HKV * D, device=dev, dtype=bf)
    dq = K.attn_bwd(qn, kc, vc, mask.iv_noisy, on, ln, do, HQ, HKV, D, k2=kn, v2=vn, ivk=mask.iv_noisy, dk=dk, dv=dv)
    torch.cuda.synchronize()

    ref = {n: torch.zeros(L, HQ * D, device=dev) for n in ("oc", "on", "dq")}
    ref.update({n: torch.zeros(L, HKV * D, device=dev) for n in ("dk", "dv")})
    ref_lc = torch.zeros(L, HQ, device=dev)
    ref_ln = torch.zeros(L, HQ, device=dev)
    rep, scale = HQ // HKV, D ** -0.5
    start = 0
    for n in segs:
        rows = slice(start, start + n)
        dense = obd.dense_mask(torch.arange(n)[None], BLOCK)[0].to(dev)      # [noisy n | clean n] x same
        allow_c = dense[n:, n:]
        allow_n = torch.cat([dense[:n, n:], dense[:n, :n]], 1)               # keys: [clean | noisy]
        for h in range(HQ):
            kv = h // rep
            hs, ks = slice(h * D, (h + 1) * D), slice(kv * D, (kv + 1) * D)
            k_c, v_c = kc[rows, ks].float(), vc[rows, ks].float()
            # clean stream: causal within the segment
            s = (qc[rows, hs].float() @ k_c.T) * scale
            s = s.masked_fill(~allow_c, float("-inf"))
            ref["oc"][rows, hs] = torch.softmax(s, -1) @ v_c
            ref_lc[rows, h] = torch.logsumexp(s, -1) / math.log(2.0)
            # noisy stream: earlier clean blocks + its own noisy block, with gradients
            q = qn[rows, hs].float().requires_grad_(True)
            k_n = kn[rows, ks].float().requires_grad_(True)
            v_n = vn[rows, ks].float().requires_grad_(True)
            s = (q @ torch.cat([k_c, k_n]).T) * scale
            s = s.masked_fill(~allow_n, float("-inf"))
            o = torch.softmax(s, -1) @ torch.cat([v_c, v_n])
            (o * do[rows, hs].float()).sum().backward()
            ref["on"][rows, hs] = o.detach()
            ref_ln[rows, h] = (torch.logsumexp(s, -1) / math.log(2.0)).detach()
            ref["dq"][rows, hs] = q.grad
            ref["dk"][rows, ks] += k_n.grad
            ref["dv"][rows, ks] += v_n.grad
            del s, o, q, k_n, v_n
        start += n
    got = {"oc": oc, "on": on, "dq": dq, "dk": dk, "dv": dv}
    for name, tol in (("oc", 1.2e-2), ("on", 1.2e-2), ("dq", 2e-2), ("dk", 2e-2), ("dv", 2e-2)):
        r = _rel(got[name], ref[name])
        print(f"   {name}: rel L2 {r:.3e} (bar {tol})", flush=True)
        assert r < tol, name
    for name, mine, theirs in (("lse clean", lc, ref_lc), ("lse noisy", ln, ref_ln)):
        err = (mine - theirs).abs().max().item()
        print(f"   {name}: max abs {err:.3e}", flush=True)
        assert err < 2e-2, name
