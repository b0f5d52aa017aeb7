"""Draft forward of Uno's two-pass block decoding on the training step's kernels.

The inference side of the conditional LoRA (nano_vllm_uno/engine/two_pass_decoding.py:243-283,
draft_stage): each sequence feeds a block [seed, noise_1, ..., noise_(L-1)] through the decoder
over its KV cache; the LoRA update is gated per row -- off on the seed, on for the noise rows
(nano_vllm_uno/layers/linear.py:166-307, `lora_mask`) -- and attention is causal over the cache and
the block (nano_vllm_uno/layers/attention.py:628-668, BLOCK_DECODE: the block's K/V are stored into
the cache first, then flash attention with causal=True over the cached lengths). After the draft
the noise K/V are discarded: only the committed rows (the seed) advance the cache.

Kernels, all shared with the training step:
* the gated LoRA is the GEMM's K-extension: h = m (.) (x A^T) by the skinny GEMM with its row gate,
  then y = x W^T + h (s B)^T (+ residual) in the 256x256 / register-staged MFMA GEMMs;
* the cache is head-major, [layers][B, Hkv, max_len, D] for K and V, so one (sequence, K/V head)
  pair's keys are contiguous rows; the block's queries of that pair (L rows x the q-heads sharing
  the K/V head, at most 128) are laid out as the 128 query rows of one attention workgroup over
  that key range, with per-row key intervals [start, start + cached + j + 1) -- the block-diffusion
  attention kernel then reads each cache row once per pair;
* a prefill (empty caches) is the causal forward of the prompt with the LoRA gated off, through
  the clean-stream attention path (keys = the prompt itself).
"""
from __future__ import annotations

import torch

from . import kernels as K
from .layers import Geometry


class BlockKVCache:
    """Per-layer K and V, head-major [B, Hkv, max_len, D], and the committed length per sequence."""

    def __init__(self, geo: Geometry, layers: int, batch: int, max_len: int, device, dtype):
        shape = (batch, geo.nk, max_len, geo.d)
        self.k = [torch.zeros(shape, device=device, dtype=dtype) for _ in range(layers)]
        self.v = [torch.zeros(shape, device=device, dtype=dtype) for _ in range(layers)]
        self.lengths = torch.zeros(batch, device=device, dtype=torch.int64)
        self.batch, self.max_len, self.geo = batch, max_len, geo


class BlockDecoder:
    """Runs prefill and draft blocks of a Uno model (UnoLoraModel or a base model with an
    adapter attached) on the HIP kernels."""

    def __init__(self, lm):
        base = lm.get_base_model() if hasattr(lm, "get_base_model") else lm
        self.base = base
        self.decoder = base.model
        self.lora = self.decoder._uno_lora
        if self.lora is None:
            raise RuntimeError("BlockDecoder needs a model with a LoRA adapter attached (create_lora_model).")
        self.geo = self.decoder.geo

    def new_cache(self, batch: int, max_len: int) -> BlockKVCache:
        return BlockKVCache(self.geo, len(self.decoder.layers), batch, max_len, self.base.device, self.base.dtype)

    # ---- public entry points ------------------------------------------------------------------
    @torch.no_grad()
    def prefill(self, cache: BlockKVCache, prompt_ids: torch.Tensor) -> torch.Tensor:
        """Causal forward of [B, P] prompt tokens into empty caches (LoRA off); returns logits
        [B, P, V] and commits all P rows."""
        if int(cache.lengths.max()) != 0:
            raise RuntimeError("prefill expects empty caches")
        B, P = prompt_ids.shape
        gate = torch.zeros((B, P), device=prompt_ids.device, dtype=torch.bool)
        return self._forward(cache, prompt_ids, gate, commit=P, prefill=True)

    @torch.no_grad()
    def draft_block(self, cache: BlockKVCache, block_ids: torch.Tensor, lora_mask: torch.Tensor | None = None,
                    commit: int = 1) -> torch.Tensor:
        """One draft block [B, L] at positions cached + 0 .. L-1; returns logits [B, L, V]. The
        LoRA gate defaults to the draft layout (off on the seed row, on for the noise rows);
        ``commit`` rows (the seed) stay in the cache, the rest are discarded."""
        B, L = block_ids.shape
        if lora_mask is None:
            lora_mask = torch.ones((B, L), device=block_ids.device, dtype=torch.bool)
            lora_mask[:, 0] = False
        if tuple(lora_mask.shape) != (B, L):
            raise RuntimeError(f"LoRA row mask {tuple(lora_mask.shape)} does not match the block {(B, L)}")
        if not 0 <= commit <= L:
            raise ValueError(f"commit must lie in [0, {L}]")
        return self._forward(cache, block_ids, lora_mask.to(torch.bool), commit=commit, prefill=False)

    def capture_draft(self, cache: BlockKVCache, block_size: int, commit: int = 1) -> "DraftGraph":
        """A draft block of [cache.batch, block_size] rows over ``cache`` captured as one HIP graph
        (see DraftGraph)."""
        return DraftGraph(self, cache, block_size, commit)

    # ---- the decoder -----------------------------------------------------------------------------
    def _forward(self, cache: BlockKVCache, ids: torch.Tensor, gate: torch.Tensor, commit: int, prefill: bool,
                 check: bool = True):
        g, lora, dec = self.geo, self.lora, self.decoder
        B, L = ids.shape
        if B != cache.batch:
            raise RuntimeError(f"block batch {B} does not match the cache batch {cache.batch}")
        lengths = cache.lengths
        if check and int((lengths + L).max()) > cache.max_len:
            raise RuntimeError("the block does not fit in the KV cache")
        rep = g.nq // g.nk
        if not prefill and rep * L > 128:
            raise NotImplementedError(f"draft blocks hold at most 128 / {rep} rows per sequence (got {L})")
        dev = ids.device
        M = B * L
        j = torch.arange(L, device=dev)
        pos = (lengths[:, None] + j[None, :]).reshape(-1).contiguous()            # [M] int64
        gate_rows = gate.reshape(-1).contiguous()
        maps = self._maps(cache, lengths, B, L, prefill)
        h = K.embedding(ids.reshape(-1).contiguous().to(torch.int64), dec.embed_tokens.weight)
        for li, layer in enumerate(dec.layers):
            lw = layer.weights()
            h = self._layer(h, lw, li, pos, gate_rows, cache, maps, B, L, prefill)
        x, _ = K.rmsnorm_fwd(h, dec.norm.weight, g.eps)
        V = self.base.lm_head.weight.shape[0]
        head = K.gemm_nt_rows if self._rows_path(M, x.dtype, prefill) and V % 4 == 0 else K.gemm_nt
        logits = head(x, self.base.lm_head.weight)
        cache.lengths += commit
        return logits.view(B, L, -1)

    def _maps(self, cache, lengths, B, L, prefill):
        """Row maps of the cache store and of the decode query layout, and the key intervals."""
        g = self.geo
        dev = lengths.device
        i32 = dict(device=dev, dtype=torch.int32)
        rep = g.nq // g.nk
        out = {}
        slot = torch.arange(128, device=dev)
        pair = torch.arange(B * g.nk, device=dev)
        valid = slot < rep * L
        tt = slot % L
        start = pair[:, None] * cache.max_len                                           # [pairs, 1]
        lens = lengths[:, None].expand(B, g.nk).reshape(-1, 1)                          # [pairs, 1]
        seen = lens + tt[None, :] + 1                                                   # causal over cache + block
        if not prefill and self._split_path(dev, cache):
            # split-key layout: S key ranges per (sequence, K/V head) pair; range s of a query row
            # holds keys [s c, (s + 1) c) of its causal prefix (c = committed length // S), the last
            # range the rest; padding rows get empty ranges
            pairs = B * g.nk
            S = max(1, min(8, 256 // pairs))
            QR = pairs * 128
            c = lens // S
            s_idx = torch.arange(S, device=dev)[:, None, None]                          # [S, 1, 1]
            lo = s_idx * c[None]                                                         # [S, pairs, 1]
            hi = torch.where(s_idx == S - 1, seen[None], torch.minimum((s_idx + 1) * c[None], seen[None]))
            hi = torch.maximum(hi, lo)
            lo = torch.where(valid[None, None, :], lo, 0)
            hi = torch.where(valid[None, None, :], hi, 0)
            ivs = torch.zeros((S * QR, 8), **i32)
            ivs[:, 0] = (start[None] + lo).reshape(-1)
            ivs[:, 1] = (start[None] + hi).reshape(-1)
            # decode row (pair b nk + kv, slot r L + t) -> output row (b L + t) nq + kv rep + r
            dst = ((pair // g.nk)[:, None] * L + tt[None, :]) * g.nq + (pair % g.nk)[:, None] * rep + (slot // L)[None, :]
            out["dst"] = torch.where(valid[None, :], dst, -1).reshape(-1).to(**i32)
            out["ivs"], out["S"], out["QR"] = ivs, S, QR
            return out
        b = torch.arange(B, device=dev)[:, None, None]
        t = torch.arange(L, device=dev)[None, :, None]
        kv = torch.arange(g.nk, device=dev)[None, None, :]
        # cache store: key row (b, t, head) of the block -> cache row (b, head, lengths_b + t)
        out["store"] = ((b * g.nk + kv) * cache.max_len + lengths[:, None, None] + t).reshape(-1).to(**i32)
        if prefill:
            starts = (torch.arange(B, device=dev) * L)[:, None]
            iv = torch.zeros((B * L, 8), **i32)
            iv[:, 0] = starts.expand(B, L).reshape(-1)
            iv[:, 1] = (starts + torch.arange(1, L + 1, device=dev)[None, :]).reshape(-1)
            out["iv"] = iv
            return out
        # decode layout: query (b, t, head h = kv * rep + r) -> row (b * nk + kv) * 128 + r * L + t
        r = torch.arange(rep, device=dev)
        qrow = ((b * g.nk + kv)[..., None] * 128 + r[None, None, None, :] * L + t[..., None])   # [B, L, nk, rep]
        out["qrow"] = qrow.reshape(-1).to(**i32)
        iv = torch.zeros((B * g.nk * 128, 8), **i32)
        # rows past rep * L are padding: they see the pair's first key and their output is dropped
        iv[:, 0] = start.expand(-1, 128).reshape(-1)
        iv[:, 1] = torch.where(valid[None, :], start + seen, start + 1).reshape(-1)
        out["iv"] = iv
        return out

    def _split_path(self, dev, cache) -> bool:
        """bf16 draft blocks run the attention as prep + split-key attention + combine."""
        return cache.k[0].dtype == torch.bfloat16 and self.geo.d in (64, 128)

    def _rows_path(self, M: int, dtype, prefill: bool) -> bool:
        """Draft blocks in bf16 take the few-row products (K ranges over the whole chip) when every
        linear's shape fits them; prefills and fp32 models take gemm_nt."""
        g, r = self.geo, self.lora.rank
        return (not prefill and dtype == torch.bfloat16 and M <= 512 and r % 8 == 0 and 3 * r <= 512
                and all(k % 128 == 0 for k in (g.H, g.q, g.F)))

    def _layer(self, h0, lw, li, pos, gate_rows, cache, maps, B, L, prefill):
        g, lora = self.geo, self.lora
        r = lora.rank
        q_end, k_end = g.q, g.q + g.kv
        M = h0.shape[0]
        few = self._rows_path(M, h0.dtype, prefill)
        qkv_segments = [(q_end, 0), (k_end, r), (k_end + g.kv, 2 * r)]

        def linear(x, w, part, segments=None, residual=None, swiglu=False):
            """Gated LoRA linear: x w^T + (m (.) x A^T)[:, seg] (s B)^T (+ residual)."""
            if few:
                return K.gemm_nt_rows(x, w, lora_a=lora.a_c(li, part), lora_b=lora.sb_c(li, part),
                                      segments=segments, residual=residual, gate=gate_rows, swiglu=swiglu)
            h = K.gemm_nt(x, lora.a_c(li, part), gate=gate_rows)
            y = K.gemm_nt(x, w, a2=h, b2=lora.sb_c(li, part), segments=segments, residual=residual)
            return K.swiglu_fwd(y, y.shape[1] // 2) if swiglu else y

        x1, _ = K.rmsnorm_fwd(h0, lw.ln_in, g.eps)
        qkv = linear(x1, lw.w_qkv, "qkv", qkv_segments)
        ck = cache.k[li].view(-1, g.d)
        cv = cache.v[li].view(-1, g.d)
        if not prefill and "ivs" in maps:
            # q/k norm + RoPE, cache store and query layout in one kernel; split-key attention; merge
            S, QR = maps["S"], maps["QR"]
            qd = torch.empty((QR, g.d), device=qkv.device, dtype=qkv.dtype)
            K.decode_prep(qkv, lw.q_norm, lw.k_norm, cache.lengths, self.decoder.inv_freq, g.eps, cache.k[li],
                          cache.v[li], qd, B, L, g.nq, g.nk, g.d)
            od, lse = K.attn_fwd_split(qd, ck, cv, maps["ivs"], QR, S, g.d)
            o = torch.empty((M, g.q), device=qkv.device, dtype=qkv.dtype)
            K.attn_split_combine(od, lse, maps["dst"], QR, S, g.d, o.view(M * g.nq, g.d))
            return self._mlp(o, h0, lw, li, linear)
        q, k, _ = K.qknorm_rope_fwd(qkv, g.nq, g.nk, g.d, lw.q_norm, lw.k_norm, pos, self.decoder.inv_freq, g.eps)
        v = qkv[:, k_end:]
        # the block's K/V into the cache rows (b, head, cached + t)
        K.rows_copy(k.reshape(M * g.nk, g.d), ck, M * g.nk, dmap=maps["store"])
        K.rows_copy(v.contiguous().view(M * g.nk, g.d), cv, M * g.nk, dmap=maps["store"])
        if prefill:
            o, _ = K.attn_fwd(q, k, v, maps["iv"], g.nq, g.nk, g.d)
        else:
            rows = maps["iv"].shape[0]
            qd = torch.zeros((rows, g.d), device=q.device, dtype=q.dtype)
            K.rows_copy(q.reshape(M * g.nq, g.d), qd, M * g.nq, dmap=maps["qrow"])
            od, _ = K.attn_fwd(qd, ck, cv, maps["iv"], 1, 1, g.d)
            o = torch.empty((M, g.q), device=q.device, dtype=q.dtype)
            K.rows_copy(od, o.view(M * g.nq, g.d), M * g.nq, smap=maps["qrow"])
        return self._mlp(o, h0, lw, li, linear)

    def _mlp(self, o, h0, lw, li, linear):
        """o projection (+ residual), post-attention norm and the SwiGLU MLP (+ residual)."""
        g, r = self.geo, self.lora.rank
        h1 = linear(o, lw.w_o, "o", residual=h0)
        x2, _ = K.rmsnorm_fwd(h1, lw.ln_post, g.eps)
        # few-row path: the reduction of the gate/up product applies the SwiGLU ([gate | up] is never stored)
        s = linear(x2, lw.w_gu, "gu", [(g.F, 0), (2 * g.F, r)], swiglu=True)
        return linear(s, lw.w_d, "d", residual=h1)


class DraftGraph:
    """A draft block of fixed shape [B, L] over one cache, captured as a single HIP graph.

    The decoder issues about twenty kernels per layer; launched one by one from Python, a block of a
    36-layer model costs more host time than device time. Replaying the captured graph is one host
    call per block. Everything that depends on the committed lengths (the positions, the cache
    store rows, the decode query layout and the key intervals) is computed on the device from
    ``cache.lengths`` inside the graph, so each replay drafts at the current lengths and then
    advances them by ``commit``, exactly as ``BlockDecoder.draft_block``.

    ``replay`` returns the graph's own logits buffer [B, L, V], overwritten by the next replay.
    The cache capacity is checked on the host against the longest committed length read at
    capture plus the commits since; after changing ``cache.lengths`` by other means, capture
    again."""

    def __init__(self, decoder: BlockDecoder, cache: BlockKVCache, block_size: int, commit: int = 1):
        B, L = cache.batch, block_size
        rep = decoder.geo.nq // decoder.geo.nk
        if rep * L > 128:
            raise NotImplementedError(f"draft blocks hold at most 128 / {rep} rows per sequence (got {L})")
        if not 0 <= commit <= L:
            raise ValueError(f"commit must lie in [0, {L}]")
        dev = cache.lengths.device
        self.cache, self.block_size, self.commit = cache, L, commit
        self.ids = torch.zeros((B, L), device=dev, dtype=torch.int64)
        self.gate = torch.ones((B, L), device=dev, dtype=torch.bool)
        self.gate[:, 0] = False
        self._len_max = int(cache.lengths.max())
        if self._len_max + L > cache.max_len:
            raise RuntimeError("the block does not fit in the KV cache")
        # One eager pass without commit before the capture: it sets each kernel's launch attributes
        # outside the graph. Its K/V rows lie past the committed lengths, where the first replay
        # writes them again.
        decoder._forward(cache, self.ids, self.gate, commit=0, prefill=False)
        torch.cuda.synchronize()
        self.graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(self.graph):
            self.logits = decoder._forward(cache, self.ids, self.gate, commit=commit, prefill=False, check=False)

    def replay(self, block_ids: torch.Tensor, lora_mask: torch.Tensor | None = None) -> torch.Tensor:
        """Draft one block [B, L] of token ids (device int64); ``lora_mask`` [B, L] replaces the
        default gate (off on the seed row, on for the noise rows) for this and later replays."""
        if tuple(block_ids.shape) != tuple(self.ids.shape):
            raise RuntimeError(f"block {tuple(block_ids.shape)} does not match the captured {tuple(self.ids.shape)}")
        if self._len_max + self.block_size > self.cache.max_len:
            raise RuntimeError("the block does not fit in the KV cache")
        self.ids.copy_(block_ids)
        if lora_mask is not None:
            if tuple(lora_mask.shape) != tuple(self.gate.shape):
                raise RuntimeError(f"LoRA row mask {tuple(lora_mask.shape)} does not match the block")
            self.gate.copy_(lora_mask)
        self.graph.replay()
        self._len_max += self.commit
        return self.logits
