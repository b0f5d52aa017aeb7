"""Block-diffusion noising, concatenation and attention-mask contract (oracle restatement).

The reference obtains these from the remote ``prepare_for_bd_training`` (call site
training/trainer.py:198-209), which is not part of the reference tree. This module states
the contract the build implements; it is pinned by brute-force loops, invariants and the
published splitmix64 vectors, not by the remote code (whose exact RNG stream is unknown).

Contract (per batch row b, per segment [s, s+l) of the packed row, in-segment index j):
  * block(j) = j // block_size;
  * t(block) = noise_level(unit_float(draw(key, STREAM_BLOCK_T, b, s + block*block_size)));
  * token noised iff not prompt and unit_float(draw(key, STREAM_TOKEN_U, b, s+j)) < t(block);
  * uniform noise replaces a noised id by 1 + draw(key, STREAM_TOKEN_ID, b, s+j) mod (mask_id-1),
    an id in [1, mask_id) (nano_vllm_uno/engine/noise.py:24-26); "mask" noise uses mask_id;
  * concatenated row: noisy copy of the segment at [2s, 2s+l), clean copy at [2s+l, 2s+2l),
    both with the segment's positions (training/modeling.py:65-81 builds the matching mask);
  * p_mask = t of each noised token's block, row-major order (indexed at trainer.py:278);
  * attention (query -> key, same segment only):
      clean(i) -> clean(j)  iff j <= i                  (causal clean stream)
      noisy(i) -> clean(j)  iff block(j) <  block(i)    (strictly earlier clean blocks)
      noisy(i) -> noisy(j)  iff block(j) == block(i)    (bidirectional inside the block;
                                                         "causal" variant: and j <= i)
"""
from __future__ import annotations

import numpy as np
import torch

from . import hashing as H
from .layout import segment_starts


def segments_of(model_pos: torch.Tensor):
    """Per row, list of (start, length) from position resets."""
    starts = segment_starts(model_pos)
    out = []
    L = model_pos.shape[1]
    for row in starts.tolist():
        idx = [t for t, s in enumerate(row) if s] + [L]
        out.append([(idx[k], idx[k + 1] - idx[k]) for k in range(len(idx) - 1)])
    return out


def noise_tokens(input_ids: torch.Tensor, model_pos: torch.Tensor, prompt_mask: torch.Tensor, *,
                 block_size: int, mask_token_id: int, seed: int, step: int, noise: str = "uniform"):
    """Returns (noised [B,L] bool, noised_ids [B,L] int64, t_full [B,L] float32)."""
    if noise not in ("uniform", "mask"):
        raise ValueError(f"unsupported noise mode {noise!r}")
    B, L = input_ids.shape
    key = H.step_key(seed, step)
    segs = segments_of(model_pos)
    seg_start = np.zeros((B, L), dtype=np.int64)
    for b, row in enumerate(segs):
        for s, l in row:
            seg_start[b, s:s + l] = s
    t_idx = np.broadcast_to(np.arange(L, dtype=np.int64), (B, L))
    rows = np.broadcast_to(np.arange(B, dtype=np.int64)[:, None], (B, L))
    j = t_idx - seg_start
    block_start = seg_start + (j // block_size) * block_size
    t_blk = H.noise_level(H.unit_float(H.draw(key, H.STREAM_BLOCK_T, rows, block_start)))
    u_tok = H.unit_float(H.draw(key, H.STREAM_TOKEN_U, rows, t_idx))
    prompt = prompt_mask.numpy().astype(bool)
    noised = (~prompt) & (u_tok < t_blk)
    if noise == "uniform":
        rep = (np.uint64(1) + H.draw(key, H.STREAM_TOKEN_ID, rows, t_idx) % np.uint64(mask_token_id - 1)).astype(np.int64)
    else:
        rep = np.full((B, L), mask_token_id, dtype=np.int64)
    ids = input_ids.numpy()
    noised_ids = np.where(noised, rep, ids)
    return (torch.from_numpy(noised.copy()), torch.from_numpy(noised_ids.astype(np.int64)),
            torch.from_numpy(t_blk.astype(np.float32)))


def concat_streams(noised_ids: torch.Tensor, input_ids: torch.Tensor, model_pos: torch.Tensor):
    """[noisy | clean] per segment: returns concat_ids [B,2L], concat_pos [B,2L]."""
    B, L = input_ids.shape
    cids = torch.empty((B, 2 * L), dtype=torch.long)
    cpos = torch.empty((B, 2 * L), dtype=torch.long)
    for b, row in enumerate(segments_of(model_pos)):
        for s, l in row:
            cids[b, 2 * s:2 * s + l] = noised_ids[b, s:s + l]
            cids[b, 2 * s + l:2 * s + 2 * l] = input_ids[b, s:s + l]
            cpos[b, 2 * s:2 * s + l] = model_pos[b, s:s + l]
            cpos[b, 2 * s + l:2 * s + 2 * l] = model_pos[b, s:s + l]
    return cids, cpos


def concat_descriptors(model_pos: torch.Tensor):
    """Per concat index: (segment id, is_noisy, in-segment index). Each [B, 2L]."""
    B, L = model_pos.shape
    seg = torch.empty((B, 2 * L), dtype=torch.long)
    noisy = torch.empty((B, 2 * L), dtype=torch.bool)
    j = torch.empty((B, 2 * L), dtype=torch.long)
    for b, row in enumerate(segments_of(model_pos)):
        for k, (s, l) in enumerate(row):
            ar = torch.arange(l)
            seg[b, 2 * s:2 * s + 2 * l] = k
            noisy[b, 2 * s:2 * s + l] = True
            noisy[b, 2 * s + l:2 * s + 2 * l] = False
            j[b, 2 * s:2 * s + l] = ar
            j[b, 2 * s + l:2 * s + 2 * l] = ar
    return seg, noisy, j


def dense_mask(model_pos: torch.Tensor, block_size: int, intra_block: str = "bidirectional") -> torch.Tensor:
    """Allowed (query, key) pairs over the concatenated layout, [B, 2L, 2L] bool."""
    seg, noisy, j = concat_descriptors(model_pos)
    same = seg[:, :, None] == seg[:, None, :]
    qn, kn = noisy[:, :, None], noisy[:, None, :]
    jq, jk = j[:, :, None], j[:, None, :]
    bq, bk = jq // block_size, jk // block_size
    clean_clean = (~qn) & (~kn) & (jk <= jq)
    noisy_clean = qn & (~kn) & (bk < bq)
    noisy_noisy = qn & kn & (bk == bq)
    if intra_block == "causal":
        noisy_noisy = noisy_noisy & (jk <= jq)
    elif intra_block != "bidirectional":
        raise ValueError(intra_block)
    return same & (clean_clean | noisy_clean | noisy_noisy)


def dense_mask_bruteforce(model_pos: torch.Tensor, block_size: int, intra_block: str = "bidirectional") -> torch.Tensor:
    """Pure-Python loop over all pairs (spec restated literally; tiny inputs only)."""
    seg, noisy, j = concat_descriptors(model_pos)
    B, L2 = seg.shape
    out = torch.zeros((B, L2, L2), dtype=torch.bool)
    for b in range(B):
        for q in range(L2):
            for k in range(L2):
                if seg[b, q] != seg[b, k]:
                    continue
                iq, ik = int(j[b, q]), int(j[b, k])
                if not noisy[b, q]:
                    ok = (not noisy[b, k]) and ik <= iq
                elif not noisy[b, k]:
                    ok = ik // block_size < iq // block_size
                else:
                    ok = ik // block_size == iq // block_size
                    if intra_block == "causal":
                        ok = ok and ik <= iq
                out[b, q, k] = ok
    return out


def prepare_for_bd_training(input_ids, model_pos, prompt_mask, *, block_size: int, mask_token_id: int,
                            seed: int, step: int, noise: str = "uniform"):
    """The 6-tuple of the call contract (training/trainer.py:198-209), with a dense mask."""
    noised, noised_ids, t_full = noise_tokens(input_ids, model_pos, prompt_mask, block_size=block_size,
                                              mask_token_id=mask_token_id, seed=seed, step=step, noise=noise)
    cids, cpos = concat_streams(noised_ids, input_ids, model_pos)
    mask = dense_mask(model_pos, block_size)
    p_mask = t_full[noised]
    return cids, cpos, mask, noised, t_full, p_mask
