"""Pins the oracle decoder against transformers' Qwen3Model and LoRA against merged weights."""
import pytest
import torch

from oracle import bd, layout
from oracle.model import Cfg, decoder, init_lora, init_params, module_path

CFG = Cfg(vocab_size=128, hidden_size=64, intermediate_size=96, num_hidden_layers=2,
          num_attention_heads=4, num_key_value_heads=2, head_dim=16, lora_rank=4, lora_alpha=8)


def _hf_model(cfg, params):
    from transformers import Qwen3Config
    from transformers.models.qwen3.modeling_qwen3 import Qwen3Model
    hc = Qwen3Config(vocab_size=cfg.vocab_size, hidden_size=cfg.hidden_size,
                     intermediate_size=cfg.intermediate_size, num_hidden_layers=cfg.num_hidden_layers,
                     num_attention_heads=cfg.num_attention_heads,
                     num_key_value_heads=cfg.num_key_value_heads, head_dim=cfg.head_dim,
                     rms_norm_eps=cfg.rms_norm_eps, rope_theta=cfg.rope_theta,
                     attn_implementation="eager")
    m = Qwen3Model(hc).eval()
    sd = {k[len("model."):]: v for k, v in params.items() if k.startswith("model.")}
    # non-trivial norm weights so a dropped norm weight would show
    m.load_state_dict(sd, strict=True)
    return m


def test_decoder_matches_transformers_qwen3_with_block_diffusion_mask():
    params = init_params(CFG, seed=0, std=0.05)
    g = torch.Generator().manual_seed(1)
    for k in params:
        if k.endswith("norm.weight") or k.endswith("layernorm.weight"):
            params[k] = 1 + 0.1 * torch.randn(params[k].shape, generator=g)
    lora = init_lora(CFG, seed=2)
    pos = torch.tensor([list(range(10)) + list(range(6))])
    ids = torch.randint(0, 128, (1, 16), generator=g)
    cids, cpos = bd.concat_streams(ids, ids, pos)
    mask = bd.dense_mask(pos, 4)
    gate = torch.zeros(1, 32, dtype=torch.bool)   # LoRA gated off everywhere -> base model
    ours = decoder(params, lora, CFG, cids, cpos, mask, gate)
    hf = _hf_model(CFG, params)
    add = torch.zeros(mask.shape).masked_fill(~mask, float("-inf"))[:, None]
    with torch.no_grad():
        hs = hf(input_ids=cids, attention_mask=add, position_ids=cpos).last_hidden_state
    assert (ours - hs).abs().max().item() < 1e-5


def test_lora_gate_on_equals_merged_weights():
    params = init_params(CFG, seed=3, std=0.05)
    lora = init_lora(CFG, seed=4, b_std=0.05)
    s = CFG.lora_scale
    merged = dict(params)
    for i in range(CFG.num_hidden_layers):
        for name in ("q_proj", "k_proj", "v_proj", "o_proj", "gate_proj", "up_proj", "down_proj"):
            p = module_path(i, name)
            merged[p + ".weight"] = params[p + ".weight"] + s * lora[p + ".lora_B.weight"] @ lora[p + ".lora_A.weight"]
    pos = torch.arange(12)[None]
    ids = torch.randint(0, 128, (1, 12))
    cids, cpos = bd.concat_streams(ids, ids, pos)
    mask = bd.dense_mask(pos, 3)
    on = torch.ones(1, 24, dtype=torch.bool)
    a = decoder(params, lora, CFG, cids, cpos, mask, on)
    b = decoder(merged, {}, CFG, cids, cpos, mask, None)
    assert (a - b).abs().max().item() < 1e-5
    # gate off on a row must give exactly the base output on that row when nothing it sees changes
    off = torch.zeros(1, 24, dtype=torch.bool)
    c = decoder(params, lora, CFG, cids, cpos, mask, off)
    d = decoder(params, {}, CFG, cids, cpos, mask, None)
    assert torch.equal(c, d)


def test_clean_stream_is_plain_causal_decoder():
    """The clean half of the 2L pass equals a causal pass over the original ids (LoRA off),
    which is what lets the GPU path run the clean stream forward-only."""
    params = init_params(CFG, seed=5, std=0.05)
    lora = init_lora(CFG, seed=6, b_std=0.05)
    L = 16
    ids = torch.randint(0, 128, (2, L))
    labels = ids.clone()
    labels[:, :4] = -100
    pos = torch.arange(L)[None].expand(2, -1)
    cids, cpos, mask, noised, _, _ = bd.prepare_for_bd_training(
        ids, pos, labels == -100, block_size=4, mask_token_id=127, seed=0, step=0)
    _, _, region = layout.prepare_uno_layout(ids, None)
    h = decoder(params, lora, CFG, cids, cpos, mask, region)
    _, clean = layout.extract_uno_regions(h, region, L)
    causal = torch.tril(torch.ones(L, L, dtype=torch.bool))[None].expand(2, -1, -1)
    plain = decoder(params, {}, CFG, ids, pos, causal, None)
    assert (clean - plain).abs().max().item() < 1e-5
