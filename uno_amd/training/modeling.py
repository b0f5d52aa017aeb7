"""Uno layout glue (semantics of training/modeling.py:9-147 in the reference)."""
from __future__ import annotations

import sys
from types import MethodType

import torch

from ..layers import GatherRows


def unwrap_base_model(model):
    while hasattr(model, "module"):
        model = model.module
    return model.get_base_model() if hasattr(model, "get_base_model") else model


def validate_uno_model(model) -> None:
    base = unwrap_base_model(model)
    missing = [n for n in ("prepare_for_bd_training", "model", "lm_head") if not hasattr(base, n)]
    if missing:
        raise RuntimeError("The selected model is not the Uno-prepared Qwen3 model. Missing required "
                           f"interface member(s): {missing}.")
    _get_sdar_helpers(base)
    if not hasattr(base.config, "block_size"):
        raise RuntimeError("The Uno model config must define block_size.")


def configure_uniform_noise_config(config):
    noise = getattr(config, "noise", None)
    if noise not in (None, "uniform"):
        raise RuntimeError(f"Public Uno training requires uniform noise, but the model config declares noise={noise!r}.")
    config.noise = "uniform"
    return config


def configure_uniform_noise(model) -> None:
    base = unwrap_base_model(model)
    validate_uno_model(base)
    base.noise = "uniform"
    configure_uniform_noise_config(base.config)


def _get_sdar_helpers(base_model):
    module = sys.modules.get(base_model.__class__.__module__)
    if module is None:
        raise RuntimeError(f"Could not resolve modeling module for {base_model.__class__.__name__}.")
    modify = getattr(module, "modify_padded_position_ids_2d", None)
    counts = getattr(module, "calculate_token_nums", None)
    if modify is None or counts is None:
        raise RuntimeError("The Uno model module must provide modify_padded_position_ids_2d and calculate_token_nums.")
    return modify, counts


def _build_noisy_region_mask(num_tokens: list[torch.Tensor], sequence_length: int) -> torch.Tensor:
    rows = []
    for lengths in num_tokens:
        pieces = []
        for n in lengths.tolist():
            pieces.append(torch.ones(n, dtype=torch.bool, device=lengths.device))
            pieces.append(torch.zeros(n, dtype=torch.bool, device=lengths.device))
        row = torch.cat(pieces)
        if row.numel() != 2 * sequence_length:
            raise RuntimeError(f"Uno noisy/clean layout has an invalid length: {row.numel()} for "
                               f"sequence_length={sequence_length}.")
        rows.append(row)
    return torch.stack(rows)


def prepare_uno_layout(base_model, input_ids: torch.Tensor, position_ids: torch.Tensor | None):
    batch, length = input_ids.shape
    if position_ids is None:
        position_ids = torch.arange(length, device=input_ids.device).unsqueeze(0).expand(batch, -1)
    modify, counts = _get_sdar_helpers(base_model)
    model_positions = modify(position_ids)
    region = _build_noisy_region_mask(counts(model_positions), length)
    return position_ids, model_positions, region


def extract_uno_regions(hidden_states: torch.Tensor, noisy_region_mask: torch.Tensor, sequence_length: int):
    """Noisy and clean rows in original token order, each [B, L, H] (row gathers on the GPU)."""
    b, two_l, h = hidden_states.shape
    flat = hidden_states.reshape(b * two_l, h)
    mask = noisy_region_mask.reshape(-1).to(flat.device)
    noisy_idx = torch.nonzero(mask).flatten().to(torch.int32)
    clean_idx = torch.nonzero(~mask).flatten().to(torch.int32)
    if noisy_idx.numel() != b * sequence_length or clean_idx.numel() != b * sequence_length:
        raise RuntimeError("shape mismatch: the noisy region does not hold sequence_length rows per batch row")
    if flat.is_cuda:
        noisy = GatherRows.apply(flat, noisy_idx)
        clean = GatherRows.apply(flat, clean_idx)
    else:
        noisy, clean = flat[noisy_idx.long()], flat[clean_idx.long()]
    return noisy.view(b, sequence_length, h), clean.view(b, sequence_length, h)


def run_prepared_uno_forward(model, base_model, inputs, concatenated_input_ids, concatenated_position_ids,
                             flex_attention_mask) -> torch.Tensor:
    """Runs the paired noisy/clean layout through the wrappers in one decoder call."""
    decoder = getattr(base_model, "model", None)
    if decoder is None:
        raise RuntimeError("The Uno model must expose its decoder as .model.")
    original = base_model.forward

    def prepared_forward(self, *args, **kwargs):
        del self, args, kwargs
        out = decoder(input_ids=concatenated_input_ids, attention_mask=flex_attention_mask,
                      position_ids=concatenated_position_ids, output_attentions=False,
                      output_hidden_states=False, return_dict=True, use_cache=False)
        return {"hidden_states": (out.last_hidden_state,)}

    base_model.forward = MethodType(prepared_forward, base_model)
    try:
        outputs = model(**inputs, output_hidden_states=True)
    finally:
        base_model.forward = original
    return outputs["hidden_states"][-1]
