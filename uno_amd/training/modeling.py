"""Layout glue of the Uno step over the two-stream MI355X decoder.

Keeps the call surface of the reference's training/modeling.py (names, arguments, return values,
error types), with its own mechanics:

* ``prepare_uno_layout`` (training/modeling.py:84-98) takes the model positions from the model
  module's ``modify_padded_position_ids_2d`` and builds the [noisy | clean] region mask on the
  device (``uno_amd.model.noisy_region_mask``: one kernel, no per-segment host loop, no host
  synchronisation). Segments follow the model module's ``calculate_token_nums`` rule: one starts at
  t = 0 and wherever the position does not increase.
* ``extract_uno_regions`` (training/modeling.py:101-113) returns the decoder's own stream tensors
  when it is handed the hidden states the two-stream decoder produced for the same region mask
  (the rows are the same values, and the gradient reaches the decoder without a scatter and a
  re-gather); any other tensor is split by device row gathers.
* ``run_prepared_uno_forward`` (training/modeling.py:116-147) hands the prepared batch to the base
  model through ``stage_prepared_batch`` (a context manager of the model, no method patching) and
  runs the caller's wrapper stack once, so every wrapper's forward hooks see the call.
"""
from __future__ import annotations

import sys

import torch

from ..layers import GatherRows

REQUIRED_MEMBERS = ("prepare_for_bd_training", "model", "lm_head")
POSITION_HELPERS = ("modify_padded_position_ids_2d", "calculate_token_nums")


def unwrap_base_model(model):
    """The base causal LM under data-parallel wrappers (``.module``) and the adapter wrapper
    (``get_base_model``)."""
    inner = model
    while getattr(inner, "module", None) is not None:
        inner = inner.module
    getter = getattr(inner, "get_base_model", None)
    return getter() if callable(getter) else inner


def _model_module(base_model):
    return sys.modules.get(type(base_model).__module__)


def validate_uno_model(model) -> None:
    """Raises RuntimeError naming everything the base model lacks for the Uno step."""
    base = unwrap_base_model(model)
    problems = [f"member {name!r}" for name in REQUIRED_MEMBERS if not hasattr(base, name)]
    module = _model_module(base)
    if module is None:
        problems.append(f"an importable modeling module for {type(base).__name__}")
    else:
        problems += [f"module-level {name}()" for name in POSITION_HELPERS
                     if not callable(getattr(module, name, None))]
    if not hasattr(getattr(base, "config", None), "block_size"):
        problems.append("config.block_size")
    if problems:
        raise RuntimeError(f"{type(base).__name__} is not a Uno-prepared Qwen3 model; it lacks: "
                           + ", ".join(problems) + ".")


def configure_uniform_noise_config(config):
    """Sets ``config.noise`` to uniform, the only noise public Uno training runs; a config that
    declares another mode is rejected."""
    declared = getattr(config, "noise", None)
    if declared is not None and declared != "uniform":
        raise RuntimeError(f"Uno training runs with uniform noise only; the model config declares {declared!r}.")
    config.noise = "uniform"
    return config


def configure_uniform_noise(model) -> None:
    base = unwrap_base_model(model)
    validate_uno_model(base)
    base.noise = "uniform"
    configure_uniform_noise_config(base.config)


def prepare_uno_layout(base_model, input_ids: torch.Tensor, position_ids: torch.Tensor | None):
    """Returns (position_ids, model_position_ids, noisy_region_mask [B, 2L] bool)."""
    from ..model import noisy_region_mask

    validate_uno_model(base_model)
    B, L = input_ids.shape
    if position_ids is None:
        position_ids = torch.arange(L, device=input_ids.device).expand(B, L)
    elif tuple(position_ids.shape) != (B, L):
        raise RuntimeError(f"position_ids of shape {tuple(position_ids.shape)} do not match input_ids {(B, L)}.")
    model_positions = getattr(_model_module(base_model), "modify_padded_position_ids_2d")(position_ids)
    region = noisy_region_mask(model_positions)
    remember = getattr(base_model, "remember_layout", None)
    if callable(remember):
        remember(model_positions, region)
    return position_ids, model_positions, region


def extract_uno_regions(hidden_states: torch.Tensor, noisy_region_mask: torch.Tensor, sequence_length: int):
    """Noisy and clean rows of a [B, 2L, H] hidden-state tensor, each [B, L, H] in token order."""
    b, two_l, h = hidden_states.shape
    if tuple(noisy_region_mask.shape) != (b, two_l) or two_l != 2 * sequence_length:
        raise RuntimeError(f"region mask {tuple(noisy_region_mask.shape)} does not fit hidden states "
                           f"{tuple(hidden_states.shape)} with sequence_length={sequence_length}.")
    streams = getattr(hidden_states, "_uno_streams", None)
    if streams is not None and streams[2] is noisy_region_mask:
        noisy, clean, _ = streams
        return noisy.view(b, sequence_length, h), clean.view(b, sequence_length, h)
    flat = hidden_states.reshape(b * two_l, h)
    mask = noisy_region_mask.reshape(-1).to(flat.device)
    rows = torch.argsort(~mask, stable=True).to(torch.int32)   # noisy rows first, then clean, in order
    n_noisy = b * sequence_length
    if flat.is_cuda:
        parts = GatherRows.apply(flat, rows)
    else:
        parts = flat[rows.long()]
    noisy, clean = parts[:n_noisy], parts[n_noisy:]
    if int(mask.sum()) != n_noisy:
        raise RuntimeError("the region mask does not hold sequence_length noisy rows per batch row.")
    return noisy.reshape(b, sequence_length, h), clean.reshape(b, sequence_length, h)


def run_prepared_uno_forward(model, base_model, inputs, concatenated_input_ids, concatenated_position_ids,
                             flex_attention_mask) -> torch.Tensor:
    """One pass of the caller's model stack over the prepared [noisy | clean] batch; returns the
    decoder's last hidden states [B, 2L, H]."""
    if getattr(base_model, "model", None) is None:
        raise RuntimeError("The Uno model must expose its decoder as .model.")
    stage = getattr(base_model, "stage_prepared_batch", None)
    if not callable(stage):
        raise RuntimeError(f"{type(base_model).__name__} cannot take a prepared block-diffusion batch "
                           "(no stage_prepared_batch).")
    with stage(concatenated_input_ids, concatenated_position_ids, flex_attention_mask):
        outputs = model(**inputs, output_hidden_states=True)
    return outputs["hidden_states"][-1]
