"""Activation recompute of the noisy stream (counterpart of training/checkpointing.py).

The reference checkpoints every decoder layer that holds LoRA weights (reentrant
torch.utils.checkpoint, training/checkpointing.py:12-52): each layer keeps only its input and
reruns its forward in the backward, over all 2L rows. Here only the noisy stream has a backward
(the clean stream runs forward-only and keeps its K/V), and the policy is per layer:

* ``recompute=True``: every noisy-stream layer keeps only its input (the reference's policy);
* ``recompute=False``: every layer keeps its activations (no recompute work);
* ``recompute="auto"`` (default): activations are kept for as many layers as fit in the HBM
  budget (``hbm_budget_bytes``, or the free HBM at forward time minus ``reserve_bytes``) and the
  remaining layers, spread over the depth, recompute. At the Qwen3-8B shape with 4 x 4096 tokens
  the activations (about 81 GB) fit in 288 GB and nothing recomputes; larger micro-batches trade
  compute for memory instead of failing.

The recomputed forward is the same deterministic kernel sequence, so gradients are bit-identical
with and without recompute.
"""
from __future__ import annotations

from .modeling import unwrap_base_model


def configure_gradient_checkpointing(model, recompute: bool | str = "auto", *, hbm_budget_bytes: int | None = None,
                                     reserve_bytes: int | None = None) -> None:
    if recompute not in (True, False, "auto"):
        raise ValueError(f"recompute must be True, False or 'auto', got {recompute!r}")
    base = unwrap_base_model(model)
    decoder = getattr(base, "model", None)
    if decoder is None or not hasattr(decoder, "recompute_plan"):
        raise RuntimeError("configure_gradient_checkpointing needs the Uno decoder (base_model.model).")
    decoder.recompute = recompute
    decoder.recompute_budget_bytes = hbm_budget_bytes
    if reserve_bytes is not None:
        decoder.recompute_reserve_bytes = int(reserve_bytes)
    base.config.use_cache = False
    base.gradient_checkpointing = recompute is not False
