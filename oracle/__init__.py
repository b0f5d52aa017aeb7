"""CPU oracle of Uno's conditional-LoRA block-diffusion training step.

TEST INFRASTRUCTURE ONLY. This package is the parity reference: a plain restatement of the
reference algorithm (fp32 PyTorch on the CPU, numpy for the integer hashing). Only the
test-suite, ``__graft_entry__.smoke()`` and the CPU-baseline leg of ``bench.py`` may import
it, and only to check or to time the reference algorithm -- never as the product path.

Modules and the reference code each one restates:
  hashing  -- counter-based splitmix64 draws (finaliser of nano_vllm_uno/engine/noise.py:43-50)
  layout   -- training/modeling.py:65-113, training/losses.py:9-18
  bd       -- the block-diffusion noising/concatenation/mask contract that the remote
              ``prepare_for_bd_training`` provides (call site training/trainer.py:198-209)
  model    -- the Qwen3 decoder (transformers/models/qwen3/modeling_qwen3.py) with PEFT LoRA
              gated per token (training/lora.py:164-174), one 2L pass with a dense mask
  losses   -- training/losses.py:21-183, training/trainer.py:223-287
  step     -- training/trainer.py:174-308 + clip/AdamW of training/train.py:282-288

Pinning status of each function is stated in its docstring and checked by tests/test_oracle_*.
"""
