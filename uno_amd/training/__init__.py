"""Drop-in counterpart of the reference's ``training`` package for the Uno step.

Module and function names, signatures and error behaviour follow the reference
(training/trainer.py, modeling.py, lora.py, losses.py, config.py, constants.py, curriculum.py,
data.py, checkpointing.py); the compute underneath runs on the uno_amd HIP kernels.
"""
