"""uno_amd: MI355X-native conditional-LoRA block-diffusion training step (Uno)."""
__version__ = "0.1.0"
