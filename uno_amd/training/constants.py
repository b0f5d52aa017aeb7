"""Fixed values of the public Uno recipe (training/constants.py of the reference)."""

DEFAULT_MODEL_ID = "s-sahoo/uno-qwen3-8B"
DEFAULT_MODEL_REVISION = "b8a7577b3223bdcf2b3af0f2fc6e95258b3bbc29"

IGNORE_INDEX = -100
COLLATED_SEQUENCE_LENGTH = 4096
DEFAULT_SEED = 20260813

DEFAULT_LEARNING_RATE = 1.0e-5
DEFAULT_CE_ALPHA = 0.0
DEFAULT_KL_BETA = 0.0
DEFAULT_TV_GAMMA = 1.0

DEFAULT_LORA_RANK = 128
DEFAULT_LORA_ALPHA_RATIO = 16
DEFAULT_LORA_DROPOUT = 0.0

SUPPORTED_LORA_MODULES = ("q_proj", "k_proj", "v_proj", "o_proj", "gate_proj", "up_proj", "down_proj")
