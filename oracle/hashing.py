"""Counter-based 64-bit draws for the noising contract (numpy uint64, wrapping arithmetic).

``mix64`` is the splitmix64 finaliser (Stafford "Mix13" constants), the same function as
``_mix_u64`` in nano_vllm_uno/engine/noise.py:43-50. Pinned by the published splitmix64
output sequence for seed 0 (tests/test_oracle_layout.py).
"""
from __future__ import annotations

import numpy as np

GOLDEN = np.uint64(0x9E3779B97F4A7C15)
_M1 = np.uint64(0xBF58476D1CE4E5B9)
_M2 = np.uint64(0x94D049BB133111EB)

STREAM_BLOCK_T = 1      # per-block noise level t
STREAM_TOKEN_U = 2      # per-token mask draw u
STREAM_TOKEN_ID = 3     # per-token replacement id


def mix64(x):
    x = np.asarray(x, dtype=np.uint64)
    with np.errstate(over="ignore"):
        x = (x ^ (x >> np.uint64(30))) * _M1
        x = (x ^ (x >> np.uint64(27))) * _M2
        return x ^ (x >> np.uint64(31))


def splitmix64_sequence(seed: int, n: int) -> list[int]:
    """The splitmix64 generator: state += GOLDEN; output mix64(state)."""
    out, state = [], np.uint64(seed)
    with np.errstate(over="ignore"):
        for _ in range(n):
            state = state + GOLDEN
            out.append(int(mix64(state)))
    return out


def step_key(seed: int, step: int) -> np.uint64:
    with np.errstate(over="ignore"):
        return mix64(np.uint64(seed & 0xFFFFFFFFFFFFFFFF) + GOLDEN * np.uint64(step + 1))


def draw(key, stream: int, row, index):
    """draw = mix64(mix64(mix64(key ^ stream) + row*GOLDEN) + index*GOLDEN), all mod 2^64."""
    key = np.uint64(key)
    row = np.asarray(row, dtype=np.uint64)
    index = np.asarray(index, dtype=np.uint64)
    with np.errstate(over="ignore"):
        a = mix64(key ^ np.uint64(stream))
        b = mix64(a + row * GOLDEN)
        return mix64(b + index * GOLDEN)


def unit_float(h):
    """Top 24 bits as an fp32 in [0, 1): exactly (h >> 40) * 2^-24."""
    return (np.asarray(h, dtype=np.uint64) >> np.uint64(40)).astype(np.float32) * np.float32(2.0 ** -24)


T_LO = np.float32(0.05)
T_SPAN = np.float32(0.95)


def noise_level(u):
    """t = fl32(fl32(u * 0.95f) + 0.05f): two fp32 roundings, no fused multiply-add."""
    u = np.asarray(u, dtype=np.float32)
    return (u * T_SPAN).astype(np.float32) + T_LO
