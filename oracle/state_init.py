"""Initial loop state s0 (src/decoding/parcae_blocks.py:129-156).

Per decode token: trunc_normal(mean 0, std, bounds +-3 std) drawn from a CPU
torch.Generator seeded (state_seed * 1_000_003 + position + 1) & (2**47 - 1),
times emb_scale. The prompt uses one stream seeded state_seed * 1_000_003 for
the whole (1, L, D) block. The distribution itself is torch's
nn.init.trunc_normal_ (a library routine), so s0 is pinned by torch.
"""
from __future__ import annotations

import numpy as np
import torch


def _draw(shape, seed: int, std: float) -> torch.Tensor:
    out = torch.empty(shape, dtype=torch.float32)
    g = torch.Generator()
    g.manual_seed(seed & 0x7FFF_FFFF_FFFF)
    torch.nn.init.trunc_normal_(out, mean=0.0, std=std, a=-3 * std, b=3 * std, generator=g)
    return out


def s0_token(d_model: int, std: float, scale: float, state_seed: int, position: int) -> np.ndarray:
    return (_draw((d_model,), state_seed * 1_000_003 + position + 1, std) * scale).numpy()


def s0_prefill(d_model: int, std: float, scale: float, state_seed: int, length: int) -> np.ndarray:
    return (_draw((1, length, d_model), state_seed * 1_000_003, std)[0] * scale).numpy()
