"""Emulated acceptance (src/decoding/emu.py:19-43): every draft/verify
decision becomes an independent Bernoulli(rate) draw from a seeded
`random.Random` stream, one stream per sequence; all compute still runs."""
from __future__ import annotations

import random


class EmulatedAcceptance:
    def __init__(self, rate: float, seed: int = 0):
        if not 0.0 <= rate <= 1.0:
            raise AssertionError(f"EmulatedAcceptance: rate {rate} is not a probability (0 <= rate <= 1)")
        self.rate = float(rate)
        self.seed = seed
        self.rng = random.Random(seed)
        self.n_draws = 0
        self.n_accepts = 0

    def draw(self) -> bool:
        self.n_draws += 1
        ok = self.rng.random() < self.rate
        self.n_accepts += int(ok)
        return ok

    @property
    def empirical_rate(self) -> float:
        return self.n_accepts / self.n_draws if self.n_draws else float("nan")
