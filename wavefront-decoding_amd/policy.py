"""WFD schedule policy (src/decoding/policy.py:16-59): verify depth T_total,
draft depth T_draft; W = T_total // T_draft tokens in flight at steady state.
Greedy (lossless) decoding only -- temperature speculative sampling is out
of scope for this build."""
from __future__ import annotations

import warnings
from dataclasses import dataclass


@dataclass
class SsdPolicy:
    T_total: int = 8
    T_draft: int = 2
    mode: str = "greedy"
    temperature: float = 1.0
    sample_seed: int = 0

    def __post_init__(self) -> None:
        if self.T_draft < 1 or self.T_total < self.T_draft:
            raise ValueError(f"SsdPolicy: the draft depth must lie in [1, T_total] "
                             f"(T_total={self.T_total}, T_draft={self.T_draft})")
        if self.mode != "greedy":
            raise ValueError(f"Unsupported sampling mode {self.mode!r}: this build decodes greedily (lossless).")
        if self.T_total % self.T_draft:
            warnings.warn(f"SsdPolicy: T_draft={self.T_draft} does not divide T_total={self.T_total}, so the "
                          "number of tokens in flight varies from tick to tick", stacklevel=2)

    @property
    def steady_state_active_size(self) -> int:
        return self.T_total // self.T_draft

    def make_sampler(self):
        from .acceptance import TokenSampler

        return TokenSampler()
