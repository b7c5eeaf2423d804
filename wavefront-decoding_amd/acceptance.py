"""Greedy sampling and draft acceptance (src/decoding/acceptance.py:40-58).

A committed token is argmax of the full-depth logits; a draft is accepted iff
it equals that argmax (lossless top-1), otherwise the argmax is committed
instead. Logits may arrive as a tensor or as a `RowLogits`, which carries the
argmax already computed on the device, so a whole coda union costs one
device->host read.
"""
from __future__ import annotations

from dataclasses import dataclass

import torch


@dataclass
class RowLogits:
    """One row of coda logits with its device-computed argmax."""

    values: torch.Tensor   # (V,) float32 (device view)
    token: int             # argmax (first index on ties)

    def argmax(self, dim: int = -1):
        return torch.tensor(self.token)


def greedy_sample(logits) -> int:
    if isinstance(logits, RowLogits):
        return logits.token
    if logits.dim() > 1:
        logits = logits.reshape(-1)
    return int(logits.argmax(dim=-1).item())


def greedy_accept(draft_token: int, verify_logits) -> tuple[bool, int]:
    target = greedy_sample(verify_logits)
    return draft_token == target, target


class TokenSampler:
    """The sampler every decode path shares so AR and WFD emit the same
    token for the same (position, logits). Greedy only."""

    temperature = 0.0

    def __call__(self, logits, position: int) -> int:
        return greedy_sample(logits)

    def draft(self, logits, position: int):
        return greedy_sample(logits), None

    def verify(self, draft_token: int, draft_probs, verify_logits, position: int) -> tuple[bool, int]:
        return greedy_accept(draft_token, verify_logits)


GREEDY = TokenSampler()
