"""Single-sequence schedulers with emulated acceptance
(src/decoding/scheduler_emu.py:33-155 generate_wavefront_emu, :156-290
generate_dtv_emu): the WFD and draft-then-verify loops of scheduler.py with
every accept decision taken from an `EmulatedAcceptance` stream instead of the
greedy comparison. All compute (P, R, C, argmax, appends, rollbacks) still
runs, so the timing is that of the real pipeline; with emu=None they are the
greedy schedulers exactly (the reference's equivalence gate,
experiments/exp4_emu/verify_step1.py:55-71).
"""
from __future__ import annotations

import torch

from .emu import EmulatedAcceptance
from .policy import SsdPolicy
from .scheduler import GenerationTrace, dtv_single, wavefront_single


@torch.no_grad()
def generate_wavefront_emu(blocks, prompt_ids: torch.Tensor, max_new_tokens: int, policy: SsdPolicy,
                           emu: EmulatedAcceptance | None = None, eos_token_id: int | None = None
                           ) -> tuple[list[int], GenerationTrace]:
    """generate_wavefront_dynamic with each draft's accept decided by emu.draw()."""
    return wavefront_single(blocks, prompt_ids, max_new_tokens, policy, emu, eos_token_id)


@torch.no_grad()
def generate_dtv_emu(blocks, prompt_ids: torch.Tensor, max_new_tokens: int, policy: SsdPolicy, draft_length: int,
                     emu: EmulatedAcceptance | None = None, eos_token_id: int | None = None
                     ) -> tuple[list[int], GenerationTrace]:
    """generate_draft_then_verify with each draft's accept decided by emu.draw()."""
    return dtv_single(blocks, prompt_ids, max_new_tokens, policy, draft_length, emu, eos_token_id)
