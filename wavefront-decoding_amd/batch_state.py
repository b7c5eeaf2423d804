"""One sequence's lane inside a fixed batch.

A `Lane` is what the batch schedulers keep per sequence: the committed
tokens, the acceptance source (an EmulatedAcceptance stream, or None for the
real argmax comparison), the per-sequence GenerationTrace, and the working
state of whichever scheduler drives it:

* wavefront decoding: `queued` (tokens that enter the wave at the next
  tick's P pass) and `flight` (tokens inside the recurrent core, in position
  order -- a sequence has at most one live token per position);
* draft-then-verify: one `DtvRound` at a time.

The reference keeps the same information in src/decoding/batch_state.py:24-75;
the layout here is this build's own: the wave is position-ordered, so the
token at a position is found by a scan of one list, a reject truncates it
with one cut, and a round's next source is derived from the round itself.
"""
from __future__ import annotations

from dataclasses import dataclass, field
from typing import Optional

from .emu import EmulatedAcceptance
from .scheduler import GenerationTrace
from .state import ActiveToken


@dataclass
class DtvRound:
    """A draft-then-verify round started from the last committed token
    (`base_tok` at `base_pos`). Source j sits at base_pos + j; its token is
    base_tok for j = 0 and draft j - 1 afterwards. `stage`: "embed" (the next
    source needs its P pass), "shallow" (the newest source runs depths
    0..T_draft), "deep" (all k + 1 sources run on to T_total)."""

    base_tok: int
    base_pos: int
    k: int
    sources: list[ActiveToken] = field(default_factory=list)
    drafts: list[int] = field(default_factory=list)
    stage: str = "embed"

    def next_source(self) -> ActiveToken:
        j = len(self.sources)
        tok = self.base_tok if j == 0 else self.drafts[j - 1]
        src = ActiveToken(token_id=tok, position=self.base_pos + j, role="verify")
        self.sources.append(src)
        self.stage = "shallow"
        return src

    def take_shallow(self, token: int) -> None:
        """The newest source's shallow argmax: the draft for the next position
        (the last source's is not needed); then embed the next source or go deep."""
        if len(self.sources) <= self.k:
            self.drafts.append(token)
        self.stage = "embed" if len(self.sources) <= self.k else "deep"


@dataclass
class Lane:
    index: int                              # batch index b (the cache's sequence)
    prompt_len: int
    limit: int                              # max new tokens of this sequence
    emu: Optional[EmulatedAcceptance] = None
    trace: GenerationTrace = field(default_factory=GenerationTrace)
    committed: list[int] = field(default_factory=list)
    done: bool = False
    queued: list[ActiveToken] = field(default_factory=list)
    flight: list[ActiveToken] = field(default_factory=list)
    round: Optional[DtvRound] = None

    # -- committing ------------------------------------------------------------
    def commit(self, token: int) -> bool:
        """Append a committed token; True once the sequence reached its limit."""
        self.committed.append(token)
        self.trace.tokens.append(token)
        self.done = len(self.committed) >= self.limit
        return self.done

    @property
    def next_position(self) -> int:
        """Position of the token after the last committed one."""
        return self.prompt_len + len(self.committed)

    def accepts(self, gold: int, draft: int) -> bool:
        """The verify decision: the emulated draw when the lane has a stream,
        else the lossless top-1 comparison."""
        return self.emu.draw() if self.emu is not None else gold == draft

    # -- wavefront decoding --------------------------------------------------------
    def enqueue(self, token: int, position: int) -> None:
        self.queued.append(ActiveToken(token_id=token, position=position, role="draft"))
        self.trace.n_p_calls += 1

    def token_at(self, position: int) -> Optional[ActiveToken]:
        """The live token speculated at `position` (in the wave, else queued)."""
        for t in self.flight:
            if t.position == position:
                return t
        for t in self.queued:
            if t.position == position:
                return t
        return None

    def truncate_from(self, position: int, cache) -> None:
        """Reject at `position`: forget this sequence's tokens from there on and
        its slot rows at or after it; other sequences are untouched."""
        self.flight = [t for t in self.flight if t.position < position]
        self.queued = [t for t in self.queued if t.position < position]
        cache.drop_positions_at_and_after(self.index, position)

    def retire(self) -> None:
        """The sequence is finished: it contributes nothing to later passes."""
        self.queued, self.flight, self.round = [], [], None
