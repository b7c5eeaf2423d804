"""Per-sequence state inside a fixed batch (src/decoding/batch_state.py:24-75)."""
from __future__ import annotations

from dataclasses import dataclass, field
from typing import Optional

from .emu import EmulatedAcceptance
from .scheduler import GenerationTrace
from .state import ActiveToken


@dataclass
class SeqState:
    idx: int
    prefix_len: int
    emu: Optional[EmulatedAcceptance] = None
    max_new_tokens: int = 0
    trace: GenerationTrace = field(default_factory=GenerationTrace)
    committed: list[int] = field(default_factory=list)
    done: bool = False
    active_p: list[ActiveToken] = field(default_factory=list)
    active_r: list[ActiveToken] = field(default_factory=list)
    active_c: list[ActiveToken] = field(default_factory=list)
    # draft-then-verify round (src/decoding/batch_state.py:44-56): phase is
    # "need_p" (the next source needs its embedding), "draft" (the current
    # source runs depths 0..T_draft) or "verify" (all K+1 sources run on to
    # T_total); K drafts this round, j = index of the current source
    phase: str = "need_p"
    K: int = 0
    j: int = 0
    sources: list[ActiveToken] = field(default_factory=list)
    drafts: list[int] = field(default_factory=list)
    cur_tok: int = 0
    cur_pos: int = 0
    last_token: int = 0
    p: int = 0

    def commit(self, token_id: int) -> None:
        self.committed.append(token_id)
        self.trace.tokens.append(token_id)

    def find_active(self, position: int) -> Optional[ActiveToken]:
        for lst in (self.active_r, self.active_p, self.active_c):
            for t in lst:
                if t.is_alive and t.position == position:
                    return t
        return None

    def rollback(self, position: int, cache) -> None:
        """Drop this sequence's tokens at/after `position` and truncate its
        slot lengths; other sequences are untouched."""
        keep = lambda lst: [t for t in lst if t.position < position]  # noqa: E731
        self.active_p, self.active_r, self.active_c = keep(self.active_p), keep(self.active_r), keep(self.active_c)
        cache.drop_positions_at_and_after(self.idx, position)

    def clear_working_state(self) -> None:
        self.active_p, self.active_r, self.active_c = [], [], []
        self.sources, self.drafts = [], []
        self.phase = "idle"
