"""Wave bookkeeping: tokens in flight and the single-sequence wave state.

Mirrors the reference's ActiveToken / WavefrontState
(src/decoding/state.py:20-109) with one change: a token's recurrent hidden
and static (prelude) state live on the device in the engine's wave-state
pool at row `row`, not in per-token tensors, so the block calls never stack
or split per-token hiddens on the host.
"""
from __future__ import annotations

from dataclasses import dataclass, field
from typing import Literal, Optional

Role = Literal["verify", "draft"]


@dataclass(slots=True)
class ActiveToken:
    """One token progressing through the recurrent core.

    role: tokens enter as "draft"; the R pass promotes a token to "verify"
    when it reaches its commit point (step == T_total). step counts the R
    passes applied so far. row is the wave-state pool row holding
    [hidden | static_state] (set by the P pass; -1 before it).
    """

    token_id: int
    position: int
    role: Role
    step: int = 0
    row: int = -1
    is_alive: bool = True
    hidden: Optional[object] = None         # optional host handle; the state lives at `row`
    static_state: Optional[object] = None
    draft_probs: Optional[object] = None    # temperature sampling is out of scope (greedy only)
    should_exit: bool = False               # adaptive early exit is out of scope: always False


@dataclass
class WavefrontState:
    """Mutable state of one single-sequence generation
    (src/decoding/state.py:79-109)."""

    active: list[ActiveToken] = field(default_factory=list)
    committed: list[int] = field(default_factory=list)
    prefix_len: int = 0
    kv_cache: object = None
    T_total: int = 8
    T_draft: int = 2
    last_committed_position: int = -1
    active_p: list[ActiveToken] = field(default_factory=list)
    active_r: list[ActiveToken] = field(default_factory=list)
    active_c: list[ActiveToken] = field(default_factory=list)

    def find_active_prc(self, position: int) -> Optional[ActiveToken]:
        """First alive token at `position` in active_r, then active_p, then active_c."""
        for lst in (self.active_r, self.active_p, self.active_c):
            for t in lst:
                if t.is_alive and t.position == position:
                    return t
        return None

    def rollback_prc(self, position: int) -> None:
        """Drop every queued / in-flight token at position >= `position` and
        truncate the slot caches there (reject)."""
        keep = lambda lst: [t for t in lst if t.position < position]  # noqa: E731
        self.active_p, self.active_r, self.active_c = keep(self.active_p), keep(self.active_r), keep(self.active_c)
        if self.kv_cache is not None:
            self.kv_cache.drop_positions_at_and_after(position)
