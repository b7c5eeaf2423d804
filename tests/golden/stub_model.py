"""A deterministic stand-in 'looped LM' for scheduler traces (no tensors).

It implements the batch union API (prefill / prelude_union / advance_union /
coda_argmax_union) that a fixed-batch WFD scheduler drives, with a Markov
next-token rule: the full-depth (step == T_total) prediction for position
p + 1 is a hash of (seq, p, token at p), and the shallow draft
(step < T_total) agrees with it unless a second hash says otherwise
(about `agree_pct` percent agreement). Nothing here depends on which
scheduler calls it, so the reference scheduler and this repo's schedulers
see the same model and must produce the same traces.
"""
from __future__ import annotations

import torch

MASK64 = (1 << 64) - 1


def mix(*xs: int) -> int:
    """splitmix64 over a tuple of ints."""
    h = 0x9E3779B97F4A7C15
    for x in xs:
        h = (h ^ (x & MASK64)) & MASK64
        h = (h + 0x9E3779B97F4A7C15) & MASK64
        z = h
        z = ((z ^ (z >> 30)) * 0xBF58476D1CE4E5B9) & MASK64
        z = ((z ^ (z >> 27)) * 0x94D049BB133111EB) & MASK64
        h = z ^ (z >> 31)
    return h


class StubCache:
    def __init__(self, B: int):
        self.B = B
        self.seqlen = [[0] * B]
        self.drops: list[tuple[int, int]] = []

    @property
    def nbytes(self) -> int:
        return 0

    def drop_positions_at_and_after(self, b: int, position: int) -> None:
        self.drops.append((int(b), int(position)))


class StubBatchBlocks:
    def __init__(self, T_total: int, B: int, vocab: int = 50, agree_pct: int = 70, salt: int = 0):
        self.T_total = T_total
        self.B = B
        self.vocab = vocab
        self.agree_pct = agree_pct
        self.salt = salt
        self.calls: list[tuple] = []       # (kind, [(seq, pos, step), ...]) in call order
        self.last_cache: StubCache | None = None

    def full(self, b: int, pos: int, tok: int) -> int:
        return mix(self.salt, 1, b, pos, tok) % self.vocab

    def shallow(self, b: int, pos: int, tok: int) -> int:
        f = self.full(b, pos, tok)
        if mix(self.salt, 2, b, pos, tok) % 100 < self.agree_pct:
            return f
        return (f + 1 + mix(self.salt, 3, b, pos, tok) % (self.vocab - 1)) % self.vocab

    def prefill(self, prompt_ids):
        rows = [torch.as_tensor(r).reshape(-1).tolist() for r in prompt_ids]
        logits = torch.zeros(len(rows), self.vocab)
        for b, r in enumerate(rows):
            logits[b, self.full(b, len(r) - 1, r[-1])] = 1.0
        self.last_cache = StubCache(len(rows))
        return self.last_cache, logits

    def prelude_union(self, seq_ids, toks, cache) -> None:
        self.calls.append(("P", [(int(b), t.position, 0) for b, t in zip(seq_ids, toks)]))
        for t in toks:
            t.hidden = ("h", t.token_id)
            t.static_state = ("e", t.token_id)
            t.step = 0

    def advance_union(self, seq_ids, toks, cache) -> None:
        self.calls.append(("R", [(int(b), t.position, t.step) for b, t in zip(seq_ids, toks)]))
        for t in toks:
            t.step += 1

    def coda_argmax_union(self, seq_ids, toks, cache) -> list[int]:
        self.calls.append(("C", [(int(b), t.position, t.step) for b, t in zip(seq_ids, toks)]))
        return [self.full(b, t.position, t.token_id) if t.step == self.T_total
                else self.shallow(b, t.position, t.token_id) for b, t in zip(seq_ids, toks)]


def stub_prompts(B: int, L: int, vocab: int = 50, salt: int = 0) -> torch.Tensor:
    return torch.tensor([[mix(salt, 9, b, i) % vocab for i in range(L)] for b in range(B)], dtype=torch.long)


def trace_record(bt, blocks: StubBatchBlocks, cache: StubCache | None, emus) -> dict:
    """Everything a batch trace pins: tokens, counters, union sizes, rollbacks,
    the per-call (seq, pos, step) schedule and the emulated draws."""
    per = [{"tokens": list(t.tokens), "n_r_calls": t.n_r_calls, "n_p_calls": t.n_p_calls,
            "n_c_calls": t.n_c_calls, "n_drafts_proposed": t.n_drafts_proposed,
            "n_drafts_accepted": t.n_drafts_accepted, "n_drafts_rejected": t.n_drafts_rejected,
            "n_rollback_events": t.n_rollback_events} for t in bt.per_seq]
    return {
        "per_seq": per,
        "n_r_calls": bt.n_r_calls, "n_p_calls": bt.n_p_calls, "n_c_calls": bt.n_c_calls,
        "r_union_total": bt.r_union_total, "r_union_max": bt.r_union_max,
        "drops": [list(d) for d in cache.drops] if cache is not None else [],
        "calls": [[k, [list(x) for x in rows]] for k, rows in blocks.calls],
        "emu": [[e.n_draws, e.n_accepts] for e in emus] if emus else None,
    }
