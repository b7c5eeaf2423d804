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

import copy

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


class StubSingleCache:
    """Single-sequence cache stand-in: a rollback at `position` is recorded as
    (0, position) on the batch stub's cache."""

    def __init__(self, inner: StubCache):
        self.inner = inner

    def drop_positions_at_and_after(self, position: int) -> None:
        self.inner.drop_positions_at_and_after(0, position)


class _Seed:
    """What the stub's prelude fills for one token (prelude_forward's row)."""

    def __init__(self, token_id: int, position: int):
        self.token_id = token_id
        self.position = position


class StubRecursiveBlocks:
    """The single-sequence block interface a dynamic WFD scheduler drives
    (prefill, P_dyn, R_dyn, C_multi_dyn; prelude_forward, advance_one_step,
    coda_logits for draft-then-verify) over the stub model at B = 1, with
    the routing that interface documents (src/decoding/blocks.py:46-66):
    R advances every alive active_r token one step; the position-ordered
    prefix of tokens at step == T_total is promoted to "verify" and moved to
    active_c; a token at step == T_draft is copied there as "draft". C returns
    one-hot logits (verifies in position order, then the draft).

    Mixed into a scheduler's own abstract blocks class: `state_cls` is that
    scheduler's WavefrontState."""

    state_cls = None

    def __init__(self, T_total: int, agree_pct: int = 70):
        self.stub = StubBatchBlocks(T_total, 1, agree_pct=agree_pct)
        self.T_total = T_total

    def _onehot(self, tok: int) -> torch.Tensor:
        v = torch.zeros(self.stub.vocab)
        v[tok] = 1.0
        return v

    def prefill(self, input_ids, T_total, T_draft):
        ids = torch.as_tensor(input_ids).reshape(-1)
        cache, logits = self.stub.prefill([ids])
        state = self.state_cls(prefix_len=len(ids), kv_cache=StubSingleCache(cache), T_total=T_total,
                               T_draft=T_draft, last_committed_position=len(ids) - 1)
        return state, logits[0]

    def P_dyn(self, state):
        if state.active_p:
            self.stub.prelude_union([0] * len(state.active_p), state.active_p, state.kv_cache)
        state.active_r.extend(state.active_p)
        state.active_p = []
        return state, True

    def R_dyn(self, state):
        toks = [t for t in state.active_r if t.is_alive]
        if toks:
            self.stub.advance_union([0] * len(toks), toks, state.kv_cache)
        front = []
        for t in sorted(toks, key=lambda t: t.position):
            if t.step != state.T_total:
                break
            front.append(t)
        moved = {id(t) for t in front}
        keep, any_c = [], False
        for t in toks:
            if id(t) in moved:
                t.role = "verify"
                state.active_c.append(t)
                any_c = True
                continue
            keep.append(t)
            if t.step == state.T_draft:
                c = copy.copy(t)
                c.role = "draft"
                state.active_c.append(c)
                any_c = True
        state.active_r = keep
        return state, any_c

    def C_multi_dyn(self, state):
        verify = sorted((t for t in state.active_c if t.role == "verify"), key=lambda t: t.position)
        draft = [t for t in state.active_c if t.role == "draft"]
        rows = verify + draft
        if not rows:
            return state, 0, []
        ids = self.stub.coda_argmax_union([0] * len(rows), rows, state.kv_cache)
        return state, len(verify), [self._onehot(i) for i in ids]

    def ar_generate(self, prompt_ids, max_new_tokens, eos_token_id=None, sampler=None):
        raise NotImplementedError("the stub model serves the WFD and draft-then-verify schedulers only")

    def prelude_forward(self, cache, token_id: int, position: int):
        row = _Seed(token_id, position)
        self.stub.prelude_union([0], [row], cache)
        return row.hidden, row.static_state

    def advance_one_step(self, toks, cache) -> None:
        if toks:
            self.stub.advance_union([0] * len(toks), toks, cache)

    def coda_logits(self, state, toks):
        return [self._onehot(i) for i in self.stub.coda_argmax_union([0] * len(toks), toks, None)]


def single_record(tokens, trace, blocks: StubRecursiveBlocks, emu, keep_calls: bool) -> dict:
    """What a single-sequence trace pins: tokens, counters, rollbacks, the
    per-call (pos, step) schedule (short runs) and the emulated draws."""
    cache = blocks.stub.last_cache
    return {
        "tokens": list(tokens),
        "counters": {k: getattr(trace, k) for k in ("n_r_calls", "n_p_calls", "n_c_calls", "n_drafts_proposed",
                                                    "n_drafts_accepted", "n_drafts_rejected", "n_rollback_events")},
        "drops": [list(d) for d in cache.drops] if cache is not None else [],
        "calls": [[k, [list(x) for x in rows]] for k, rows in blocks.stub.calls] if keep_calls else None,
        "emu": [emu.n_draws, emu.n_accepts] if emu is not None else None,
    }
