"""Fixed-batch schedulers: sequential looped decode (AR), wavefront decoding
(WFD) and draft-then-verify (DtV), each over one shared slot cache
(behaviour of src/decoding/scheduler_batch.py:36-505).

A fixed batch of B sequences (lanes): a finished lane idles (no refill).
Every tick runs P, R and C once over the union of what every live lane
needs -- one launch sequence, one graph replay when the blocks fuse passes
(`run_passes`) -- and then each lane settles on its own: accept/reject comes
from its EmulatedAcceptance stream when it has one (Bernoulli(alpha)), else
from the real argmax comparison, and a reject rolls back only that lane.

Extensions over the reference (its behaviour is the default): prompts may
have different lengths (a list of 1-D id sequences; the reference needs
equal lengths, huginn_blocks_batch.py:180-185), and max_new_tokens may be a
per-sequence list (the reference takes one value, scheduler_batch.py:348-349).
Sampled ids stay on the device as token handles, read back once at the end,
whenever nothing on the host needs their values: emulated decisions, AR, and
greedy WFD on blocks that compare the argmaxes on the device (then a tick
reads back one accept flag per C row instead of the ids).
"""
from __future__ import annotations

import time
from dataclasses import dataclass, field

import torch

from .batch_state import DtvRound, Lane
from .policy import SsdPolicy
from .state import ActiveToken


def _rate(n: float, seconds: float) -> float:
    return n / seconds if seconds > 0 else float("nan")


@dataclass
class BatchTrace:
    """Whole-batch counters (field names as in the reference's trace)."""

    walltime_s: float = 0.0
    prefill_s: float = 0.0
    n_r_calls: int = 0
    n_p_calls: int = 0
    n_c_calls: int = 0
    r_union_total: int = 0
    r_union_max: int = 0
    peak_alloc_gb: float = 0.0
    peak_reserved_gb: float = 0.0
    cache_gb: float = 0.0
    per_seq: list = field(default_factory=list)

    def count_r(self, rows: int) -> None:
        self.n_r_calls += 1
        self.r_union_total += rows
        self.r_union_max = max(self.r_union_max, rows)

    n_tokens = property(lambda self: sum(len(t.tokens) for t in self.per_seq))
    walltime_decode_s = property(lambda self: max(self.walltime_s - self.prefill_s, 0.0))
    tokens_per_s = property(lambda self: _rate(self.n_tokens, self.walltime_s))
    decode_tokens_per_s = property(lambda self: _rate(self.n_tokens, self.walltime_decode_s))
    r_union_mean = property(lambda self: self.r_union_total / self.n_r_calls if self.n_r_calls else 0.0)

    @property
    def acceptance_rate(self) -> float:
        prop = sum(t.n_drafts_proposed for t in self.per_seq)
        return sum(t.n_drafts_accepted for t in self.per_seq) / prop if prop else float("nan")


@dataclass
class SharedPrefill:
    """One prompt prefill reused by several decode runs. Decode writes only
    positions at or past each prompt's length, so the prompt rows stay valid
    and a run only needs the logical slot lengths rewound."""

    cache: object
    first_tokens: list[int]
    prefill_s: float
    prompt_lens: list[int]
    lengths: list = field(default_factory=list)

    def restore(self) -> None:
        self.cache.seqlen = [list(row) for row in self.lengths]


def _prompts(prompt_ids) -> list:
    return list(prompt_ids) if isinstance(prompt_ids, (list, tuple)) else [row for row in prompt_ids]


def _device_of(prompt_ids) -> torch.device:
    return torch.as_tensor(_prompts(prompt_ids)[0]).device


def _sync(device: torch.device) -> None:
    if device.type == "cuda":
        torch.cuda.synchronize()


@torch.no_grad()
def prefill_once(blocks, prompt_ids) -> SharedPrefill:
    """Prefill the prompts once, timed like a run's own prefill, so several
    runs can borrow it (the first tokens are the prompts' greedy argmaxes)."""
    t0 = time.perf_counter()
    cache, last = blocks.prefill(prompt_ids)
    first = last.argmax(dim=-1).tolist()
    _sync(_device_of(prompt_ids))
    lens = [int(torch.as_tensor(p).numel()) for p in _prompts(prompt_ids)]
    return SharedPrefill(cache, first, time.perf_counter() - t0, lens, [list(r) for r in cache.seqlen])


class _BatchRun:
    """One generation over a fixed batch: prefill (or a borrowed one), the
    lanes, per-tick launches and counters, and the closing bookkeeping."""

    def __init__(self, blocks, prompt_ids, max_new_tokens, emus=None, prefilled: SharedPrefill | None = None,
                 handles: bool = False):
        self.blocks = blocks
        self.device = _device_of(prompt_ids)
        if self.device.type == "cuda":
            torch.cuda.reset_peak_memory_stats()
        self.trace = BatchTrace()
        t0 = time.perf_counter()
        if prefilled is None:
            prefilled = prefill_once(blocks, prompt_ids)
        else:
            prefilled.restore()
            t0 -= prefilled.prefill_s  # its prefill cost is charged to this run
        self.t0 = t0
        self.cache = prefilled.cache
        self.trace.prefill_s = prefilled.prefill_s
        B = len(prefilled.prompt_lens)
        limits = list(max_new_tokens) if isinstance(max_new_tokens, (list, tuple)) else [max_new_tokens] * B
        self.lanes = [Lane(b, prefilled.prompt_lens[b], limits[b], emus[b] if emus is not None else None)
                      for b in range(B)]
        for lane, tok in zip(self.lanes, prefilled.first_tokens):
            lane.commit(tok)
        # ids may stay on the device when nothing reads them before the end
        self.handles = handles and hasattr(blocks, "resolve_tokens") and hasattr(blocks, "reset_token_ring")
        if self.handles:
            blocks.reset_token_ring()
        self.accept_flags: list[bool] | None = None

    def live(self) -> list[Lane]:
        return [lane for lane in self.lanes if not lane.done]

    def launch(self, p_rows, r_rows, c_rows, r_repeat: int = 1, expect=None):
        """P, R (r_repeat times) and C over [(lane, token)] rows as one launch
        sequence when the blocks fuse passes; returns the C rows' ids (or token
        handles) and updates the whole-batch counters. `expect` (one entry per
        C row: the token speculated at the row's next position, or None) asks
        for the greedy comparisons on the device; their flags land in
        `accept_flags`."""
        passes = [("P", p_rows)] + [("R", r_rows)] * r_repeat + [("C", c_rows)]
        passes = [(kind, [lane.index for lane, _ in rows], [t for _, t in rows]) for kind, rows in passes if rows]
        ids = None
        self.accept_flags = None
        fused = getattr(self.blocks, "run_passes", None)
        if fused is not None and passes:
            if expect is not None and c_rows:
                ids = fused(passes, self.cache, self.handles, expect=expect)
                self.accept_flags = self.blocks.last_accept
            else:
                ids = fused(passes, self.cache, self.handles)
        else:
            for kind, seqs, toks in passes:
                if kind == "P":
                    self.blocks.prelude_union(seqs, toks, self.cache)
                elif kind == "R":
                    self.blocks.advance_union(seqs, toks, self.cache)
                elif self.handles:
                    ids = self.blocks.coda_argmax_union(seqs, toks, self.cache, lazy=True)
                else:
                    ids = self.blocks.coda_argmax_union(seqs, toks, self.cache)
        if p_rows:
            self.trace.n_p_calls += 1
        if r_rows:
            for _ in range(r_repeat):
                self.trace.count_r(len(r_rows))
        if c_rows:
            self.trace.n_c_calls += 1
        return ids

    def finish(self) -> BatchTrace:
        if self.handles:  # one read of the token ring for the whole generation
            for lane in self.lanes:
                lane.committed[:] = self.blocks.resolve_tokens(lane.committed)
                lane.trace.tokens[:] = self.blocks.resolve_tokens(lane.trace.tokens)
        _sync(self.device)
        bt = self.trace
        bt.walltime_s = time.perf_counter() - self.t0
        bt.per_seq = [lane.trace for lane in self.lanes]
        for t in bt.per_seq:
            t.walltime_s = bt.walltime_s
        if self.device.type == "cuda":
            bt.peak_alloc_gb = torch.cuda.max_memory_allocated() / 1e9
            bt.peak_reserved_gb = torch.cuda.max_memory_reserved() / 1e9
        bt.cache_gb = self.cache.nbytes / 1e9
        return bt


# ---------------------------------------------------------------------------
# sequential looped decode
# ---------------------------------------------------------------------------
@torch.no_grad()
def ar_generate_batch(blocks, prompt_ids, max_new_tokens, prefilled: SharedPrefill | None = None) -> BatchTrace:
    """Lockstep sequential looped decode: every live lane's next token runs
    P, T_total x R and C (one launch sequence per token)."""
    run = _BatchRun(blocks, prompt_ids, max_new_tokens, prefilled=prefilled, handles=True)
    T = blocks.T_total
    while live := run.live():
        rows = [(lane, ActiveToken(token_id=lane.committed[-1], position=lane.next_position - 1, role="verify"))
                for lane in live]
        ids = run.launch(rows, rows, rows, r_repeat=T)
        for (lane, _), tok in zip(rows, ids):
            lane.trace.n_p_calls += 1
            lane.trace.n_r_calls += T
            lane.trace.n_c_calls += 1
            lane.commit(tok)
    return run.finish()


# ---------------------------------------------------------------------------
# wavefront decoding
# ---------------------------------------------------------------------------
def _route(lane: Lane, T_total: int, T_draft: int):
    """Route a lane's wave by the depth each token reaches in this tick's R:
    the tokens reaching T_total leave the wave as verifies (position order);
    the token reaching T_draft stays and a copy of it is the lane's draft
    row (src/decoding/parcae_blocks.py:540-581 routing)."""
    verifies, draft, stay = [], None, []
    for t in lane.flight:
        depth = t.step + 1
        if depth == T_total:
            t.role = "verify"
            verifies.append(t)
            continue
        stay.append(t)
        if depth == T_draft:
            draft = ActiveToken(token_id=t.token_id, position=t.position, role="draft", step=depth, row=t.row)
    lane.flight = stay
    verifies.sort(key=lambda t: t.position)
    return verifies, draft


def _settle(lane: Lane, verifies, draft, gold: dict, cache, decide) -> None:
    """Walk a lane's verify chain in position order. Verify v finalizes
    position v + 1 against the token speculated there: accept commits it;
    reject commits the full-depth argmax, truncates the lane from there and
    re-enters the argmax; nothing speculated yet (the wave's edge) commits the
    argmax and enters it. After an untroubled walk the draft row's argmax is
    the new leading token."""
    rejected = False
    for i, v in enumerate(verifies):
        g = gold[id(v)]
        v.is_alive = False
        at = v.position + 1
        nxt = verifies[i + 1] if i + 1 < len(verifies) else lane.token_at(at)
        if nxt is None:  # the wave's edge
            edge = True
            lane.commit(g)
            lane.enqueue(g, at)
        else:
            edge = False
            lane.trace.n_drafts_proposed += 1
            if decide(v, g, nxt):
                lane.trace.n_drafts_accepted += 1
                lane.commit(nxt.token_id)
            else:
                lane.trace.n_drafts_rejected += 1
                lane.trace.n_rollback_events += 1
                rejected = True
                lane.commit(g)
                lane.truncate_from(at, cache)
                lane.enqueue(g, at)
        if lane.done or rejected or edge:
            break
    if lane.done:
        lane.retire()
    elif draft is not None and not rejected:
        lane.enqueue(gold[id(draft)], draft.position + 1)


@torch.no_grad()
def generate_wavefront_batch(blocks, prompt_ids, max_new_tokens, policy: SsdPolicy, emus=None,
                             prefilled: SharedPrefill | None = None) -> BatchTrace:
    """One independent wave per sequence; P, R and C once per tick over the union.

    Greedy (no emulated streams) on blocks that compare on the device: each
    verify row carries the token speculated at its next position, the argmax
    kernel compares them, and the tick reads back one accept flag per C row
    while every id stays on the device (read once at the end). Other blocks
    compare the ids on the host."""
    emulated = emus is not None and all(e is not None for e in emus)
    greedy = emus is None or all(e is None for e in emus)
    on_device = greedy and getattr(blocks, "device_accept", False) and hasattr(blocks, "run_passes")
    run = _BatchRun(blocks, prompt_ids, max_new_tokens, emus, prefilled, handles=emulated or on_device)
    T_total, T_draft = policy.T_total, policy.T_draft
    for lane in run.live():
        lane.enqueue(lane.committed[-1], lane.prompt_len)
    guard = max(lane.limit for lane in run.lanes) * (T_total + 4) + 100
    tick = 0
    while live := run.live():
        tick += 1
        if tick > guard:
            raise RuntimeError(f"wfd batch exceeded tick guard ({guard}) -- scheduler bug?")
        p_rows = [(lane, t) for lane in live for t in lane.queued]
        for lane in live:
            lane.flight += lane.queued
            lane.queued = []
        r_rows = [(lane, t) for lane in live for t in lane.flight]
        plan = []
        for lane in live:
            if lane.flight:
                lane.trace.n_r_calls += 1
            verifies, draft = _route(lane, T_total, T_draft)
            if verifies or draft is not None:
                plan.append((lane, verifies, draft))
        c_rows = [(lane, t) for lane, vs, d in plan for t in vs + ([d] if d is not None else [])]
        expect = None
        if on_device and c_rows:
            expect = []
            for lane, vs, d in plan:
                for i, v in enumerate(vs):
                    nxt = vs[i + 1] if i + 1 < len(vs) else lane.token_at(v.position + 1)
                    expect.append(None if nxt is None else nxt.token_id)
                if d is not None:
                    expect.append(None)
        ids = run.launch(p_rows, r_rows, c_rows, expect=expect)
        gold = {id(t): g for (_, t), g in zip(c_rows, ids or [])}
        if expect is not None:
            flag = {id(t): f for (_, t), f in zip(c_rows, run.accept_flags)}
            decide = lambda v, g, nxt: flag[id(v)]  # noqa: E731
        for lane, verifies, draft in plan:
            lane.trace.n_c_calls += 1
            if expect is None:
                decide = lambda v, g, nxt, lane=lane: lane.accepts(g, nxt.token_id)  # noqa: E731
            _settle(lane, verifies, draft, gold, run.cache, decide)
    return run.finish()


# ---------------------------------------------------------------------------
# draft-then-verify
# ---------------------------------------------------------------------------
def _open_round(lane: Lane, draft_length: int, tok: int, pos: int) -> None:
    lane.round = DtvRound(base_tok=tok, base_pos=pos, k=min(draft_length, lane.limit - len(lane.committed)))


def _verify_round(lane: Lane, golds: list[int], cache) -> tuple[int, int] | None:
    """Check the round's drafts in order against the full-depth argmaxes.
    Returns the next round's (token, position), or None when the lane is done."""
    r = lane.round
    for i in range(r.k):
        lane.trace.n_drafts_proposed += 1
        if lane.accepts(golds[i], r.drafts[i]):
            lane.trace.n_drafts_accepted += 1
            if lane.commit(r.drafts[i]):
                return None
            continue
        lane.trace.n_drafts_rejected += 1
        lane.trace.n_rollback_events += 1
        at = r.base_pos + i + 1
        done = lane.commit(golds[i])
        cache.drop_positions_at_and_after(lane.index, at)
        return None if done else (golds[i], at)
    bonus = golds[r.k]  # every draft accepted: the last source's argmax is free
    return None if lane.commit(bonus) else (bonus, r.base_pos + r.k + 1)


@torch.no_grad()
def generate_dtv_batch(blocks, prompt_ids, max_new_tokens, policy: SsdPolicy, draft_length: int, emus=None,
                       prefilled: SharedPrefill | None = None) -> BatchTrace:
    """Draft-then-verify with nested reuse, one round per lane
    (behaviour of src/decoding/scheduler_batch.py:368-505).

    A round drafts k tokens: sources p, p + 1, ..., p + k each get their P
    pass and the shallow depths 0..T_draft one after another (a source's
    shallow argmax is the next source's token and the draft for its
    position), then all k + 1 sources continue together from T_draft to
    T_total -- the draft's recurrence is the prefix of the verify's, nothing
    is recomputed -- and their full-depth argmaxes check the drafts in order:
    the first rejected draft commits the full-depth token and truncates the
    lane past it; if all k hold, the last source's argmax is a free bonus
    token. Lanes drift apart freely; P, R and C run once per tick over the
    union of what every live lane needs."""
    if draft_length < 1 or draft_length + 1 > getattr(blocks, "max_in_flight", draft_length + 1):
        raise ValueError(f"draft_length={draft_length}: a round keeps draft_length + 1 sources in flight, "
                         f"at most {getattr(blocks, 'max_in_flight', '?')} fit")
    emulated = emus is not None and all(e is not None for e in emus)
    run = _BatchRun(blocks, prompt_ids, max_new_tokens, emus, prefilled, handles=emulated)
    T_total, T_draft = policy.T_total, policy.T_draft
    for lane in run.live():
        _open_round(lane, draft_length, lane.committed[-1], lane.prompt_len)
    guard = max(lane.limit for lane in run.lanes) * ((draft_length + 1) * max(T_draft, 1) + T_total + 4) + 100
    tick = 0
    while live := run.live():
        tick += 1
        if tick > guard:
            raise RuntimeError(f"dtv batch exceeded tick guard ({guard}) -- scheduler bug?")
        p_rows = []
        for lane in live:
            if lane.round.stage == "embed":
                p_rows.append((lane, lane.round.next_source()))
                lane.trace.n_p_calls += 1
        r_rows, c_plan = [], []
        for lane in live:
            r = lane.round
            if r.stage == "shallow":
                moving = [r.sources[-1]]
            elif r.stage == "deep" and r.sources[0].step < T_total:
                moving = list(r.sources)
            else:
                continue
            lane.trace.n_r_calls += 1
            r_rows += [(lane, t) for t in moving]
            if moving[0].step + 1 == (T_draft if r.stage == "shallow" else T_total):
                c_plan.append((lane, moving))
        c_rows = [(lane, t) for lane, ts in c_plan for t in ts]
        ids = run.launch(p_rows, r_rows, c_rows)
        k = 0
        for lane, ts in c_plan:
            out = ids[k: k + len(ts)]
            k += len(ts)
            lane.trace.n_c_calls += 1
            if lane.round.stage == "shallow":
                lane.round.take_shallow(out[0])
                continue
            nxt = _verify_round(lane, out, run.cache)
            if nxt is None:
                lane.retire()
            else:
                _open_round(lane, draft_length, *nxt)
    return run.finish()
