"""Oracle schedulers: plain-Python restatements of the reference's WFD loops.

All of them drive a blocks object through the union API
(prefill / prelude_union / advance_union / coda_argmax_union), so the same
code runs over the stub model of tests/golden/stub_model.py (pinned against
traces written by the reference's own scheduler) and over the numpy looped
LM of oracle/looped_lm.py.

  wfd_batch   src/decoding/scheduler_batch.py:228-362
  ar_batch    src/decoding/scheduler_batch.py:185-222
  wfd_single  src/decoding/scheduler.py:88-224 with the R_dyn routing of
              src/decoding/parcae_blocks.py:540-581 and the C_multi_dyn
              ordering of parcae_blocks.py:583-597; emulated acceptance as
              src/decoding/scheduler_emu.py:33-155
  ar_single   src/decoding/ar_baseline.py:133-193
"""
from __future__ import annotations

import copy
import random


class Tok:
    """A token in flight (the fields of src/decoding/state.py:20-70 that the loop uses)."""

    def __init__(self, token_id: int, position: int, role: str):
        self.token_id = token_id
        self.position = position
        self.role = role
        self.step = 0
        self.hidden = None
        self.static_state = None
        self.is_alive = True


class Counters:
    def __init__(self):
        self.tokens: list[int] = []
        self.n_r_calls = self.n_p_calls = self.n_c_calls = 0
        self.n_drafts_proposed = self.n_drafts_accepted = self.n_drafts_rejected = self.n_rollback_events = 0


class BatchResult:
    def __init__(self, per_seq):
        self.per_seq = per_seq
        self.n_r_calls = self.n_p_calls = self.n_c_calls = 0
        self.r_union_total = self.r_union_max = 0


class Emu:
    """Bernoulli(rate) decisions from random.Random(seed) (src/decoding/emu.py:19-35)."""

    def __init__(self, rate: float, seed: int):
        assert 0.0 <= rate <= 1.0
        self.rng = random.Random(seed)
        self.rate = rate
        self.n_draws = self.n_accepts = 0

    def draw(self) -> bool:
        self.n_draws += 1
        ok = self.rng.random() < self.rate
        self.n_accepts += ok
        return ok


class _Seq:
    def __init__(self, b: int, L: int, emu, limit: int):
        self.b, self.L, self.emu, self.limit = b, L, emu, limit
        self.c = Counters()
        self.done = False
        self.P: list[Tok] = []
        self.R: list[Tok] = []
        self.C: list[Tok] = []

    def find(self, pos: int):
        for lst in (self.R, self.P, self.C):
            for t in lst:
                if t.is_alive and t.position == pos:
                    return t
        return None

    def commit(self, tok: int) -> None:
        self.c.tokens.append(tok)

    def rollback(self, pos: int, cache) -> None:
        """Reject at `pos`: drop this sequence's tokens at/after pos and truncate
        its slot lengths (src/decoding/batch_state.py:63-69)."""
        self.P = [t for t in self.P if t.position < pos]
        self.R = [t for t in self.R if t.position < pos]
        self.C = [t for t in self.C if t.position < pos]
        cache.drop_positions_at_and_after(self.b, pos)


def _first_tokens(blocks, prompts):
    cache, logits = blocks.prefill(prompts)
    first = [int(max(range(len(row)), key=lambda j: (row[j], -j))) for row in logits.tolist()]
    return cache, first


def _lens(prompts) -> list[int]:
    return [len(list(p)) for p in prompts]


def wfd_batch(blocks, prompts, max_new_tokens, T_total: int, T_draft: int, emus=None) -> BatchResult:
    cache, first = _first_tokens(blocks, prompts)
    lens = _lens(prompts)
    B = len(lens)
    limits = max_new_tokens if isinstance(max_new_tokens, (list, tuple)) else [max_new_tokens] * B
    seqs = [_Seq(b, lens[b], emus[b] if emus else None, limits[b]) for b in range(B)]
    res = BatchResult([s.c for s in seqs])
    for s in seqs:
        s.commit(first[s.b])
        s.done = len(s.c.tokens) >= s.limit
        if not s.done:
            s.P.append(Tok(first[s.b], s.L, "draft"))
            s.c.n_p_calls += 1
    guard = max(limits) * (T_total + 4) + 100
    tick = 0
    while any(not s.done for s in seqs):
        tick += 1
        if tick > guard:
            raise RuntimeError("tick guard")
        live = [s for s in seqs if not s.done]
        pp = [(s, t) for s in live for t in s.P]
        if pp:
            blocks.prelude_union([s.b for s, _ in pp], [t for _, t in pp], cache)
            for s, t in pp:
                s.R.append(t)
            for s in live:
                s.P = []
            res.n_p_calls += 1
        rr = [(s, t) for s in live for t in s.R if t.is_alive]
        if rr:
            blocks.advance_union([s.b for s, _ in rr], [t for _, t in rr], cache)
            res.n_r_calls += 1
            res.r_union_total += len(rr)
            res.r_union_max = max(res.r_union_max, len(rr))
            for s in live:
                if any(t.is_alive for t in s.R):
                    s.c.n_r_calls += 1
        for s in live:
            stay = []
            for t in s.R:
                if not t.is_alive:
                    continue
                if t.step == T_total:
                    t.role = "verify"
                    s.C.append(t)
                    continue
                stay.append(t)
                if t.step == T_draft:
                    d = copy.copy(t)
                    d.role = "draft"
                    s.C.append(d)
            s.R = stay
        order = []
        for s in live:
            if s.C:
                v = sorted([t for t in s.C if t.role == "verify"], key=lambda t: t.position)
                d = [t for t in s.C if t.role == "draft"]
                order.append((s, v, d))
        flat = [(s, t) for s, v, d in order for t in v + d]
        gold = {}
        if flat:
            out = blocks.coda_argmax_union([s.b for s, _ in flat], [t for _, t in flat], cache)
            gold = {id(t): g for (_, t), g in zip(flat, out)}
            res.n_c_calls += 1
            for s, _, _ in order:
                s.c.n_c_calls += 1
        for s, v, d in order:
            rej = bnd = False
            for i, vt in enumerate(v):
                g = gold[id(vt)]
                vt.is_alive = False
                np_ = vt.position + 1
                nxt = v[i + 1] if i + 1 < len(v) else s.find(np_)
                if nxt is None:
                    s.commit(g)
                    s.P.append(Tok(g, np_, "draft"))
                    s.c.n_p_calls += 1
                    bnd = True
                else:
                    acc = s.emu.draw() if s.emu is not None else (g == nxt.token_id)
                    s.c.n_drafts_proposed += 1
                    if acc:
                        s.c.n_drafts_accepted += 1
                        s.commit(nxt.token_id)
                    else:
                        s.c.n_drafts_rejected += 1
                        s.c.n_rollback_events += 1
                        rej = True
                        s.commit(g)
                        s.rollback(np_, cache)
                        s.P.append(Tok(g, np_, "draft"))
                        s.c.n_p_calls += 1
                if len(s.c.tokens) >= s.limit:
                    s.done = True
                if s.done or rej or bnd:
                    break
            if s.done:
                s.P, s.R, s.C = [], [], []
                continue
            if d and not rej:
                s.P.append(Tok(gold[id(d[0])], d[0].position + 1, "draft"))
                s.c.n_p_calls += 1
            s.C = []
    return res


def ar_batch(blocks, prompts, max_new_tokens, T_total: int) -> BatchResult:
    cache, first = _first_tokens(blocks, prompts)
    lens = _lens(prompts)
    B = len(lens)
    limits = max_new_tokens if isinstance(max_new_tokens, (list, tuple)) else [max_new_tokens] * B
    seqs = [_Seq(b, lens[b], None, limits[b]) for b in range(B)]
    res = BatchResult([s.c for s in seqs])
    for s in seqs:
        s.commit(first[s.b])
        s.done = len(s.c.tokens) >= s.limit
    while any(not s.done for s in seqs):
        act = [s for s in seqs if not s.done]
        toks = []
        for s in act:
            toks.append(Tok(s.c.tokens[-1], s.L + len(s.c.tokens) - 1, "verify"))
            s.c.n_p_calls += 1
        ids = [s.b for s in act]
        blocks.prelude_union(ids, toks, cache)
        res.n_p_calls += 1
        for _ in range(T_total):
            blocks.advance_union(ids, toks, cache)
            res.n_r_calls += 1
            res.r_union_total += len(toks)
            res.r_union_max = max(res.r_union_max, len(toks))
            for s in act:
                s.c.n_r_calls += 1
        out = blocks.coda_argmax_union(ids, toks, cache)
        res.n_c_calls += 1
        for s, g in zip(act, out):
            s.c.n_c_calls += 1
            s.commit(g)
            s.done = len(s.c.tokens) >= s.limit
    return res


def wfd_single(blocks, prompt, max_new_tokens: int, T_total: int, T_draft: int, emu=None,
               eos: int | None = None) -> Counters:
    """B = 1 dynamic loop; returns the counters (tokens in .tokens). With
    `emu` each accept is its next draw (src/decoding/scheduler_emu.py:33-155);
    `eos` stops at a committed eos token, the first included."""
    cache, first = _first_tokens(blocks, [prompt])
    L = _lens([prompt])[0]
    c = Counters()
    P: list[Tok] = []
    R: list[Tok] = []
    Cq: list[Tok] = []

    def find(pos):
        for lst in (R, P, Cq):
            for t in lst:
                if t.is_alive and t.position == pos:
                    return t
        return None

    c.tokens.append(first[0])
    if len(c.tokens) >= max_new_tokens or first[0] == eos:
        return c
    P.append(Tok(first[0], L, "draft"))
    c.n_p_calls += 1
    while len(c.tokens) < max_new_tokens:
        if P:
            blocks.prelude_union([0] * len(P), P, cache)
            R.extend(P)
            P = []
        alive = [t for t in R if t.is_alive]
        if alive:
            blocks.advance_union([0] * len(alive), alive, cache)
        c.n_r_calls += 1
        commit = set()
        for t in sorted(alive, key=lambda t: t.position):
            if t.step != T_total:
                break
            commit.add(id(t))
        stay = []
        for t in R:
            if not t.is_alive:
                continue
            if id(t) in commit:
                t.role = "verify"
                Cq.append(t)
            else:
                stay.append(t)
                if t.step == T_draft:
                    d = copy.copy(t)
                    d.role = "draft"
                    Cq.append(d)
        R = stay
        v = sorted([t for t in Cq if t.role == "verify"], key=lambda t: t.position)
        d = [t for t in Cq if t.role == "draft"]
        assert len(d) <= 1
        gold = []
        if v or d:
            gold = blocks.coda_argmax_union([0] * (len(v) + len(d)), v + d, cache)
            c.n_c_calls += 1
        rej = stop = False
        for i, vt in enumerate(v):
            vt.is_alive = False
            np_ = vt.position + 1
            nxt = v[i + 1] if i + 1 < len(v) else find(np_)
            if nxt is None:
                c.tokens.append(gold[i])
                P.append(Tok(gold[i], np_, "draft"))
                c.n_p_calls += 1
            else:
                c.n_drafts_proposed += 1
                if (gold[i] == nxt.token_id) if emu is None else emu.draw():
                    c.n_drafts_accepted += 1
                    c.tokens.append(nxt.token_id)
                else:
                    c.n_drafts_rejected += 1
                    c.n_rollback_events += 1
                    rej = True
                    c.tokens.append(gold[i])
                    P = [t for t in P if t.position < np_]
                    R = [t for t in R if t.position < np_]
                    Cq = [t for t in Cq if t.position < np_]
                    cache.drop_positions_at_and_after(0, np_)
                    P.append(Tok(gold[i], np_, "draft"))
                    c.n_p_calls += 1
            stop = len(c.tokens) >= max_new_tokens or c.tokens[-1] == eos
            if stop or rej or nxt is None:
                break
        if stop:
            break
        if d and not rej:
            P.append(Tok(gold[len(v)], d[0].position + 1, "draft"))
            c.n_p_calls += 1
        Cq = []
    return c


def ar_single(blocks, prompt, max_new_tokens: int, T_total: int) -> list[int]:
    cache, first = _first_tokens(blocks, [prompt])
    pos = _lens([prompt])[0]
    out = [first[0]]
    while len(out) < max_new_tokens:
        t = Tok(out[-1], pos, "verify")
        blocks.prelude_union([0], [t], cache)
        for _ in range(T_total):
            blocks.advance_union([0], [t], cache)
        out.append(blocks.coda_argmax_union([0], [t], cache)[0])
        pos += 1
    return out
