"""Fixed-batch schedulers: sequential looped decode (AR) and WFD with
per-sequence waves (src/decoding/scheduler_batch.py:36-362).

A fixed batch of B sequences: a finished sequence idles (no refill); each
tick runs P, R and C once over the union of whatever every live sequence
needs; each sequence settles independently -- accept/reject comes from its
EmulatedAcceptance stream when given (Bernoulli(alpha)), else from the real
argmax comparison -- and a reject rolls back only that sequence.

Extensions over the reference (both optional, the reference's behaviour is
the default): prompts may have different lengths (a list of 1-D id
sequences; the reference needs equal lengths, huginn_blocks_batch.py:180-185),
and max_new_tokens may be a per-sequence list (the reference takes one value,
scheduler_batch.py:348-349).
"""
from __future__ import annotations

import copy
import time
from dataclasses import dataclass, field

import torch

from .batch_state import SeqState
from .policy import SsdPolicy
from .state import ActiveToken


@dataclass
class BatchTrace:
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

    @property
    def n_tokens(self) -> int:
        return sum(len(t.tokens) for t in self.per_seq)

    @property
    def tokens_per_s(self) -> float:
        return self.n_tokens / self.walltime_s if self.walltime_s > 0 else float("nan")

    @property
    def walltime_decode_s(self) -> float:
        return max(self.walltime_s - self.prefill_s, 0.0)

    @property
    def decode_tokens_per_s(self) -> float:
        d = self.walltime_decode_s
        return self.n_tokens / d if d > 0 else float("nan")

    @property
    def r_union_mean(self) -> float:
        return self.r_union_total / self.n_r_calls if self.n_r_calls else 0.0

    @property
    def acceptance_rate(self) -> float:
        prop = sum(t.n_drafts_proposed for t in self.per_seq)
        acc = sum(t.n_drafts_accepted for t in self.per_seq)
        return acc / prop if prop else float("nan")


@dataclass
class SharedPrefill:
    """One prompt prefill reused by several decode runs: decode only writes
    positions >= the prompt length, so restoring the logical lengths is enough
    (src/decoding/scheduler_batch.py:83-120)."""

    cache: object
    first_tokens: list[int]
    prefill_s: float
    prompt_lens: list[int]
    _seqlen0: list = field(default_factory=list)

    def restore(self) -> None:
        self.cache.seqlen = [row[:] for row in self._seqlen0]


def _prompt_lens(prompt_ids) -> list[int]:
    if isinstance(prompt_ids, (list, tuple)):
        return [int(torch.as_tensor(p).numel()) for p in prompt_ids]
    return [int(prompt_ids.shape[1])] * int(prompt_ids.shape[0])


def _device_of(prompt_ids):
    p = prompt_ids[0] if isinstance(prompt_ids, (list, tuple)) else prompt_ids
    return torch.as_tensor(p).device


@torch.no_grad()
def prefill_once(blocks, prompt_ids) -> SharedPrefill:
    t0 = time.perf_counter()
    cache, last = blocks.prefill(prompt_ids)
    first = last.argmax(dim=-1).tolist()
    if _device_of(prompt_ids).type == "cuda":
        torch.cuda.synchronize()
    return SharedPrefill(cache=cache, first_tokens=first, prefill_s=time.perf_counter() - t0,
                         prompt_lens=_prompt_lens(prompt_ids), _seqlen0=[row[:] for row in cache.seqlen])


def _start(blocks, prompt_ids, emus, max_new_tokens, bt: BatchTrace, t0: float, prefilled: SharedPrefill | None):
    """Prefill (or borrow one) and commit every sequence's first token."""
    if prefilled is not None:
        prefilled.restore()
        cache, first = prefilled.cache, prefilled.first_tokens
        bt.prefill_s = prefilled.prefill_s
        t0 = time.perf_counter() - prefilled.prefill_s
        lens = prefilled.prompt_lens
    else:
        cache, last = blocks.prefill(prompt_ids)
        first = last.argmax(dim=-1).tolist()
        if _device_of(prompt_ids).type == "cuda":
            torch.cuda.synchronize()
        bt.prefill_s = time.perf_counter() - t0
        lens = _prompt_lens(prompt_ids)
    B = len(lens)
    limits = list(max_new_tokens) if isinstance(max_new_tokens, (list, tuple)) else [max_new_tokens] * B
    seqs = []
    for b in range(B):
        s = SeqState(idx=b, prefix_len=lens[b], emu=emus[b] if emus is not None else None, max_new_tokens=limits[b])
        s.commit(first[b])
        s.done = len(s.committed) >= limits[b]
        seqs.append(s)
    return cache, seqs, t0


def _lazy_tokens(blocks) -> bool:
    """Blocks that can hand out device token handles (no host sync per commit)."""
    ok = hasattr(blocks, "resolve_tokens") and hasattr(blocks, "reset_token_ring")
    if ok:
        blocks.reset_token_ring()
    return ok


def _finish(bt: BatchTrace, seqs, t0: float, device, cache, blocks=None, lazy: bool = False) -> BatchTrace:
    if lazy:  # one read of the token ring for the whole generation
        for s in seqs:
            s.committed[:] = blocks.resolve_tokens(s.committed)
            s.trace.tokens[:] = blocks.resolve_tokens(s.trace.tokens)
    if device.type == "cuda":
        torch.cuda.synchronize()
    bt.walltime_s = time.perf_counter() - t0
    for s in seqs:
        s.trace.walltime_s = bt.walltime_s
    bt.per_seq = [s.trace for s in seqs]
    if device.type == "cuda":
        bt.peak_alloc_gb = torch.cuda.max_memory_allocated() / 1e9
        bt.peak_reserved_gb = torch.cuda.max_memory_reserved() / 1e9
    bt.cache_gb = cache.nbytes / 1e9
    return bt


def _passes(blocks, cache, passes, lazy: bool):
    """A tick's P / R / C passes, [(kind, seq_ids, toks)] in order. Blocks
    that can fuse them run the tick as one launch sequence; others get one
    call per pass. Returns the C pass's ids (or token handles), else None."""
    fused = getattr(blocks, "run_passes", None)
    if fused is not None:
        return fused([p for p in passes if p[2]], cache, lazy)
    out = None
    for kind, ids, toks in passes:
        if not toks:
            continue
        if kind == "P":
            blocks.prelude_union(ids, toks, cache)
        elif kind == "R":
            blocks.advance_union(ids, toks, cache)
        else:
            out = blocks.coda_argmax_union(ids, toks, cache, lazy=True) if lazy else blocks.coda_argmax_union(
                ids, toks, cache)
    return out


def _record_r(bt: BatchTrace, n: int) -> None:
    bt.n_r_calls += 1
    bt.r_union_total += n
    bt.r_union_max = max(bt.r_union_max, n)


@torch.no_grad()
def ar_generate_batch(blocks, prompt_ids, max_new_tokens, prefilled: SharedPrefill | None = None) -> BatchTrace:
    """Lockstep sequential looped decode: per token P -> R x T_total -> C."""
    device = _device_of(prompt_ids)
    if device.type == "cuda":
        torch.cuda.reset_peak_memory_stats()
    bt = BatchTrace()
    cache, seqs, t0 = _start(blocks, prompt_ids, None, max_new_tokens, bt, time.perf_counter(), prefilled)
    lazy = _lazy_tokens(blocks)  # sequential decode never compares ids: keep them on the device
    while True:
        act = [s for s in seqs if not s.done]
        if not act:
            break
        toks = []
        for s in act:
            toks.append(ActiveToken(token_id=s.committed[-1], position=s.prefix_len + len(s.committed) - 1,
                                    role="verify"))
            s.trace.n_p_calls += 1
        ids = [s.idx for s in act]
        # the whole token: P, T_total R passes and C as one launch sequence
        out = _passes(blocks, cache, [("P", ids, toks)] + [("R", ids, toks)] * blocks.T_total + [("C", ids, toks)],
                      lazy)
        bt.n_p_calls += 1
        for _ in range(blocks.T_total):
            _record_r(bt, len(toks))
            for s in act:
                s.trace.n_r_calls += 1
        bt.n_c_calls += 1
        for s, nid in zip(act, out):
            s.trace.n_c_calls += 1
            s.commit(nid)
            s.done = len(s.committed) >= s.max_new_tokens
    return _finish(bt, seqs, t0, device, cache, blocks, lazy)


@torch.no_grad()
def generate_wavefront_batch(blocks, prompt_ids, max_new_tokens, policy: SsdPolicy, emus=None,
                             prefilled: SharedPrefill | None = None) -> BatchTrace:
    """One independent wave per sequence; P, R and C once per tick over the union."""
    device = _device_of(prompt_ids)
    if device.type == "cuda":
        torch.cuda.reset_peak_memory_stats()
    bt = BatchTrace()
    cache, seqs, t0 = _start(blocks, prompt_ids, emus, max_new_tokens, bt, time.perf_counter(), prefilled)
    T_total, T_draft = policy.T_total, policy.T_draft
    # emulated acceptance never compares ids, so they can stay on the device
    lazy = emus is not None and all(e is not None for e in emus) and _lazy_tokens(blocks)
    for s in seqs:
        if not s.done:
            s.active_p.append(ActiveToken(token_id=s.committed[-1], position=s.prefix_len, role="draft"))
            s.trace.n_p_calls += 1

    max_new = max(s.max_new_tokens for s in seqs)
    ticks, guard = 0, max_new * (T_total + 4) + 100
    while True:
        live = [s for s in seqs if not s.done]
        if not live:
            break
        ticks += 1
        if ticks > guard:
            raise RuntimeError(f"wfd batch exceeded tick guard ({guard}) -- scheduler bug?")

        # P: everything queued by the previous settle; it joins the R union
        p_pairs = [(s, t) for s in live for t in s.active_p]
        for s, t in p_pairs:
            s.active_r.append(t)
        for s in live:
            s.active_p = []
        # R: one tick for every live wave
        r_pairs = [(s, t) for s in live for t in s.active_r if t.is_alive]
        # routing by the depth each token reaches in this tick's R: commit
        # point -> verify (moved); draft point -> draft (copied)
        for s in live:
            keep = []
            for t in s.active_r:
                if not t.is_alive:
                    continue
                after = t.step + 1
                if after == T_total:
                    t.role = "verify"
                    s.active_c.append(t)
                else:
                    keep.append(t)
                    if after == T_draft:
                        d = copy.copy(t)
                        d.role = "draft"
                        d.step = after
                        s.active_c.append(d)
            s.active_r = keep
        # C: one union over every sequence's verifies + draft
        plan, c_toks, c_ids = [], [], []
        for s in live:
            if s.active_c:
                vs = sorted((t for t in s.active_c if t.role == "verify"), key=lambda t: t.position)
                ds = [t for t in s.active_c if t.role == "draft"]
                plan.append((s, vs, ds))
                c_toks += vs + ds
                c_ids += [s.idx] * (len(vs) + len(ds))
        golds = _passes(blocks, cache, [("P", [s.idx for s, _ in p_pairs], [t for _, t in p_pairs]),
                                        ("R", [s.idx for s, _ in r_pairs], [t for _, t in r_pairs]),
                                        ("C", c_ids, c_toks)], lazy)
        if p_pairs:
            bt.n_p_calls += 1
        if r_pairs:
            _record_r(bt, len(r_pairs))
            for s in live:
                if any(t.is_alive for t in s.active_r) or any(t.role == "verify" for t in s.active_c):
                    s.trace.n_r_calls += 1
        gold_of: dict[int, int] = {}
        if c_toks:
            gold_of = {id(t): g for t, g in zip(c_toks, golds)}
            bt.n_c_calls += 1
            for s, _, _ in plan:
                s.trace.n_c_calls += 1

        # settle each sequence, then seed its new leading draft
        for s, vs, ds in plan:
            rejected = boundary = False
            for i, v in enumerate(vs):
                gold = gold_of[id(v)]
                v.is_alive = False
                nxt_pos = v.position + 1
                nxt = vs[i + 1] if i + 1 < len(vs) else s.find_active(nxt_pos)
                if nxt is None:
                    s.commit(gold)
                    s.active_p.append(ActiveToken(token_id=gold, position=nxt_pos, role="draft"))
                    s.trace.n_p_calls += 1
                    boundary = True
                else:
                    ok = s.emu.draw() if s.emu is not None else gold == nxt.token_id
                    s.trace.n_drafts_proposed += 1
                    if ok:
                        s.trace.n_drafts_accepted += 1
                        s.commit(nxt.token_id)
                    else:
                        s.trace.n_drafts_rejected += 1
                        s.trace.n_rollback_events += 1
                        rejected = True
                        s.commit(gold)
                        s.rollback(nxt_pos, cache)
                        s.active_p.append(ActiveToken(token_id=gold, position=nxt_pos, role="draft"))
                        s.trace.n_p_calls += 1
                s.done = len(s.committed) >= s.max_new_tokens
                if s.done or rejected or boundary:
                    break
            if s.done:
                s.clear_working_state()
                continue
            if ds and not rejected:
                src = ds[0]
                s.active_p.append(ActiveToken(token_id=gold_of[id(src)], position=src.position + 1, role="draft"))
                s.trace.n_p_calls += 1
            s.active_c = []
    return _finish(bt, seqs, t0, device, cache, blocks, lazy)


def _dtv_round(s: SeqState, draft_length: int) -> None:
    """Open a draft-then-verify round from the last committed token (at s.p)."""
    s.K = min(draft_length, s.max_new_tokens - len(s.committed))
    s.j = 0
    s.sources, s.drafts = [], []
    s.cur_tok, s.cur_pos = s.last_token, s.p
    s.phase = "need_p"


@torch.no_grad()
def generate_dtv_batch(blocks, prompt_ids, max_new_tokens, policy: SsdPolicy, draft_length: int, emus=None,
                       prefilled: SharedPrefill | None = None) -> BatchTrace:
    """Draft-then-verify with nested reuse, one round state machine per
    sequence (src/decoding/scheduler_batch.py:368-505).

    A round drafts K tokens: sources p, p+1, ..., p+K each run P and the
    shallow depths 0..T_draft one after another (a source's shallow argmax is
    the next source's token), then all K+1 sources continue together from
    T_draft to T_total -- the draft's recurrence is the prefix of the
    verify's, nothing is recomputed -- and their full-depth argmaxes verify
    the drafts in order: the first rejected draft commits the gold token and
    rolls the sequence back past it; if all K are accepted the last source's
    gold is a free bonus token. Sequences desync freely: P, R and C run once
    per tick over the union of what every live sequence needs."""
    if draft_length < 1 or draft_length + 1 > getattr(blocks, "max_in_flight", draft_length + 1):
        raise ValueError(f"draft_length={draft_length}: a round keeps draft_length + 1 sources in flight, "
                         f"at most {getattr(blocks, 'max_in_flight', '?')} fit")
    device = _device_of(prompt_ids)
    if device.type == "cuda":
        torch.cuda.reset_peak_memory_stats()
    bt = BatchTrace()
    cache, seqs, t0 = _start(blocks, prompt_ids, emus, max_new_tokens, bt, time.perf_counter(), prefilled)
    T_total, T_draft = policy.T_total, policy.T_draft
    lazy = emus is not None and all(e is not None for e in emus) and _lazy_tokens(blocks)
    for s in seqs:
        if not s.done:
            s.last_token, s.p = s.committed[-1], s.prefix_len
            _dtv_round(s, draft_length)

    max_new = max(s.max_new_tokens for s in seqs)
    ticks, guard = 0, max_new * ((draft_length + 1) * max(T_draft, 1) + T_total + 4) + 100
    while True:
        live = [s for s in seqs if not s.done]
        if not live:
            break
        ticks += 1
        if ticks > guard:
            raise RuntimeError(f"dtv batch exceeded tick guard ({guard}) -- scheduler bug?")

        # P: each sequence whose next source needs its embedding
        pneed = [s for s in live if s.phase == "need_p"]
        new = []
        for s in pneed:
            t = ActiveToken(token_id=s.cur_tok, position=s.cur_pos, role="verify")
            s.sources.append(t)
            new.append(t)
            s.trace.n_p_calls += 1
            s.phase = "draft"
        # R: a drafting sequence advances its current source, a verifying one all K+1
        r_pairs, moved = [], []
        for s in live:
            if s.phase == "draft":
                r_pairs.append((s, s.sources[-1]))
                moved.append(s)
            elif s.phase == "verify" and s.sources[0].step < T_total:
                r_pairs += [(s, t) for t in s.sources]
                moved.append(s)
        # C: a draft source that reaches T_draft in this R, or all sources at T_total
        stepped = {id(t) for _, t in r_pairs}
        after = lambda t: t.step + (id(t) in stepped)  # noqa: E731
        entries = []
        for s in live:
            if s.phase == "draft" and after(s.sources[-1]) == T_draft:
                entries.append((s, "draft", [s.sources[-1]]))
            elif s.phase == "verify" and after(s.sources[0]) == T_total:
                entries.append((s, "verify", list(s.sources)))
        c_toks = [t for _, _, ts in entries for t in ts]
        c_ids = [s.idx for s, _, ts in entries for _ in ts]
        out = _passes(blocks, cache, [("P", [s.idx for s in pneed], new),
                                      ("R", [s.idx for s, _ in r_pairs], [t for _, t in r_pairs]),
                                      ("C", c_ids, c_toks)], lazy)
        if pneed:
            bt.n_p_calls += 1
        if r_pairs:
            _record_r(bt, len(r_pairs))
            for s in moved:
                s.trace.n_r_calls += 1
        if not entries:
            continue
        bt.n_c_calls += 1
        k = 0
        for s, kind, ts in entries:
            ids = out[k: k + len(ts)]
            k += len(ts)
            s.trace.n_c_calls += 1
            if kind == "draft":
                nxt = ids[0]
                if s.j < s.K:
                    s.drafts.append(nxt)  # the draft for position cur_pos + 1
                s.cur_tok, s.cur_pos = nxt, s.cur_pos + 1
                s.j += 1
                s.phase = "need_p" if s.j <= s.K else "verify"
                continue
            # verify: source p + i's gold predicts p + i + 1
            rejected = False
            for i in range(s.K):
                s.trace.n_drafts_proposed += 1
                ok = s.emu.draw() if s.emu is not None else ids[i] == s.drafts[i]
                if ok:
                    s.trace.n_drafts_accepted += 1
                    s.commit(s.drafts[i])
                    if len(s.committed) >= s.max_new_tokens:
                        s.done = True
                        break
                else:
                    s.trace.n_drafts_rejected += 1
                    s.trace.n_rollback_events += 1
                    rejected = True
                    s.commit(ids[i])
                    cache.drop_positions_at_and_after(s.idx, s.p + i + 1)
                    s.last_token, s.p = ids[i], s.p + i + 1
                    s.done = len(s.committed) >= s.max_new_tokens
                    break
            if not rejected and not s.done:
                s.commit(ids[s.K])  # all K accepted: the bonus token
                s.last_token, s.p = ids[s.K], s.p + s.K + 1
                s.done = len(s.committed) >= s.max_new_tokens
            if s.done:
                s.clear_working_state()
            else:
                _dtv_round(s, draft_length)
    return _finish(bt, seqs, t0, device, cache, blocks, lazy)
