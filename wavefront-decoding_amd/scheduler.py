"""Single-sequence wavefront decoding (WFD) scheduler.

Semantics of the reference's flag-driven loop (src/decoding/scheduler.py:88-224):
every iteration is one R tick over the whole wave; P runs for tokens queued
by the previous iteration; C runs when the tick brought a token to its draft
point (step == T_draft, copied) or commit point (step == T_total, moved).
The verify at position N finalizes N+1 against the token already speculated
there: equal argmax -> accept; otherwise commit the argmax, roll back every
slot at/after N+1 and re-enter the corrected token (cascade). A boundary
(nothing speculated at N+1 yet) commits the argmax directly. After an
accepted (or boundary) settle, the draft logits of this tick seed the next
leading-edge token.

Counter semantics match the reference's GenerationTrace
(scheduler.py:51-70) call for call.
"""
from __future__ import annotations

import time
from dataclasses import dataclass, field

import torch

from .policy import SsdPolicy
from .state import ActiveToken, WavefrontState


@dataclass
class GenerationTrace:
    tokens: list[int] = field(default_factory=list)
    walltime_s: float = 0.0
    walltime_steady_s: float = 0.0
    n_r_calls: int = 0
    n_p_calls: int = 0
    n_c_calls: int = 0
    n_drafts_proposed: int = 0
    n_drafts_accepted: int = 0
    n_drafts_rejected: int = 0
    n_rollback_events: int = 0

    @property
    def acceptance_rate(self) -> float:
        return self.n_drafts_accepted / self.n_drafts_proposed if self.n_drafts_proposed else float("nan")

    def counters(self) -> dict:
        return {k: getattr(self, k) for k in ("n_r_calls", "n_p_calls", "n_c_calls", "n_drafts_proposed",
                                             "n_drafts_accepted", "n_drafts_rejected", "n_rollback_events")}


def _sync(device) -> None:
    if torch.device(device).type == "cuda":
        torch.cuda.synchronize()


@torch.no_grad()
def generate_wavefront_dynamic(blocks, prompt_ids: torch.Tensor, max_new_tokens: int, policy: SsdPolicy,
                               eos_token_id: int | None = None) -> tuple[list[int], GenerationTrace]:
    """Greedy lossless WFD for one sequence. Stops at max_new_tokens or when a
    committed token equals eos_token_id. Returns (tokens, trace)."""
    return wavefront_single(blocks, prompt_ids, max_new_tokens, policy, None, eos_token_id)


def _decide(sampler, emu, draft_token: int, draft_probs, logits, position: int) -> tuple[bool, int]:
    """(accept, gold) for a draft at `position`: the greedy comparison, or the
    next Bernoulli draw of an emulated-acceptance stream (gold is still the
    full-depth argmax, committed on a reject)."""
    if emu is None:
        return sampler.verify(draft_token, draft_probs, logits, position)
    return emu.draw(), sampler(logits, position)


def wavefront_single(blocks, prompt_ids: torch.Tensor, max_new_tokens: int, policy: SsdPolicy, emu=None,
                     eos_token_id: int | None = None) -> tuple[list[int], GenerationTrace]:
    """The WFD loop behind generate_wavefront_dynamic (emu None: greedy
    comparisons) and generate_wavefront_emu (each accept decided by emu.draw())."""
    trace = GenerationTrace()
    device = prompt_ids.device
    sampler = policy.make_sampler()
    t0 = time.perf_counter()
    state, last_logits = blocks.prefill(prompt_ids.view(1, -1), T_total=policy.T_total, T_draft=policy.T_draft)

    def commit(tok: int, pos: int) -> None:
        state.committed.append(tok)
        state.last_committed_position = pos
        trace.tokens.append(tok)

    def enqueue(tok: int, pos: int) -> None:
        state.active_p.append(ActiveToken(token_id=tok, position=pos, role="draft"))
        trace.n_p_calls += 1

    first = sampler(last_logits, state.prefix_len)
    commit(first, state.prefix_len)
    warm: float | None = None
    if len(state.committed) >= max_new_tokens or (eos_token_id is not None and first == eos_token_id):
        return _finish(trace, device, t0, warm)
    enqueue(first, state.prefix_len)

    while len(state.committed) < max_new_tokens:
        if state.active_p:
            blocks.P_dyn(state)
        _, call_c = blocks.R_dyn(state)
        trace.n_r_calls += 1
        n_verify, logits = 0, []
        if call_c:
            _, n_verify, logits = blocks.C_multi_dyn(state)
            trace.n_c_calls += 1

        rejected = stop = False
        verifies = sorted((t for t in state.active_c if t.role == "verify"), key=lambda t: t.position)[:n_verify]
        for i, v in enumerate(verifies):
            v.is_alive = False
            nxt_pos = v.position + 1
            nxt = verifies[i + 1] if i + 1 < len(verifies) else state.find_active_prc(nxt_pos)
            if nxt is None:                                   # boundary: nothing speculated at nxt_pos
                gold = sampler(logits[i], nxt_pos)
                commit(gold, nxt_pos)
                enqueue(gold, nxt_pos)
            else:
                ok, gold = _decide(sampler, emu, nxt.token_id, nxt.draft_probs, logits[i], nxt_pos)
                trace.n_drafts_proposed += 1
                if ok:
                    trace.n_drafts_accepted += 1
                    commit(nxt.token_id, nxt_pos)
                else:                                         # reject: cascade rollback, re-enter gold
                    trace.n_drafts_rejected += 1
                    trace.n_rollback_events += 1
                    rejected = True
                    commit(gold, nxt_pos)
                    state.rollback_prc(nxt_pos)
                    enqueue(gold, nxt_pos)
            last = state.committed[-1]
            stop = len(state.committed) >= max_new_tokens or (eos_token_id is not None and last == eos_token_id)
            if stop or rejected or nxt is None:
                break
        if stop:
            break

        drafts = logits[n_verify:]
        if drafts and not rejected:                           # new leading-edge draft
            src = next((t for t in state.active_c if t.role == "draft"), None)
            if src is not None:
                tok, _ = sampler.draft(drafts[0], src.position + 1)
                enqueue(tok, src.position + 1)
        state.active_c = []
        if warm is None and len(state.active_r) >= policy.steady_state_active_size:
            warm = time.perf_counter()
    return _finish(trace, device, t0, warm)


def _finish(trace: GenerationTrace, device, t0: float, warm: float | None):
    _sync(device)
    t1 = time.perf_counter()
    trace.walltime_s = t1 - t0
    trace.walltime_steady_s = (t1 - warm) if warm is not None else trace.walltime_s
    return list(trace.tokens), trace


@torch.no_grad()
def generate_draft_then_verify(blocks, prompt_ids: torch.Tensor, max_new_tokens: int, policy: SsdPolicy,
                               draft_length: int, eos_token_id: int | None = None
                               ) -> tuple[list[int], GenerationTrace]:
    """Greedy draft-then-verify with nested reuse for one sequence
    (src/decoding/scheduler.py:227-367). Each round forwards sources p..p+K one
    after another at the shallow depth T_draft (a source's shallow argmax is
    the next source's token and the draft for its position), then continues
    all K+1 sources together to T_total -- the shallow recurrence is the prefix
    of the full one, nothing is recomputed -- and verifies the drafts in order
    against the full-depth argmaxes: the first mismatch commits the gold token
    and drops every slot row from there on; if all K match, the last source's
    gold is a free bonus token. Lossless: every committed token is a
    full-depth argmax. Stops at max_new_tokens or a committed eos_token_id."""
    return dtv_single(blocks, prompt_ids, max_new_tokens, policy, draft_length, None, eos_token_id)


def dtv_single(blocks, prompt_ids: torch.Tensor, max_new_tokens: int, policy: SsdPolicy, draft_length: int,
               emu=None, eos_token_id: int | None = None) -> tuple[list[int], GenerationTrace]:
    """The draft-then-verify loop behind generate_draft_then_verify (emu None)
    and generate_dtv_emu (each accept decided by emu.draw())."""
    if draft_length < 1 or draft_length + 1 > getattr(blocks, "max_in_flight", draft_length + 1):
        raise ValueError(f"draft_length={draft_length}: a round keeps draft_length + 1 sources in flight, "
                         f"at most {getattr(blocks, 'max_in_flight', '?')} fit")
    trace = GenerationTrace()
    device = prompt_ids.device
    sampler = policy.make_sampler()
    t0 = time.perf_counter()
    state, last_logits = blocks.prefill(prompt_ids.reshape(1, -1), T_total=policy.T_total, T_draft=policy.T_draft)
    cache = state.kv_cache
    first = sampler(last_logits, state.prefix_len)
    state.committed.append(first)
    state.last_committed_position = state.prefix_len
    trace.tokens.append(first)
    warm = None

    def commit(tok: int, pos: int) -> bool:
        state.committed.append(tok)
        state.last_committed_position = pos
        trace.tokens.append(tok)
        return len(state.committed) >= max_new_tokens or (eos_token_id is not None and tok == eos_token_id)

    stop = len(state.committed) >= max_new_tokens or (eos_token_id is not None and first == eos_token_id)
    p, last = state.prefix_len, first
    while not stop:
        K = min(draft_length, max_new_tokens - len(state.committed))
        # draft: sources p..p+K at depths 0..T_draft, autoregressively
        sources, drafts = [], []
        tok, pos = last, p
        for j in range(K + 1):
            src = ActiveToken(token_id=tok, position=pos, role="verify")
            blocks.prelude_tokens(cache, [src])
            trace.n_p_calls += 1
            for _ in range(policy.T_draft):
                blocks.advance_one_step([src], cache)
                trace.n_r_calls += 1
            sources.append(src)
            nxt, _ = sampler.draft(blocks.coda_logits(state, [src])[0], pos + 1)
            trace.n_c_calls += 1
            if j < K:
                drafts.append(nxt)
            tok, pos = nxt, pos + 1
        # verify: all sources from T_draft to T_total together
        for _ in range(policy.T_total - policy.T_draft):
            blocks.advance_one_step(sources, cache)
            trace.n_r_calls += 1
        golds = blocks.coda_logits(state, sources)
        trace.n_c_calls += 1
        rejected = False
        for i in range(K):
            ok, gold = _decide(sampler, emu, drafts[i], None, golds[i], p + i + 1)
            trace.n_drafts_proposed += 1
            if ok:
                trace.n_drafts_accepted += 1
                if commit(drafts[i], p + i + 1):
                    stop = True
                    break
            else:
                trace.n_drafts_rejected += 1
                trace.n_rollback_events += 1
                rejected = True
                stop = commit(gold, p + i + 1)
                cache.drop_positions_at_and_after(p + i + 1)
                last, p = gold, p + i + 1
                break
        if not rejected and not stop:
            bonus = sampler(golds[K], p + K + 1)
            stop = commit(bonus, p + K + 1)
            last, p = bonus, p + K + 1
        if warm is None:
            warm = time.perf_counter()
    return _finish(trace, device, t0, warm)
