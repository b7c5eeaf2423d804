"""P / R / C block forwards over the device engine.

`RecursiveBlocks` is the interface the WFD scheduler drives
(src/decoding/blocks.py:22-116). `LoopedBlocks` implements it for one
sequence and `LoopedBlocksBatch` implements the fixed-batch union API
(src/decoding/huginn_blocks_batch.py:46-346). Both run every pass as one
union launch sequence on `engine.LoopedModel`, so P, R and C each cost one
pass over the weights per tick whatever the number of rows.

Routing inside R_dyn follows src/decoding/parcae_blocks.py:540-581: after
the tick, the maximal position-ordered prefix of tokens at their commit point
(step == T_total) is promoted to "verify" and moved to the C queue; a token
reaching step == T_draft is copied to the C queue as a "draft" and keeps
advancing.
"""
from __future__ import annotations

import copy
import time
from abc import ABC, abstractmethod

import numpy as np
import torch

from .acceptance import GREEDY, RowLogits
from .engine import NO_EXPECT, LoopedModel
from .kv_cache import BatchStaticKVCache, StaticKVCache
from .state import ActiveToken, WavefrontState


class RecursiveBlocks(ABC):
    """P / R / C primitives of a looped LM for the dynamic WFD scheduler."""

    T_total: int

    @abstractmethod
    def prefill(self, input_ids: torch.Tensor, T_total: int, T_draft: int): ...

    @abstractmethod
    def P_dyn(self, state: WavefrontState): ...

    @abstractmethod
    def R_dyn(self, state: WavefrontState): ...

    @abstractmethod
    def C_multi_dyn(self, state: WavefrontState): ...

    @abstractmethod
    def ar_generate(self, prompt_ids, max_new_tokens, eos_token_id=None, sampler=None): ...

    @abstractmethod
    def prelude_forward(self, cache, token_id: int, position: int): ...

    @abstractmethod
    def prelude_tokens(self, cache, toks: list) -> None: ...

    @abstractmethod
    def advance_one_step(self, toks: list, cache) -> None: ...

    @abstractmethod
    def coda_logits(self, state, toks: list) -> list: ...

    def find_active(self, state: WavefrontState, position: int):
        return state.find_active_prc(position)


def _row_logits(logits: torch.Tensor, ids: torch.Tensor) -> list[RowLogits]:
    return [RowLogits(values=logits[i], token=t) for i, t in enumerate(ids.tolist())]


class LoopedBlocks(RecursiveBlocks):
    """Single-sequence blocks (B = 1 view of the engine)."""

    def __init__(self, model: LoopedModel, T_total: int | None = None):
        if T_total is not None and T_total != model.cfg.T_total:
            raise ValueError(f"T_total={T_total} does not match the model's {model.cfg.T_total}")
        self.model = model
        self.cfg = model.cfg
        self.T_total = model.cfg.T_total
        self.device = model.device
        self.max_seq_len = model.max_seq_len

    # -- cache / prefill ----------------------------------------------------------
    def create_cache(self) -> StaticKVCache:
        c = self.cfg
        return StaticKVCache(c.n_kv_heads, c.head_dim, self.max_seq_len, self.model.dtype, self.device,
                             n_slots=c.n_slots)

    @torch.no_grad()
    def prefill(self, input_ids: torch.Tensor, T_total: int, T_draft: int):
        """Prompt prefill into this blocks object's cache. The cache is allocated
        once and reused by every generation (its lengths are reset here), so
        captured decode graphs stay valid; one generation at a time."""
        if T_total != self.T_total:
            raise AssertionError("Prefill T_total must match the blocks' T_total")
        ids = input_ids.reshape(-1).tolist()
        if getattr(self, "_cache", None) is None:
            self._cache = self.create_cache()
        cache = self._cache
        cache.reset_lengths()
        logits = self.model.prefill_seq(cache, 0, ids)
        L = len(ids)
        cache._seen_tokens = L
        state = WavefrontState(prefix_len=L, kv_cache=cache, T_total=T_total, T_draft=T_draft,
                               last_committed_position=L - 1)
        return state, logits

    # -- primitives --------------------------------------------------------------------
    def _prelude(self, cache, toks: list[ActiveToken]) -> None:
        rows = self.model.prelude_union(cache, [0] * len(toks), [t.position for t in toks],
                                        [t.token_id for t in toks])
        for t, r in zip(toks, rows.tolist()):
            t.row = r
            t.step = 0

    @property
    def max_in_flight(self) -> int:
        """Tokens of one sequence that may be in flight at once (wave-state pool rows per sequence)."""
        return self.model.R

    def prelude_tokens(self, cache, toks: list[ActiveToken]) -> None:
        """Prelude these tokens (each gets its wave-state pool row, step 0)."""
        self._prelude(cache, toks)

    def prelude_forward(self, cache, token_id: int, position: int):
        """Prelude one token; returns (hidden, static_state) device views of its pool row."""
        t = ActiveToken(token_id=token_id, position=position, role="verify")
        self._prelude(cache, [t])
        D = self.cfg.d_model
        return self.model.pool[t.row, :D], self.model.pool[t.row, D:]

    def advance_one_step(self, toks: list, cache) -> None:
        if not toks:
            return
        self.model.core_union(cache, [0] * len(toks), [t.position for t in toks], [t.step for t in toks])
        for t in toks:
            t.step += 1

    def coda_logits(self, state, toks: list) -> list[RowLogits]:
        logits, ids = self.model.coda_union(state.kv_cache, [0] * len(toks), [t.position for t in toks])
        return _row_logits(logits, ids)

    # -- dynamic-scheduler blocks -------------------------------------------------------
    @torch.no_grad()
    def P_dyn(self, state: WavefrontState):
        if state.active_p:
            self._prelude(state.kv_cache, state.active_p)
            state.active_r.extend(state.active_p)
            state.active_p = []
        return state, True

    @torch.no_grad()
    def R_dyn(self, state: WavefrontState):
        toks = [t for t in state.active_r if t.is_alive]
        self.advance_one_step(toks, state.kv_cache)
        T_draft, T_total = state.T_draft, state.T_total
        commit_ids: set[int] = set()
        for t in sorted(toks, key=lambda t: t.position):
            if t.step != T_total:
                break
            commit_ids.add(id(t))
        survivors, any_c = [], False
        for t in state.active_r:
            if not t.is_alive:
                continue
            if id(t) in commit_ids:
                t.role = "verify"
                state.active_c.append(t)
                any_c = True
            else:
                survivors.append(t)
                if t.step == T_draft:
                    d = copy.copy(t)
                    d.role = "draft"
                    state.active_c.append(d)
                    any_c = True
        state.active_r = survivors
        return state, any_c

    @torch.no_grad()
    def C_multi_dyn(self, state: WavefrontState):
        verify = sorted((t for t in state.active_c if t.role == "verify"), key=lambda t: t.position)
        draft = [t for t in state.active_c if t.role == "draft"]
        assert len(draft) <= 1, "dyn wave invariant: <= 1 draft per C"
        ordered = verify + draft
        if not ordered:
            return state, 0, []
        return state, len(verify), self.coda_logits(state, ordered)

    # -- sequential looped decode (the losslessness reference) ----------------------------
    @torch.no_grad()
    def ar_generate(self, prompt_ids, max_new_tokens, eos_token_id=None, sampler=None):
        """One token at a time at full depth: P -> R x T_total -> C on the same
        primitives as WFD (src/decoding/ar_baseline.py:133-193). Returns
        (tokens, walltime_s)."""
        sampler = sampler or GREEDY
        t0 = time.perf_counter()
        state, last = self.prefill(prompt_ids.view(1, -1), self.T_total, self.T_total)
        cache = state.kv_cache
        nid = sampler(last, state.prefix_len)
        out = [nid]
        pos = state.prefix_len
        while len(out) < max_new_tokens and not (eos_token_id is not None and nid == eos_token_id):
            tok = ActiveToken(token_id=nid, position=pos, role="verify")
            self._prelude(cache, [tok])
            for _ in range(self.T_total):
                self.advance_one_step([tok], cache)
            nid = sampler(self.coda_logits(state, [tok])[0], pos + 1)
            out.append(nid)
            pos += 1
        if self.device.type == "cuda":
            torch.cuda.synchronize()
        return out, time.perf_counter() - t0


class LoopedBlocksBatch:
    """Fixed-batch union blocks: every P / R / C call takes (seq, token) pairs
    from any sequences and runs them as one union."""

    def __init__(self, model: LoopedModel, batch_size: int | None = None, T_total: int | None = None):
        if T_total is not None and T_total != model.cfg.T_total:
            raise ValueError("T_total mismatch")
        self.model = model
        self.cfg = model.cfg
        self.T_total = model.cfg.T_total
        self.B = batch_size or model.max_batch
        if self.B > model.max_batch:
            raise ValueError(f"batch_size {self.B} > model.max_batch {model.max_batch}")
        self.n_prelude, self.n_core, self.n_coda = self.cfg.n_prelude, self.cfg.n_core, self.cfg.n_coda
        self.device = model.device
        self.max_seq_len = model.max_seq_len

    # slots (src/decoding/huginn_blocks_batch.py:84-100)
    def slot_prelude(self, i: int) -> int:
        return self.model.slot_prelude(i)

    def slot_core(self, step: int, layer: int) -> int:
        return self.model.slot_core(step, layer)

    def slot_coda(self, i: int) -> int:
        return self.model.slot_coda(i)

    def n_slots(self) -> int:
        return self.cfg.n_slots

    def create_cache(self) -> BatchStaticKVCache:
        return self.model.create_cache(self.B)

    def cache_nbytes_estimate(self) -> int:
        elem = torch.tensor([], dtype=self.model.dtype).element_size()
        return self.n_slots() * self.B * self.max_seq_len * self.cfg.n_kv_heads * self.cfg.head_dim * elem * 2

    @torch.no_grad()
    def prefill(self, input_ids):
        """input_ids: (B, L) tensor, or a list of B 1-D id sequences (ragged
        prompt lengths). Returns (cache, last_logits (B, V) float32)."""
        seqs = [row for row in input_ids] if not isinstance(input_ids, (list, tuple)) else list(input_ids)
        if len(seqs) != self.B:
            raise AssertionError(f"prefill expects B={self.B} prompts, got {len(seqs)}")
        # one cache per blocks object, reused across generations (keeps captured graphs valid)
        if getattr(self, "_cache", None) is None:
            self._cache = self.create_cache()
        cache = self._cache
        cache.reset_lengths()
        last = torch.stack([self.model.prefill_seq(cache, b, torch.as_tensor(s).reshape(-1).tolist())
                            for b, s in enumerate(seqs)])
        return cache, last

    @property
    def max_in_flight(self) -> int:
        """Tokens of one sequence that may be in flight at once (wave-state pool rows per sequence)."""
        return self.model.R

    @torch.no_grad()
    def prelude_union(self, seq_ids, toks, cache) -> None:
        if not toks:
            return
        rows = self.model.prelude_union(cache, seq_ids, [t.position for t in toks], [t.token_id for t in toks])
        for t, r in zip(toks, rows.tolist()):
            t.row = r
            t.step = 0

    @torch.no_grad()
    def advance_union(self, seq_ids, toks, cache) -> None:
        if not toks:
            return
        self.model.core_union(cache, seq_ids, [t.position for t in toks], [t.step for t in toks])
        for t in toks:
            t.step += 1

    @torch.no_grad()
    def coda_argmax_union(self, seq_ids, toks, cache, lazy: bool = False) -> list[int]:
        """Greedy next-token ids of the union (src/decoding/huginn_blocks_batch.py:323-346).
        lazy=True returns token handles (negative ints naming device token-ring
        slots) without waiting for the GPU; `resolve_tokens` turns them into ids,
        and prelude_union accepts them as token ids directly."""
        if not toks:
            return []
        _, ids = self.model.coda_union(cache, seq_ids, [t.position for t in toks])
        if lazy and self.model.last_c_handles is not None:
            return list(self.model.last_c_handles)
        return ids.tolist()

    # the C pass can compare each row's argmax with the token speculated at
    # the next position on the device (wfd_argmax's accept flags)
    device_accept = True

    # no torch.no_grad() wrapper here: it costs ~5 us per call, once per tick,
    # and the engine creates no autograd state (weights and tables never
    # require grad); the schedulers run inside their own no-grad context
    def run_passes(self, passes, cache, lazy: bool = False, expect=None) -> list[int] | None:
        """A tick's passes -- [(kind, seq_ids, toks)] with kind "P", "R" or "C"
        (C last) -- as one launch sequence (one graph replay, one table upload),
        with the token bookkeeping prelude_union / advance_union /
        coda_argmax_union would do. Returns the C pass's ids (or handles).
        `expect` (C rows, each a plain id, a ring handle or None): the C pass
        also compares every row's argmax with it on the device, and
        `last_accept` receives the flags (polled from mapped host memory, no copy)."""
        eng, R = [], self.model.R
        for kind, seq_ids, toks in passes:
            if not toks:
                continue
            pos = [t.position for t in toks]
            if kind == "P":
                eng.append(("P", seq_ids, pos, [t.token_id for t in toks]))
                for b, t in zip(seq_ids, toks):
                    t.row = int(b) * R + t.position % R
                    t.step = 0
            elif kind == "R":
                eng.append(("R", seq_ids, pos, [t.step for t in toks]))
                for t in toks:
                    t.step += 1
            else:
                exp = None if expect is None else [NO_EXPECT if e is None else e for e in expect]
                eng.append(("C", seq_ids, pos, exp))
        out = self.model.run_passes(cache, eng) if eng else None
        self.last_accept = None
        if out is None:
            return None
        if expect is not None:
            self.last_accept = self.model.accept_flags()
        if lazy and self.model.last_c_handles is not None:
            return list(self.model.last_c_handles)
        return out[1].tolist()

    def reset_token_ring(self) -> None:
        self.model.reset_token_ring()

    def resolve_tokens(self, values) -> list[int]:
        return self.model.resolve_tokens(values)


def seq_positions(toks) -> np.ndarray:
    return np.asarray([t.position for t in toks], dtype=np.int64)
