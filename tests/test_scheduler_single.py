"""Single-sequence WFD scheduler and block routing on the CPU (stub compute).

The product's LoopedBlocks routing (P_dyn / R_dyn / C_multi_dyn) and
generate_wavefront_dynamic run over the stub model; with real greedy
comparisons a B = 1 run must reproduce the reference batch scheduler's B = 1
golden trace (tokens and counters) -- the reference's own gate that the
single-sequence and batch schedulers agree at B = 1
(experiments/exp4_emu/verify_batch.py:105-125). The oracle's wfd_single is
held to the same traces.

They are also held to traces of the reference's own single-sequence
schedulers (src/decoding/scheduler.py generate_wavefront_dynamic /
generate_draft_then_verify, src/decoding/scheduler_emu.py
generate_wavefront_emu / generate_dtv_emu; tests/golden/
scheduler_single_traces.json): greedy at 70 % and 95 % draft agreement,
emulated alpha 0 / 0.5 / 0.9 / 1, eos stops -- tokens, counters, rollbacks,
the per-call schedule and the draws. The reference's emulated-alpha gate
(experiments/exp4_emu/verify_step1.py:84-95: empirical acceptance within 0.06
of alpha over 384 tokens at alpha 0.5 / 0.8) holds for the product's emulated
schedulers.
"""
from __future__ import annotations

import json
import os

import pytest
import torch

from oracle import scheduler as osched
from tests.golden.stub_model import StubBatchBlocks, stub_prompts
from wavefront_decoding_amd.acceptance import RowLogits
from wavefront_decoding_amd.blocks import LoopedBlocks
from wavefront_decoding_amd.policy import SsdPolicy
from wavefront_decoding_amd.emu import EmulatedAcceptance
from wavefront_decoding_amd.scheduler import generate_draft_then_verify, generate_wavefront_dynamic
from wavefront_decoding_amd.scheduler_emu import generate_dtv_emu, generate_wavefront_emu
from wavefront_decoding_amd.state import WavefrontState

GOLDEN = json.load(open(os.path.join(os.path.dirname(__file__), "golden", "scheduler_traces.json")))
B1 = [r for r in GOLDEN["wfd"] if r["B"] == 1 and r["alpha"] is None]
B1_DTV = [r for r in GOLDEN["dtv"] if r["B"] == 1 and r["alpha"] is None]
# traces of the reference's own single-sequence schedulers (scheduler.py / scheduler_emu.py)
SINGLE = json.load(open(os.path.join(os.path.dirname(__file__), "golden", "scheduler_single_traces.json")))


class _SingleCache:
    def __init__(self, inner):
        self.inner = inner

    def drop_positions_at_and_after(self, position: int) -> None:
        self.inner.drop_positions_at_and_after(0, position)


class StubSingleBlocks(LoopedBlocks):
    """Product routing over stub compute."""

    def __init__(self, T_total: int, agree_pct: int = 70):  # noqa: D401 -- no engine on the CPU
        self.stub = StubBatchBlocks(T_total, 1, agree_pct=agree_pct)
        self.T_total = T_total
        self.device = torch.device("cpu")

    def prefill(self, input_ids, T_total, T_draft):
        ids = input_ids.reshape(-1)
        cache, logits = self.stub.prefill([ids])
        state = WavefrontState(prefix_len=len(ids), kv_cache=_SingleCache(cache), T_total=T_total, T_draft=T_draft,
                               last_committed_position=len(ids) - 1)
        return state, logits[0]

    def _prelude(self, cache, toks):
        self.stub.prelude_union([0] * len(toks), toks, cache)

    def advance_one_step(self, toks, cache):
        if toks:
            self.stub.advance_union([0] * len(toks), toks, cache)

    def coda_logits(self, state, toks):
        return [RowLogits(values=None, token=t) for t in self.stub.coda_argmax_union([0] * len(toks), toks, None)]


def _counters(per):
    return {k: per[k] for k in ("n_r_calls", "n_p_calls", "n_c_calls", "n_drafts_proposed", "n_drafts_accepted",
                                "n_drafts_rejected", "n_rollback_events")}


@pytest.mark.parametrize("ref", B1, ids=lambda r: f"T{r['T_total']}/{r['T_draft']}-N{r['max_new_tokens']}")
def test_dynamic_scheduler_matches_batch_b1_trace(ref):
    blocks = StubSingleBlocks(ref["T_total"])
    toks, trace = generate_wavefront_dynamic(blocks, stub_prompts(1, 5)[0], ref["max_new_tokens"],
                                             SsdPolicy(T_total=ref["T_total"], T_draft=ref["T_draft"]))
    per = ref["per_seq"][0]
    assert toks == per["tokens"]
    assert trace.counters() == _counters(per)
    assert [list(d) for d in blocks.stub.last_cache.drops] == ref["drops"]
    if ref["calls"] is not None:
        assert [[k, [list(x) for x in rows]] for k, rows in blocks.stub.calls] == ref["calls"]


@pytest.mark.parametrize("ref", B1, ids=lambda r: f"T{r['T_total']}/{r['T_draft']}-N{r['max_new_tokens']}")
def test_oracle_single_matches_batch_b1_trace(ref):
    blocks = StubBatchBlocks(ref["T_total"], 1)
    c = osched.wfd_single(blocks, stub_prompts(1, 5)[0].tolist(), ref["max_new_tokens"], ref["T_total"],
                          ref["T_draft"])
    per = ref["per_seq"][0]
    assert c.tokens == per["tokens"]
    assert {k: getattr(c, k) for k in _counters(per)} == _counters(per)


def test_t_draft_equal_t_total_is_sequential():
    """WFD at T_draft == T_total is sequential decode call for call:
    (N - 1) * T_total R ticks, every token committed at a boundary."""
    for T in (4, 8):
        for N in (1, 9):
            blocks = StubSingleBlocks(T)
            toks, tr = generate_wavefront_dynamic(blocks, stub_prompts(1, 5)[0], N, SsdPolicy(T_total=T, T_draft=T))
            assert tr.n_r_calls == (N - 1) * T and tr.n_drafts_proposed == 0
            ar = osched.ar_single(StubBatchBlocks(T, 1), stub_prompts(1, 5)[0].tolist(), N, T)
            assert toks == ar


def test_steady_state_wave_shape():
    """At alpha = 1 the wave fills to W = T_total / T_draft tokens at steps
    (W-1-j)*T_draft (src/decoding/forced_schedule.py:43-64)."""
    T, d = 8, 2
    blocks = StubSingleBlocks(T)
    blocks.stub.agree_pct = 100
    seen = []
    orig = blocks.stub.advance_union

    def spy(seq_ids, toks, cache):
        seen.append(sorted(t.step for t in toks))
        orig(seq_ids, toks, cache)

    blocks.stub.advance_union = spy
    toks, tr = generate_wavefront_dynamic(blocks, stub_prompts(1, 5)[0], 20, SsdPolicy(T_total=T, T_draft=d))
    W = T // d
    assert tr.n_drafts_rejected == 0
    assert [(W - 1 - j) * d for j in range(W)][::-1] in seen
    assert max(len(s) for s in seen) == W


def test_policy_validation():
    with pytest.raises(ValueError):
        SsdPolicy(T_total=2, T_draft=3)
    with pytest.raises(ValueError):
        SsdPolicy(T_total=4, T_draft=0)
    with pytest.raises(ValueError):
        SsdPolicy(mode="temperature")
    with pytest.warns(UserWarning):
        SsdPolicy(T_total=5, T_draft=2)


@pytest.mark.parametrize("ref", B1_DTV,
                         ids=lambda r: f"T{r['T_total']}/{r['T_draft']}-K{r['draft_length']}-N{r['max_new_tokens']}")
def test_dtv_single_matches_batch_b1_trace(ref):
    """Single-sequence draft-then-verify reproduces the reference batch DtV's
    B = 1 trace with real greedy comparisons: tokens, counters, rollbacks and
    the per-call schedule."""
    blocks = StubSingleBlocks(ref["T_total"])
    toks, trace = generate_draft_then_verify(blocks, stub_prompts(1, 5)[0], ref["max_new_tokens"],
                                             SsdPolicy(T_total=ref["T_total"], T_draft=ref["T_draft"]),
                                             ref["draft_length"])
    per = ref["per_seq"][0]
    assert toks == per["tokens"]
    assert trace.counters() == _counters(per)
    assert [list(d) for d in blocks.stub.last_cache.drops] == ref["drops"]
    if ref["calls"] is not None:
        assert [[k, [list(x) for x in rows]] for k, rows in blocks.stub.calls] == ref["calls"]


def _single_id(r):
    a = "greedy" if r["alpha"] is None else f"a{r['alpha']}"
    k = f"-K{r['draft_length']}" if "draft_length" in r else ""
    e = "" if r["eos"] is None else f"-eos{r['eos']}"
    return f"T{r['T_total']}/{r['T_draft']}{k}-N{r['max_new_tokens']}-{a}-agree{r['agree_pct']}{e}"


def _check_single(ref, toks, trace, blocks, emu):
    assert toks == ref["tokens"]
    assert trace.counters() == ref["counters"]
    assert [list(d) for d in blocks.stub.last_cache.drops] == ref["drops"]
    if ref["calls"] is not None:
        assert [[k, [list(x) for x in rows]] for k, rows in blocks.stub.calls] == ref["calls"]
    assert ([emu.n_draws, emu.n_accepts] if emu is not None else None) == ref["emu"]


@pytest.mark.parametrize("ref", SINGLE["wfd"], ids=_single_id)
def test_wfd_single_matches_reference_single_trace(ref):
    blocks = StubSingleBlocks(ref["T_total"], ref["agree_pct"])
    policy = SsdPolicy(T_total=ref["T_total"], T_draft=ref["T_draft"])
    emu = None if ref["alpha"] is None else EmulatedAcceptance(ref["alpha"], ref["seed"])
    if emu is None:
        toks, trace = generate_wavefront_dynamic(blocks, stub_prompts(1, 5)[0], ref["max_new_tokens"], policy,
                                                 eos_token_id=ref["eos"])
    else:
        toks, trace = generate_wavefront_emu(blocks, stub_prompts(1, 5)[0], ref["max_new_tokens"], policy, emu=emu,
                                             eos_token_id=ref["eos"])
    _check_single(ref, toks, trace, blocks, emu)


@pytest.mark.parametrize("ref", SINGLE["dtv"], ids=_single_id)
def test_dtv_single_matches_reference_single_trace(ref):
    blocks = StubSingleBlocks(ref["T_total"], ref["agree_pct"])
    policy = SsdPolicy(T_total=ref["T_total"], T_draft=ref["T_draft"])
    emu = None if ref["alpha"] is None else EmulatedAcceptance(ref["alpha"], ref["seed"])
    args = (blocks, stub_prompts(1, 5)[0], ref["max_new_tokens"], policy, ref["draft_length"])
    if emu is None:
        toks, trace = generate_draft_then_verify(*args, eos_token_id=ref["eos"])
    else:
        toks, trace = generate_dtv_emu(*args, emu=emu, eos_token_id=ref["eos"])
    _check_single(ref, toks, trace, blocks, emu)


@pytest.mark.parametrize("ref", SINGLE["wfd"], ids=_single_id)
def test_oracle_wfd_single_matches_reference_single_trace(ref):
    blocks = StubBatchBlocks(ref["T_total"], 1, agree_pct=ref["agree_pct"])
    emu = None if ref["alpha"] is None else osched.Emu(ref["alpha"], ref["seed"])
    c = osched.wfd_single(blocks, stub_prompts(1, 5)[0].tolist(), ref["max_new_tokens"], ref["T_total"],
                          ref["T_draft"], emu=emu, eos=ref["eos"])
    assert c.tokens == ref["tokens"]
    assert {k: getattr(c, k) for k in ref["counters"]} == ref["counters"]
    assert [list(d) for d in blocks.last_cache.drops] == ref["drops"]
    assert ([emu.n_draws, emu.n_accepts] if emu is not None else None) == ref["emu"]


@pytest.mark.parametrize("alpha", [0.5, 0.8])
@pytest.mark.parametrize("kind", ["wfd", "dtv"])
def test_emulated_alpha_gate(kind, alpha):
    """The reference's gate 3 (experiments/exp4_emu/verify_step1.py:84-95):
    T_total 4, T_draft 1, 384 tokens, seed 7 (draft length 4 for DtV): the
    empirical acceptance is within 0.06 of alpha, and the run is the
    reference's own, draw for draw."""
    ref = next(r for r in SINGLE[kind] if r["max_new_tokens"] == 384 and r["alpha"] == alpha)
    blocks = StubSingleBlocks(4)
    emu = EmulatedAcceptance(alpha, 7)
    policy = SsdPolicy(T_total=4, T_draft=1)
    if kind == "wfd":
        toks, trace = generate_wavefront_emu(blocks, stub_prompts(1, 5)[0], 384, policy, emu=emu)
    else:
        toks, trace = generate_dtv_emu(blocks, stub_prompts(1, 5)[0], 384, policy, 4, emu=emu)
    assert len(toks) == 384 and abs(emu.empirical_rate - alpha) < 0.06, emu.empirical_rate
    _check_single(ref, toks, trace, blocks, emu)


def test_emulated_alpha_one_and_equivalence():
    """The reference's gates 1 and 2 (verify_step1.py:55-82): emu=None is the
    greedy scheduler exactly; alpha = 1 gives no rejects and exactly N commits."""
    for T_draft in (1, 2):
        pol = SsdPolicy(T_total=4, T_draft=T_draft)
        a = generate_wavefront_dynamic(StubSingleBlocks(4), stub_prompts(1, 5)[0], 48, pol)
        b = generate_wavefront_emu(StubSingleBlocks(4), stub_prompts(1, 5)[0], 48, pol, emu=None)
        assert a[0] == b[0] and a[1].counters() == b[1].counters()
    pol = SsdPolicy(T_total=4, T_draft=1)
    a = generate_draft_then_verify(StubSingleBlocks(4), stub_prompts(1, 5)[0], 48, pol, 4)
    b = generate_dtv_emu(StubSingleBlocks(4), stub_prompts(1, 5)[0], 48, pol, 4, emu=None)
    assert a[0] == b[0] and a[1].counters() == b[1].counters()
    for fn, extra in ((generate_wavefront_emu, ()), (generate_dtv_emu, (4,))):
        toks, tr = fn(StubSingleBlocks(4), stub_prompts(1, 5)[0], 48, pol, *extra, emu=EmulatedAcceptance(1.0, 0))
        assert tr.n_drafts_rejected == 0 and len(toks) == 48
