"""Schedulers vs golden traces written by the reference's own batch scheduler (CPU).

tests/golden/scheduler_traces.json was produced by
tests/golden/make_scheduler_traces.py running the reference's
generate_wavefront_batch / ar_generate_batch / generate_dtv_batch over the stub model of
tests/golden/stub_model.py. Both this repo's product schedulers and the
oracle's restatement must reproduce every trace exactly: committed tokens,
per-sequence and global counters, union sizes, rollback calls, the per-call
(seq, position, step) schedule and the emulated draws.
"""
from __future__ import annotations

import json
import os

import pytest

from oracle import scheduler as osched
from tests.golden.stub_model import StubBatchBlocks, stub_prompts, trace_record
from wavefront_decoding_amd import scheduler_batch as sb
from wavefront_decoding_amd.emu import EmulatedAcceptance
from wavefront_decoding_amd.policy import SsdPolicy

GOLDEN = json.load(open(os.path.join(os.path.dirname(__file__), "golden", "scheduler_traces.json")))


def _strip(rec: dict) -> dict:
    return {k: v for k, v in rec.items() if k not in ("B", "T_total", "T_draft", "max_new_tokens", "alpha")}


def _case_id(r):
    return f"B{r['B']}-T{r['T_total']}/{r.get('T_draft', '-')}-N{r['max_new_tokens']}-a{r.get('alpha')}"


@pytest.mark.parametrize("ref", GOLDEN["wfd"], ids=_case_id)
def test_product_wfd_batch_matches_reference_trace(ref):
    blocks = StubBatchBlocks(ref["T_total"], ref["B"])
    emus = None if ref["alpha"] is None else [EmulatedAcceptance(ref["alpha"], seed=1000 + b) for b in range(ref["B"])]
    bt = sb.generate_wavefront_batch(blocks, stub_prompts(ref["B"], 5), ref["max_new_tokens"],
                                     SsdPolicy(T_total=ref["T_total"], T_draft=ref["T_draft"]), emus)
    got = trace_record(bt, blocks, blocks.last_cache, emus)
    if ref["calls"] is None:
        got["calls"] = None
    assert got == _strip(ref)


@pytest.mark.parametrize("ref", GOLDEN["wfd"], ids=_case_id)
def test_oracle_wfd_batch_matches_reference_trace(ref):
    blocks = StubBatchBlocks(ref["T_total"], ref["B"])
    emus = None if ref["alpha"] is None else [osched.Emu(ref["alpha"], 1000 + b) for b in range(ref["B"])]
    res = osched.wfd_batch(blocks, stub_prompts(ref["B"], 5).tolist(), ref["max_new_tokens"], ref["T_total"],
                           ref["T_draft"], emus)
    got = trace_record(res, blocks, blocks.last_cache, emus)
    if ref["calls"] is None:
        got["calls"] = None
    assert got == _strip(ref)


def _dtv_id(r):
    return f"B{r['B']}-T{r['T_total']}/{r['T_draft']}-K{r['draft_length']}-N{r['max_new_tokens']}-a{r['alpha']}"


@pytest.mark.parametrize("ref", GOLDEN["dtv"], ids=_dtv_id)
def test_product_dtv_batch_matches_reference_trace(ref):
    """Draft-then-verify: the same rounds, drafts, verify cascades, bonus
    tokens, rollbacks and per-tick unions as the reference's generate_dtv_batch."""
    blocks = StubBatchBlocks(ref["T_total"], ref["B"])
    emus = None if ref["alpha"] is None else [EmulatedAcceptance(ref["alpha"], seed=1000 + b) for b in range(ref["B"])]
    bt = sb.generate_dtv_batch(blocks, stub_prompts(ref["B"], 5), ref["max_new_tokens"],
                               SsdPolicy(T_total=ref["T_total"], T_draft=ref["T_draft"]), ref["draft_length"], emus)
    got = trace_record(bt, blocks, blocks.last_cache, emus)
    if ref["calls"] is None:
        got["calls"] = None
    want = {k: v for k, v in _strip(ref).items() if k != "draft_length"}
    assert got == want


def test_reference_dtv_traces_are_lossless():
    """On the golden data itself: DtV with real comparisons commits exactly
    the sequential (AR) stub tokens -- verify runs every source to full depth."""
    for ref in GOLDEN["dtv"]:
        if ref["alpha"] is not None:
            continue
        blocks = StubBatchBlocks(ref["T_total"], ref["B"])
        bt = sb.ar_generate_batch(blocks, stub_prompts(ref["B"], 5), ref["max_new_tokens"])
        assert [list(t.tokens) for t in bt.per_seq] == [p["tokens"] for p in ref["per_seq"]], _dtv_id(ref)


@pytest.mark.parametrize("ref", GOLDEN["ar"], ids=_case_id)
def test_ar_batch_matches_reference_trace(ref):
    blocks = StubBatchBlocks(ref["T_total"], ref["B"])
    bt = sb.ar_generate_batch(blocks, stub_prompts(ref["B"], 5), ref["max_new_tokens"])
    assert trace_record(bt, blocks, blocks.last_cache, None) == _strip(ref)
    blocks = StubBatchBlocks(ref["T_total"], ref["B"])
    res = osched.ar_batch(blocks, stub_prompts(ref["B"], 5).tolist(), ref["max_new_tokens"], ref["T_total"])
    assert trace_record(res, blocks, blocks.last_cache, None) == _strip(ref)


def test_reference_traces_are_lossless():
    """On the golden data itself: WFD with real comparisons commits exactly the
    sequential (AR) tokens for the same model, prompts and length."""
    ar = {(r["B"], r["T_total"], r["max_new_tokens"]): [s["tokens"] for s in r["per_seq"]] for r in GOLDEN["ar"]}
    checked = 0
    for r in GOLDEN["wfd"]:
        key = (r["B"], r["T_total"], r["max_new_tokens"])
        if r["alpha"] is None and key in ar:
            assert [s["tokens"] for s in r["per_seq"]] == ar[key]
            checked += 1
    assert checked >= 8


def test_alpha_extremes():
    for r in GOLDEN["wfd"]:
        for s in r["per_seq"]:
            if r["alpha"] == 1.0:
                assert s["n_drafts_rejected"] == 0 and s["n_drafts_accepted"] == s["n_drafts_proposed"]
            if r["alpha"] == 0.0:
                assert s["n_drafts_accepted"] == 0 and s["n_rollback_events"] == s["n_drafts_proposed"]
            assert len(s["tokens"]) == r["max_new_tokens"]
