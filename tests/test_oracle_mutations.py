"""Plant plausible mistakes in the oracle (on the CPU) and show the pinning
checks catch each one -- the checks are not a retyping of the oracle.

Each mutation patches one oracle function for the duration of the test and
re-runs the check that is meant to catch it; the check must now fail.
"""
from __future__ import annotations

import json
import os

import numpy as np
import pytest

from oracle import kernels as ok
from oracle import scheduler as osched
from tests import test_oracle_kernels as tk
from tests.golden.stub_model import StubBatchBlocks, stub_prompts, trace_record

_ATT = ok.attention
_ROPE = ok.rope
_RMS = ok.rmsnorm


def _fails(fn, *args):
    with pytest.raises(AssertionError):
        fn(*args)


def test_catches_dropped_softmax_scale(monkeypatch):
    monkeypatch.setattr(ok, "attention", lambda q, K, V, n, scale=None: _ATT(q, K, V, n, 1.0))
    _fails(tk.test_attention_matches_sdpa, 4, 4, 64, 50, 37)


def test_catches_off_by_one_cutoff(monkeypatch):
    monkeypatch.setattr(ok, "attention", lambda q, K, V, n, scale=None: _ATT(q, K, V, n - 1, scale))
    _fails(tk.test_attention_matches_sdpa, 4, 4, 64, 50, 37)


def test_catches_wrong_gqa_head_map(monkeypatch):
    def bad(q, K, V, n, scale=None):
        H, Hkv = q.shape[0], K.shape[1]
        G = H // Hkv
        perm = [(h % Hkv) * G + h // Hkv for h in range(H)]   # kv head h % Hkv instead of h // G
        out = _ATT(q[perm], K, V, n, scale)
        res = np.empty_like(out)
        res[perm] = out
        return res

    monkeypatch.setattr(ok, "attention", bad)
    _fails(tk.test_attention_special_cases)


def test_catches_transposed_kv(monkeypatch):
    monkeypatch.setattr(ok, "attention", lambda q, K, V, n, scale=None: _ATT(q, V, K, n, scale))
    _fails(tk.test_attention_matches_sdpa, 16, 4, 128, 300, 300)


def test_catches_rope_sign_flip(monkeypatch):
    monkeypatch.setattr(ok, "rope", lambda x, p, c, s: _ROPE(x, p, c, -s))
    _fails(tk.test_rope_is_complex_rotation)


def test_catches_rmsnorm_without_mean(monkeypatch):
    monkeypatch.setattr(ok, "rmsnorm", lambda x, w, eps: x / np.sqrt(np.sum(x * x, -1, keepdims=True) + eps) * w)
    _fails(tk.test_rmsnorm_matches_torch)


def test_catches_scheduler_mistakes(monkeypatch):
    golden = json.load(open(os.path.join(os.path.dirname(__file__), "golden", "scheduler_traces.json")))
    ref = next(r for r in golden["wfd"] if r["B"] == 3 and r["T_total"] == 8 and r["max_new_tokens"] == 9
               and r["alpha"] == 0.5)

    def run():
        blocks = StubBatchBlocks(ref["T_total"], 3)
        emus = [osched.Emu(0.5, 1000 + b) for b in range(3)]
        res = osched.wfd_batch(blocks, stub_prompts(3, 5).tolist(), 9, 8, ref["T_draft"], emus)
        got = trace_record(res, blocks, blocks.last_cache, emus)
        want = {k: v for k, v in ref.items() if k not in ("B", "T_total", "T_draft", "max_new_tokens", "alpha")}
        assert got == want

    run()  # unmutated: passes
    # a reject truncates the cache but leaves the in-flight tokens stepping
    orig_rb = osched._Seq.rollback
    monkeypatch.setattr(osched._Seq, "rollback", lambda self, pos, cache: cache.drop_positions_at_and_after(self.b, pos))
    _fails(run)
    monkeypatch.setattr(osched._Seq, "rollback", orig_rb)
    # inverted accept decision
    orig = osched.Emu.draw
    monkeypatch.setattr(osched.Emu, "draw", lambda self: not orig(self))
    _fails(run)
