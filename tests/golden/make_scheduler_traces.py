"""Write golden scheduler traces from the REFERENCE's own batch scheduler.

Runs in the build container only (it reads the reference checkout at
/root/reference; the GPU box never runs it). It loads the reference's
parcae-free scheduler modules file by file -- src/decoding/scheduler_batch.py
and what it imports (batch_state, emu, policy, state, scheduler, blocks,
acceptance) -- under a private package name, bypassing
src/decoding/__init__.py (which imports the un-vendored parcae_lm), and drives
generate_wavefront_batch / ar_generate_batch / generate_dtv_batch with the
deterministic stub model of stub_model.py. The recorded vectors (tokens, counters, union sizes,
rollbacks, the per-call (seq, pos, step) schedule, emulated draws) land in
scheduler_traces.json next to this script.

    python tests/golden/make_scheduler_traces.py
"""
from __future__ import annotations

import importlib
import itertools
import json
import os
import sys
import types

HERE = os.path.dirname(os.path.abspath(__file__))
REF_DECODING = "/root/reference/src/decoding"
PKG = "_wfd_reference_decoding"

sys.path.insert(0, HERE)
from stub_model import StubBatchBlocks, stub_prompts, trace_record  # noqa: E402


def load_reference():
    pkg = types.ModuleType(PKG)
    pkg.__path__ = [REF_DECODING]
    sys.modules[PKG] = pkg
    sb = importlib.import_module(PKG + ".scheduler_batch")
    emu = importlib.import_module(PKG + ".emu")
    pol = importlib.import_module(PKG + ".policy")
    return sb, emu, pol


CASES = dict(
    B=(1, 3),
    schedule=((4, 1), (4, 2), (4, 4), (8, 2), (16, 2)),
    max_new=(1, 2, 9, 33),
    alpha=(None, 0.0, 0.5, 0.9, 1.0),
)


def main() -> None:
    sb, emu_mod, pol_mod = load_reference()
    out = {"source": "reference src/decoding/scheduler_batch.py generate_wavefront_batch / ar_generate_batch / "
                     "generate_dtv_batch",
           "stub": "tests/golden/stub_model.py (vocab=50, agree_pct=70, salt=0), prompt length 5",
           "wfd": [], "ar": [], "dtv": []}
    for B, (T_total, T_draft), N, alpha in itertools.product(*CASES.values()):
        blocks = StubBatchBlocks(T_total, B)
        prompts = stub_prompts(B, 5)
        emus = None if alpha is None else [emu_mod.EmulatedAcceptance(alpha, seed=0 * 100003 + 1000 + b)
                                           for b in range(B)]
        policy = pol_mod.SsdPolicy(T_total=T_total, T_draft=T_draft)
        bt = sb.generate_wavefront_batch(blocks, prompts, N, policy, emus)
        rec = trace_record(bt, blocks, blocks.last_cache, emus)
        if N > 9:
            rec["calls"] = None     # long runs keep tokens/counters only (fixture size)
        rec.update(B=B, T_total=T_total, T_draft=T_draft, max_new_tokens=N, alpha=alpha)
        out["wfd"].append(rec)
    for B, T_total, N in itertools.product((1, 3), (4, 8), (1, 9)):
        blocks = StubBatchBlocks(T_total, B)
        bt = sb.ar_generate_batch(blocks, stub_prompts(B, 5), N)
        rec = trace_record(bt, blocks, blocks.last_cache, None)
        rec.update(B=B, T_total=T_total, max_new_tokens=N)
        out["ar"].append(rec)
    for B, (T_total, T_draft), K, N, alpha in itertools.product(
            (1, 3), ((4, 1), (4, 2), (8, 2)), (1, 3), (1, 2, 9, 33), (None, 0.0, 0.5, 1.0)):
        blocks = StubBatchBlocks(T_total, B)
        emus = None if alpha is None else [emu_mod.EmulatedAcceptance(alpha, seed=1000 + b) for b in range(B)]
        policy = pol_mod.SsdPolicy(T_total=T_total, T_draft=T_draft)
        bt = sb.generate_dtv_batch(blocks, stub_prompts(B, 5), N, policy, K, emus)
        rec = trace_record(bt, blocks, blocks.last_cache, emus)
        if N > 9:
            rec["calls"] = None
        rec.update(B=B, T_total=T_total, T_draft=T_draft, draft_length=K, max_new_tokens=N, alpha=alpha)
        out["dtv"].append(rec)
    path = os.path.join(HERE, "scheduler_traces.json")
    with open(path, "w") as f:
        json.dump(out, f, separators=(",", ":"))
    print(f"wrote {len(out['wfd'])} wfd + {len(out['ar'])} ar + {len(out['dtv'])} dtv traces -> {path} "
          f"({os.path.getsize(path)} bytes)")


if __name__ == "__main__":
    main()
