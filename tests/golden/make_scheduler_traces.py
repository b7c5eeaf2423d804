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

It also loads the single-sequence schedulers -- src/decoding/scheduler.py
(generate_wavefront_dynamic, generate_draft_then_verify) and
src/decoding/scheduler_emu.py (generate_wavefront_emu, generate_dtv_emu) --
and drives them with stub_model.StubRecursiveBlocks mixed into the
reference's own abstract RecursiveBlocks (src/decoding/blocks.py), with the
reference's WavefrontState / ActiveToken. Those traces (tokens, counters,
rollbacks, per-call schedule, emulated draws; greedy, emulated alpha and eos
stops) land in scheduler_single_traces.json.

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
from stub_model import (StubBatchBlocks, StubRecursiveBlocks, single_record, stub_prompts,  # noqa: E402
                        trace_record)


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


SINGLE = dict(
    wfd_schedule=((4, 1), (4, 2), (4, 4), (8, 2), (16, 2)),
    dtv_schedule=((4, 1), (4, 2), (8, 2)),
    max_new=(1, 2, 9, 33),
)


def single_traces() -> dict:
    sched = importlib.import_module(PKG + ".scheduler")
    sched_emu = importlib.import_module(PKG + ".scheduler_emu")
    blocks_mod = importlib.import_module(PKG + ".blocks")
    state_mod = importlib.import_module(PKG + ".state")
    emu_mod = importlib.import_module(PKG + ".emu")
    pol_mod = importlib.import_module(PKG + ".policy")
    Blocks = type("ReferenceStubBlocks", (StubRecursiveBlocks, blocks_mod.RecursiveBlocks),
                  {"state_cls": state_mod.WavefrontState})
    prompt = stub_prompts(1, 5)[0]
    out = {"source": "reference src/decoding/scheduler.py generate_wavefront_dynamic / generate_draft_then_verify, "
                     "src/decoding/scheduler_emu.py generate_wavefront_emu / generate_dtv_emu",
           "stub": "tests/golden/stub_model.py StubRecursiveBlocks (vocab=50, salt=0), prompt stub_prompts(1, 5)[0]",
           "wfd": [], "dtv": []}

    def run_wfd(T_total, T_draft, N, agree, alpha, eos, seed=7):
        blocks = Blocks(T_total, agree)
        policy = pol_mod.SsdPolicy(T_total=T_total, T_draft=T_draft)
        emu = None if alpha is None else emu_mod.EmulatedAcceptance(alpha, seed=seed)
        if alpha is None:
            toks, tr = sched.generate_wavefront_dynamic(blocks, prompt, N, policy, eos_token_id=eos)
        else:
            toks, tr = sched_emu.generate_wavefront_emu(blocks, prompt, N, policy, emu=emu, eos_token_id=eos)
        rec = single_record(toks, tr, blocks, emu, keep_calls=N <= 9)
        rec.update(T_total=T_total, T_draft=T_draft, max_new_tokens=N, agree_pct=agree, alpha=alpha, seed=seed,
                   eos=eos)
        return rec

    def run_dtv(T_total, T_draft, K, N, agree, alpha, eos, seed=7):
        blocks = Blocks(T_total, agree)
        policy = pol_mod.SsdPolicy(T_total=T_total, T_draft=T_draft)
        emu = None if alpha is None else emu_mod.EmulatedAcceptance(alpha, seed=seed)
        if alpha is None:
            toks, tr = sched.generate_draft_then_verify(blocks, prompt, N, policy, K, eos_token_id=eos)
        else:
            toks, tr = sched_emu.generate_dtv_emu(blocks, prompt, N, policy, K, emu=emu, eos_token_id=eos)
        rec = single_record(toks, tr, blocks, emu, keep_calls=N <= 9)
        rec.update(T_total=T_total, T_draft=T_draft, draft_length=K, max_new_tokens=N, agree_pct=agree,
                   alpha=alpha, seed=seed, eos=eos)
        return rec

    for (T, Td), N, agree in itertools.product(SINGLE["wfd_schedule"], SINGLE["max_new"], (70, 95)):
        out["wfd"].append(run_wfd(T, Td, N, agree, None, None))
    for (T, Td), N, alpha in itertools.product(SINGLE["wfd_schedule"], (9, 33), (0.0, 0.5, 0.9, 1.0)):
        out["wfd"].append(run_wfd(T, Td, N, 70, alpha, None))
    for (T, Td), K, N, agree in itertools.product(SINGLE["dtv_schedule"], (1, 3, 4), SINGLE["max_new"], (70, 95)):
        out["dtv"].append(run_dtv(T, Td, K, N, agree, None, None))
    for (T, Td), K, alpha in itertools.product(SINGLE["dtv_schedule"], (1, 4), (0.0, 0.5, 1.0)):
        out["dtv"].append(run_dtv(T, Td, K, 33, 70, alpha, None))
    # eos stops: the eos id is the 7th token of the run without one
    for T, Td in ((4, 1), (8, 2)):
        ref = run_wfd(T, Td, 33, 70, None, None)
        out["wfd"].append(run_wfd(T, Td, 33, 70, None, ref["tokens"][6]))
        out["wfd"].append(run_wfd(T, Td, 33, 70, 0.5, ref["tokens"][6]))
        ref = run_dtv(T, Td, 3, 33, 70, None, None)
        out["dtv"].append(run_dtv(T, Td, 3, 33, 70, None, ref["tokens"][6]))
    # the reference's emulated-alpha gate shape (experiments/exp4_emu/verify_step1.py:84-95):
    # T_total 4, T_draft 1, 384 tokens, seed 7, alpha 0.5 / 0.8; draft-then-verify with draft length 4
    for alpha in (0.5, 0.8):
        out["wfd"].append(run_wfd(4, 1, 384, 70, alpha, None))
        out["dtv"].append(run_dtv(4, 1, 4, 384, 70, alpha, None))
    return out


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
    single = single_traces()
    path = os.path.join(HERE, "scheduler_single_traces.json")
    with open(path, "w") as f:
        json.dump(single, f, separators=(",", ":"))
    print(f"wrote {len(single['wfd'])} single wfd + {len(single['dtv'])} single dtv traces -> {path} "
          f"({os.path.getsize(path)} bytes)")


if __name__ == "__main__":
    main()
