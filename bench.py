"""Benchmark of the MI355X wavefront decode step (one GPU).

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--quick] [--no-cpu] [--only LIST]

Prints ONE JSON line. `value` is bs=1 decode tokens/s of greedy wavefront
decoding on the 2048-d bf16 looped LM (2 prelude + 4-layer core looped 16
times + 2 coda, 16 heads x 128, SwiGLU 5632, V=32000, random init N(0, 0.02)
seed 0): 512-token prompt (uniform ids, seed 0), 256 new tokens, T_total=16,
T_draft=2 (wavefront width 8), real argmax acceptance decided on the device.
A step is one whole 256-token decode from the prefilled prompt (the prompt
cache is reused, prefill is outside the timed region; graphs are captured in
the warm-up steps); value = the 255 tokens each step decodes (the first comes
from the prefill) x steps / timed seconds. Every step's tokens are checked
against sequential looped decode of the same prompt in the same run.

Extra fields: the end-to-end fraction of the HBM roofline for the headline
(algorithmic bytes of every launched pass over the wall time); sequential
decode; acceptance emulated at alpha 0.9 (the reference's exp4 setting) and
draft-then-verify; greedy decode on the same model with an adapter that makes
every draft exact; bs=32 with ragged prompts U[128, 2048] and generation
lengths U[64, 512] at emulated alpha 0.5 / 0.7 / 0.9 and greedy; the
wavefront attention op alone (bf16, 16 heads x 64, W=8, L in {1k, 4k, 16k})
and at the 2048-d decode shapes; a long-context GQA decode tick and the
long-context configuration end to end; causal prefill attention on MFMA; the
per-shape weight-stream linears at 8 rows; and the CPU oracle on bounded
samples of the workloads on this host's cores.

`roofline` is the wavefront attention kernel at the headline's shape (one
layer tick of the 2048-d model at bs=1: 8 rows x 16 heads x Dh 128 over
512..778-key prefixes), the kernel the decode target is stated for;
`extra.roofline_linear` is the largest single kernel of that tick, the
gate|up projection with the SwiGLU epilogue at 8 rows. Both take `achieved`
from HIP events around graph replays on the launch stream and `traffic` from
the committed rocprofv3 FETCH_SIZE / WRITE_SIZE passes.

Opt-in sections (`--only`, never part of the default run): attnkeys (the
bs=1 attention launch against its key count), attnoverlap (Wqkv and the
attention in sequence and side by side), foldlin (the folded norm pairs'
linears and chains against separate norms), linsweep (a few-row linear's time
against its weight bytes) and tick (a bs=1 tick's GPU and host time).
"""
from __future__ import annotations

import argparse
import json
import math
import os
import platform
import sys
import time

REPO = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, REPO)

HBM_PEAK_GBS = 8000.0
MALL_BYTES = 256e6
MFMA_BF16_PEAK_TFLOPS = 2500.0  # dense bf16 MFMA, MI355X


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=3)
    ap.add_argument("--warmup", type=int, default=1)
    ap.add_argument("--quick", action="store_true", help="fewer extras (development)")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU oracle baseline")
    ap.add_argument("--only", default="", help="comma list of sections: bs1,roofline,attn,linrows,bs32,prefill,c5,gqa,cpu (and the opt-in attnkeys, attnoverlap, foldlin, linsweep, tick)")
    ap.add_argument("--eager", action="store_true", help="launch every pass eagerly (no hipGraph capture)")
    return ap.parse_args()


# ---------------------------------------------------------------------------
def timed(fn, iters: int, stream=None) -> float:
    """Average milliseconds per call with HIP events on the launch stream."""
    import torch

    st = stream or torch.cuda.current_stream()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(st)
    for i in range(iters):
        fn(i)
    e1.record(st)
    e1.synchronize()
    return e0.elapsed_time(e1) / iters


def attn_bench(dev, n, H, Hkv, Dh, lens, iters=24):
    """Wavefront attention alone over the engine's cache layout (head-major
    blocks of S rows, one per query's slot); rotates KV sets totalling > 512 MB
    so the 256 MB MALL cannot serve repeats. Returns (us/call, algorithmic bytes)."""
    import torch
    from wavefront_decoding_amd import ops

    S = max(lens) + 1
    per_set = n * S * Hkv * Dh * 2 * 2
    nsets = max(3, math.ceil(2 * MALL_BYTES / per_set) + 1)
    g = torch.Generator(device=dev).manual_seed(0)
    sets = [(torch.randn(n, Hkv, S, Dh, device=dev, dtype=torch.bfloat16, generator=g),
             torch.randn(n, Hkv, S, Dh, device=dev, dtype=torch.bfloat16, generator=g)) for _ in range(nsets)]
    q = torch.randn(n, H, Dh, device=dev, dtype=torch.bfloat16, generator=g)
    rb = torch.tensor([i * S for i in range(n)], dtype=torch.int64, device=dev)
    kl = torch.tensor(lens, dtype=torch.int32, device=dev)
    out = torch.empty_like(q)
    ws = ops.attn_workspace(n, H, Dh, max(lens), dev)
    def loop():
        for i in range(iters):
            ops.attn_decode(q, sets[i % nsets][0], sets[i % nsets][1], rb, kl, kv_len_max=max(lens), out=out,
                            workspace=ws)

    # captured once, so the launches run back to back (no host gaps between them)
    loop()
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        loop()
    graph.replay()
    ms = timed(lambda i: graph.replay(), 3) / iters
    del graph
    by = sum(lens) * Hkv * Dh * 2 * 2 + 2 * n * H * Dh * 2
    del sets
    torch.cuda.empty_cache()
    return ms * 1e3, by


def linear_roofline(dev, cfg, n: int, iters: int = 24):
    """The weight-stream linear kernel at the decode shapes of one R tick
    (n rows): per shape, average launch duration (HIP events on the launch
    stream around graph replays of `iters` back-to-back launches) and
    algorithmic bytes (W + x + y) per launch, over rotating weight copies
    (> 512 MB, so HBM, not the MALL, serves every launch). Returns
    {name: (us, bytes)}."""
    import torch
    from wavefront_decoding_amd import ops

    c = cfg
    D = c.d_model
    shapes = [("fc_swiglu", 2 * c.ffn, D, True), ("Wqkv", c.qkv_dim, D, False),
              ("proj", D, c.n_heads * c.head_dim, False), ("mlp_proj", D, c.ffn, False),
              ("adapter", D, 2 * D, False)]
    per_tick = sum(N * K * 2 for _, N, K, _ in shapes)
    copies = max(2, math.ceil(2 * MALL_BYTES / per_tick) + 1)
    g = torch.Generator(device=dev).manual_seed(1)
    Ws = [[ops.pack_linear((0.02 * torch.randn(N, K, device=dev, generator=g)).to(torch.bfloat16), swiglu=sw)
           for _, N, K, sw in shapes] for _ in range(copies)]
    x = torch.randn(n, 2 * D, device=dev, generator=g).to(torch.bfloat16)
    xf = torch.randn(n, c.ffn, device=dev, generator=g).to(torch.bfloat16)
    out = torch.empty(n, 2 * c.ffn, device=dev, dtype=torch.bfloat16)
    res = {}
    for j, (name, N, K, sw) in enumerate(shapes):
        src = xf if K == c.ffn else x

        def loop(j=j, K=K, sw=sw, src=src):
            for i in range(iters):
                ops.linear(src, Ws[i % copies][j], n=n, out=out, swiglu=sw, k=K)

        # captured once, so the launches are back to back (no host gaps between them)
        loop()
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            loop()
        graph.replay()
        ms = timed(lambda i: graph.replay(), 3) / iters
        width = N // 2 if sw else N
        res[name] = (ms * 1e3, N * K * 2 + n * K * 2 + n * width * 2)
        del graph
    del Ws
    torch.cuda.empty_cache()
    return res


def foldlin_section(args, dev, res):
    """Opt-in (`--only foldlin`): the few-row linears of one layer with and
    without their folded norm work, at the bs=1 tick's 1 and 8 rows: Wqkv
    (+RoPE, append) and gate|up + SwiGLU reading their row scales from group
    sums, proj / mlp_proj with the residual-prep epilogue, against the plain
    kernels and the separate residual norm they replace. Each form: average
    launch duration from HIP events around graph replays of 24 launches over
    rotating weight copies (> 512 MB)."""
    import torch
    from wavefront_decoding_amd import model as M
    from wavefront_decoding_amd import ops

    c = M.CONFIGS["looped-2048"]
    D, F, H, Hkv, Dh = c.d_model, c.ffn, c.n_heads, c.n_kv_heads, c.head_dim
    eps = c.norm_eps
    iters = 24
    shapes = {"Wqkv": (c.qkv_dim, D, False), "fc": (2 * F, D, True), "proj": (D, H * Dh, False),
              "mlp_proj": (D, F, False)}
    per = sum(N * K * 2 for N, K, _ in shapes.values())
    copies = max(2, math.ceil(2 * MALL_BYTES / per) + 1)
    g = torch.Generator(device=dev).manual_seed(3)
    bf = torch.bfloat16
    Ws = [{k: ops.pack_linear((0.02 * torch.randn(N, K, device=dev, generator=g)).to(bf), swiglu=sw)
           for k, (N, K, sw) in shapes.items()} for _ in range(copies)]
    wv = lambda: (1 + 0.1 * torch.randn(D, device=dev, generator=g)).to(bf)  # noqa: E731
    w2, w3 = wv(), wv()
    S = 1024
    cos = torch.rand(S, Dh // 2, device=dev, generator=g)
    sin = torch.rand(S, Dh // 2, device=dev, generator=g)
    kc = torch.zeros(16, Hkv, Dh, dtype=bf, device=dev)
    vc = torch.zeros_like(kc)
    out = {}
    for n in (1, 8):
        x = torch.randn(n, max(D, F), device=dev, generator=g).to(bf)
        r_in = torch.randn(n, D, device=dev, generator=g).to(bf)
        s_in = torch.rand(n, device=dev, generator=g) + 0.5
        r_out = torch.empty(n, D, dtype=bf, device=dev)
        A = torch.empty(n, D, dtype=bf, device=dev)
        gp = torch.empty(n * ops.FOLD_SLOTS * 2, dtype=torch.float32, device=dev)
        s_out = torch.empty(n, dtype=torch.float32, device=dev)
        y = torch.empty(n, 2 * F, dtype=bf, device=dev)
        q = torch.empty(n, H, Dh, dtype=bf, device=dev)
        pos = torch.arange(n, dtype=torch.int32, device=dev)
        fr = torch.arange(n, dtype=torch.int64, device=dev)
        ops.linear_prep(x, Ws[0]["proj"], n=n, r_in=r_in, s_in=s_in, w_in=w2, r_out=r_out, a_out=A, wa=w2, wb=w3,
                        part=gp)
        rs = ops.RowScale(D=D, eps=eps, two=True, part=gp, s_out=s_out)
        forms = {
            "Wqkv_plain": lambda W: ops.linear_qkv_rope_append(A, W["Wqkv"], pos, cos, sin, fr, kc, vc, H, Hkv, Dh,
                                                               n=n, q_out=q),
            "Wqkv_scaled": lambda W: ops.linear_qkv_rope_append(A, W["Wqkv"], pos, cos, sin, fr, kc, vc, H, Hkv, Dh,
                                                                n=n, q_out=q, rowscale=rs),
            "fc_plain": lambda W: ops.linear(A, W["fc"], n=n, out=y, swiglu=True),
            "fc_scaled": lambda W: ops.linear(A, W["fc"], n=n, out=y, swiglu=True, rowscale=rs),
            "proj_plain": lambda W: ops.linear(x, W["proj"], n=n, out=y, k=H * Dh),
            "proj_prep": lambda W: ops.linear_prep(x, W["proj"], n=n, r_in=r_in, s_in=s_in, w_in=w2, r_out=r_out,
                                                   a_out=A, wa=w2, wb=w3, part=gp),
            "mlp_proj_plain": lambda W: ops.linear(x, W["mlp_proj"], n=n, out=y, k=F),
            "mlp_proj_prep": lambda W: ops.linear_prep(x, W["mlp_proj"], n=n, r_in=r_in, s_in=s_in, w_in=w2,
                                                       r_out=r_out, a_out=A, wa=w2, wb=w3, part=gp),
            "residual_norm": lambda W: ops.add_rmsnorm(A, w2, eps, res=r_in, w2=w3, n=n, x_out=r_out, h_out=y[:, :D]),
            "final_norm": lambda W: ops.norm_prep(n=n, D=D, dtype=bf, eps=eps, a=r_out, wa=w2, h_out=A),
            # producer -> consumer chains, as a layer runs them
            "chain_norm": lambda W: (ops.linear(x, W["mlp_proj"], n=n, out=y, k=F),
                                     ops.add_rmsnorm(y[:, :D], w2, eps, res=r_in, w2=w3, n=n, x_out=r_out, h_out=A),
                                     ops.linear_qkv_rope_append(A, W["Wqkv"], pos, cos, sin, fr, kc, vc, H, Hkv,
                                                                Dh, n=n, q_out=q)),
            "chain_fold": lambda W: (ops.linear_prep(x, W["mlp_proj"], n=n, r_in=r_in, s_in=s_in, w_in=w2,
                                                     r_out=r_out, a_out=A, wa=w2, wb=w3, part=gp),
                                     ops.linear_qkv_rope_append(A, W["Wqkv"], pos, cos, sin, fr, kc, vc, H, Hkv,
                                                                Dh, n=n, q_out=q, rowscale=rs)),
        }
        row = {}
        for name, fn in forms.items():
            def loop(fn=fn):
                for i in range(iters):
                    fn(Ws[i % copies])
            loop()
            torch.cuda.synchronize()
            graph = torch.cuda.CUDAGraph()
            with torch.cuda.graph(graph):
                loop()
            graph.replay()
            row[name] = round(timed(lambda i: graph.replay(), 3) / iters * 1e3, 2)
            del graph
        out[f"n{n}"] = row
        log(f"foldlin n={n}: {row}")
    res["extra"]["fold_linears_us"] = out
    del Ws
    torch.cuda.empty_cache()


def tick_section(args, dev, res):
    """Opt-in (`--only tick`): where a bs=1 greedy tick's wall time goes. One
    greedy WFD step of the headline is recorded pass for pass (the run_passes
    calls the scheduler makes); the same passes are then replayed back to back
    with no accept-flag read between them (the C passes' expected tokens
    dropped), so the host stays ahead and HIP events measure the GPU's time
    per tick. The difference to the real step is the host's share of the
    critical path: reading the flags, routing, planning and launching the
    next tick while the GPU waits. A further step with host timestamps gives
    the mean host time of a launch call and of the routing between a verify
    tick's flags and the next launch call."""
    import torch
    from wavefront_decoding_amd import model as M
    from wavefront_decoding_amd.blocks import LoopedBlocksBatch
    from wavefront_decoding_amd.engine import LoopedModel
    from wavefront_decoding_amd.policy import SsdPolicy
    from wavefront_decoding_amd.scheduler_batch import generate_wavefront_batch, prefill_once

    cfg = M.CONFIGS["looped-2048"]
    L, N = 512, 256
    model = LoopedModel(cfg, M.init_weights(cfg, 0), dev, max_seq_len=L + N + 16, max_batch=1, use_graphs=True)
    prompt = torch.randint(0, cfg.vocab_size, (1, L), generator=torch.Generator().manual_seed(0)).to(dev)
    bb = LoopedBlocksBatch(model, batch_size=1)
    pf = prefill_once(bb, prompt)
    policy = SsdPolicy(cfg.T_total, 2)
    generate_wavefront_batch(bb, prompt, N, policy, prefilled=pf)  # captures every pass shape
    rec = []
    inner = model.run_passes

    def recording(cache, passes):
        rec.append([(k, list(sq), list(ps), None if (k == "C" or ex is None) else list(ex))
                    for k, sq, ps, ex in passes])
        return inner(cache, passes)

    model.run_passes = recording
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    generate_wavefront_batch(bb, prompt, N, policy, prefilled=pf)
    torch.cuda.synchronize()
    step_ms = (time.perf_counter() - t0) * 1e3
    # the host's own share: a second step with host timestamps around every
    # launch call and every accept-flag read (the scheduler's routing sits
    # between a verify tick's flags and the next launch call)
    flags_in, stamps = model.accept_flags, []

    def stamped_launch(cache, passes):
        a = time.perf_counter()
        r = inner(cache, passes)
        stamps.append(("launch", a, time.perf_counter()))
        return r

    def stamped_flags(timeout_s=30.0):
        a = time.perf_counter()
        r = flags_in(timeout_s)
        stamps.append(("flags", a, time.perf_counter()))
        return r

    model.run_passes, model.accept_flags = stamped_launch, stamped_flags
    generate_wavefront_batch(bb, prompt, N, policy, prefilled=pf)
    torch.cuda.synchronize()
    model.run_passes, model.accept_flags = inner, flags_in
    launch_us = [1e6 * (b - a) for k, a, b in stamps if k == "launch"]
    route_us = [1e6 * (nxt[1] - cur[2]) for cur, nxt in zip(stamps, stamps[1:])
                if cur[0] == "flags" and nxt[0] == "launch"]
    cache = pf.cache
    for passes in rec[:64]:  # warm: any pass shape not captured yet
        model.run_passes(cache, passes)
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    e0.record()
    for passes in rec:
        model.run_passes(cache, passes)
    e1.record()
    e1.synchronize()
    wall_ms = (time.perf_counter() - t0) * 1e3
    gpu_ms = e0.elapsed_time(e1)
    ticks = len(rec)
    out = {"ticks": ticks, "step_us_per_tick": round(step_ms / ticks * 1e3, 1),
           "replay_gpu_us_per_tick": round(gpu_ms / ticks * 1e3, 1),
           "replay_wall_us_per_tick": round(wall_ms / ticks * 1e3, 1),
           "passes_per_tick": round(sum(len(p) for p in rec) / ticks, 2),
           "host_launch_call_us": round(sum(launch_us) / max(len(launch_us), 1), 1),
           "host_route_after_flags_us": round(sum(route_us) / max(len(route_us), 1), 1),
           "rows_per_tick": {k: round(sum(len(ps) for pp in rec for kk, _, ps, _ in pp if kk == k) / ticks, 2)
                             for k in "PRC"}}
    res["extra"]["bs1_tick_breakdown"] = out
    log(f"tick: {out}")
    del model, bb, pf
    torch.cuda.empty_cache()


# ---------------------------------------------------------------------------
def _accepting(cfg, w, c: float) -> dict:
    """The same weights with adapter [c R | I] (R the random block on s,
    identity on e): c = 0 gives every loop step the input e, so every shallow
    draft equals the full-depth result and real greedy acceptance is 1."""
    import torch

    D = cfg.d_model
    ad = w["adapter"].clone()
    ad[:, D:] = torch.eye(D)
    ad[:, :D] *= c
    return dict(w, adapter=ad.to(cfg.torch_dtype).float())


def bs1_section(args, dev, res):
    """The headline: greedy WFD on the 2048-d model at bs=1, decode only."""
    import torch
    from wavefront_decoding_amd import model as M
    from wavefront_decoding_amd.blocks import LoopedBlocksBatch
    from wavefront_decoding_amd.emu import EmulatedAcceptance
    from wavefront_decoding_amd.engine import LoopedModel
    from wavefront_decoding_amd.policy import SsdPolicy
    from wavefront_decoding_amd.scheduler_batch import (ar_generate_batch, generate_dtv_batch,
                                                        generate_wavefront_batch, prefill_once)

    cfg = M.CONFIGS["looped-2048"]
    L, N, T_draft = 512, 256, 2
    t0 = time.perf_counter()
    w = M.init_weights(cfg, 0)
    model = LoopedModel(cfg, w, dev, max_seq_len=L + N + 16, max_batch=1, use_graphs=not args.eager)
    log(f"bs1: model ready in {time.perf_counter() - t0:.1f}s")
    prompt = torch.randint(0, cfg.vocab_size, (1, L), generator=torch.Generator().manual_seed(0)).to(dev)
    bb = LoopedBlocksBatch(model, batch_size=1)
    pf = prefill_once(bb, prompt)
    log(f"bs1: prefill {pf.prefill_s * 1e3:.1f} ms")
    policy = SsdPolicy(cfg.T_total, T_draft)

    # sequential looped decode of the same prompt: the lossless reference and the AR rate
    ar_generate_batch(bb, prompt, 8, prefilled=pf)  # graph capture
    t0 = time.perf_counter()
    ar = ar_generate_batch(bb, prompt, N, prefilled=pf)
    torch.cuda.synchronize()
    ar_dt = time.perf_counter() - t0
    ar_tokens = ar.per_seq[0].tokens
    res["extra"]["bs1_sequential_tokens_per_s"] = (N - 1) / ar_dt

    def step():  # real greedy acceptance, decided on the device
        return generate_wavefront_batch(bb, prompt, N, policy, prefilled=pf)

    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    b0 = model.bytes_moved
    t0 = time.perf_counter()
    traces = [step() for _ in range(args.steps)]
    torch.cuda.synchronize()
    dt = time.perf_counter() - t0
    moved = model.bytes_moved - b0
    for tr in traces:  # lossless: every step commits exactly the sequential tokens
        if tr.per_seq[0].tokens != ar_tokens:
            raise AssertionError("greedy WFD tokens differ from sequential decode")
    decoded = sum(tr.n_tokens - 1 for tr in traces)  # the first token of a step comes from the prefill
    res["value"] = decoded / dt
    res["ms_per_step"] = dt * 1e3 / args.steps
    tr = traces[-1]
    res["tokens_identical_to_sequential"] = True
    res["hbm_roofline_end_to_end"] = {
        "bytes_per_step": int(moved / args.steps), "achieved_GBs": round(moved / dt / 1e9, 1),
        "frac": round(moved / dt / 1e9 / HBM_PEAK_GBS, 4),
        "note": "algorithmic bytes of every pass the engine launched (weights of each pass's layers once, each "
                "row's slot prefix and append, activation rows, embedding / lm_head) over the timed steps' wall time"}
    res["extra"]["bs1_greedy"] = {"acceptance": round(tr.acceptance_rate, 4), "r_ticks_per_step": tr.n_r_calls,
                                  "c_passes_per_step": tr.n_c_calls}
    log(f"bs1: greedy WFD {res['value']:.1f} tok/s ({res['ms_per_step']:.1f} ms/step, acceptance "
        f"{tr.acceptance_rate:.3f}, {tr.n_r_calls} R ticks); sequential {res['extra']['bs1_sequential_tokens_per_s']:.1f}"
        f" tok/s; end-to-end HBM fraction {res['hbm_roofline_end_to_end']['frac']}")

    # the reference's throughput setting (exp4): acceptance emulated at alpha = 0.9
    emu_step = lambda: generate_wavefront_batch(bb, prompt, N, policy, [EmulatedAcceptance(0.9, 1000)],  # noqa: E731
                                                prefilled=pf)
    emu_step()
    torch.cuda.synchronize()
    b0 = model.bytes_moved
    t0 = time.perf_counter()
    et = [emu_step() for _ in range(args.steps)]
    torch.cuda.synchronize()
    edt = time.perf_counter() - t0
    res["extra"]["bs1_emulated_alpha0.9"] = {
        "tokens_per_s": round(sum(t.n_tokens - 1 for t in et) / edt, 1), "acceptance": round(et[-1].acceptance_rate, 3),
        "r_ticks_per_step": et[-1].n_r_calls, "hbm_frac": round((model.bytes_moved - b0) / edt / 1e9 / HBM_PEAK_GBS, 4),
        "note": "emulated Bernoulli(0.9) accept decisions (seed 1000), all compute runs; not token-identical by design"}
    log(f"bs1: emulated alpha 0.9: {res['extra']['bs1_emulated_alpha0.9']}")

    if not args.quick:
        # draft-then-verify on the same workload (the reference's exp4 comparison:
        # T_draft = 1, draft lengths 4 and 8, emulated alpha = 0.9)
        dtv = {}
        for dl in (4, 8):
            generate_dtv_batch(bb, prompt, 32, SsdPolicy(cfg.T_total, 1), dl, [EmulatedAcceptance(0.9, 1000)],
                               prefilled=pf)
            torch.cuda.synchronize()
            t0 = time.perf_counter()
            bt = generate_dtv_batch(bb, prompt, N, SsdPolicy(cfg.T_total, 1), dl,
                                    [EmulatedAcceptance(0.9, 1000)], prefilled=pf)
            torch.cuda.synchronize()
            dtv[f"dl{dl}"] = {"tokens_per_s": round((bt.n_tokens - 1) / (time.perf_counter() - t0), 1),
                              "acceptance": round(bt.acceptance_rate, 3), "r_ticks": bt.n_r_calls}
        res["extra"]["bs1_dtv_emulated_alpha0.9_Tdraft1"] = dtv
        log(f"bs1: DtV {dtv}")
    del model, bb, pf
    torch.cuda.empty_cache()

    if not args.quick:
        # real greedy acceptance where drafts hold: adapter [0 | I] (every draft is exact)
        m2 = LoopedModel(cfg, _accepting(cfg, w, 0.0), dev, max_seq_len=L + N + 16, max_batch=1,
                         use_graphs=not args.eager)
        b2 = LoopedBlocksBatch(m2, batch_size=1)
        pf2 = prefill_once(b2, prompt)
        ar2 = ar_generate_batch(b2, prompt, N, prefilled=pf2).per_seq[0].tokens
        generate_wavefront_batch(b2, prompt, N, policy, prefilled=pf2)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        g2 = generate_wavefront_batch(b2, prompt, N, policy, prefilled=pf2)
        torch.cuda.synchronize()
        gdt = time.perf_counter() - t0
        if g2.per_seq[0].tokens != ar2:
            raise AssertionError("greedy WFD tokens differ from sequential decode (accepting adapter)")
        res["extra"]["bs1_greedy_accepting_adapter"] = {
            "tokens_per_s": round((g2.n_tokens - 1) / gdt, 1), "acceptance": round(g2.acceptance_rate, 4),
            "r_ticks": g2.n_r_calls, "tokens_identical_to_sequential": True,
            "note": "same model with adapter [0 | I]: real greedy acceptance 1.0 (every draft exact)"}
        log(f"bs1: greedy, accepting adapter: {res['extra']['bs1_greedy_accepting_adapter']}")
        del m2, b2, pf2
        torch.cuda.empty_cache()
    return w


def linrows_section(args, dev, res):
    """The decode linears of the 2048-d model at the row counts of bs=32
    passes (17-256 rows): per shape, the launches the engine uses -- for the
    2048-column projections the split-K slice launch plus the row kernel of
    the folded norm pair after it (residual add, both norms' scales, the next
    linear's operand and norm a's output); gate|up + SwiGLU and Wqkv as one
    launch that scales its rows by the pair's precomputed scale -- timed like
    the n=8 shapes (HIP events around graph replays over rotating weight
    copies)."""
    import torch
    from wavefront_decoding_amd import model as M
    from wavefront_decoding_amd import ops

    c = M.CONFIGS["looped-2048"]
    D = c.d_model
    shapes = [("gate_up_swiglu", 2 * c.ffn, D, True), ("Wqkv", c.qkv_dim, D, False),
              ("proj", D, c.n_heads * c.head_dim, False), ("mlp_proj", D, c.ffn, False), ("adapter", D, 2 * D, False)]
    g = torch.Generator(device=dev).manual_seed(2)
    w1 = (1 + 0.1 * torch.randn(D, device=dev, generator=g)).to(torch.bfloat16)
    w2 = (1 + 0.1 * torch.randn(D, device=dev, generator=g)).to(torch.bfloat16)
    rows = (17, 64, 128, 256)
    part = torch.empty(4 * max(rows) * D, dtype=torch.float32, device=dev)
    out = {}
    iters = 12
    for name, N, K, sw in shapes:
        copies = max(2, math.ceil(2 * MALL_BYTES / (N * K * 2)) + 1)
        Ws = [ops.pack_linear((0.02 * torch.randn(N, K, device=dev, generator=g)).to(torch.bfloat16), swiglu=sw)
              for _ in range(copies)]
        for n in rows:
            x = torch.randn(n, K + 32, device=dev, generator=g).to(torch.bfloat16)[:, :K]
            res_ = torch.randn(n, D, device=dev, generator=g).to(torch.bfloat16)
            y = torch.empty(n, N // 2 if sw else N, device=dev, dtype=torch.bfloat16)
            Ao, ho = torch.empty(n, D, device=dev, dtype=torch.bfloat16), torch.empty(n, D, device=dev,
                                                                                      dtype=torch.bfloat16)
            scale = torch.rand(n, device=dev, generator=g) + 0.5
            rs = ops.RowScale(D=D, eps=1e-6, two=True, scale=scale)
            split = N == D

            def loop(Ws=Ws, x=x, y=y, n=n, sw=sw, split=split, res_=res_, Ao=Ao, ho=ho, scale=scale, rs=rs):
                for i in range(iters):
                    if split:
                        S = ops.linear_partials(x, Ws[i % copies], part, n=n)
                        ops.norm_prep(n=n, D=D, dtype=torch.bfloat16, eps=1e-6, part=part, nslices=S, r_in=res_,
                                      a_out=Ao, wa=w1, wb=w2, two=True, scale_out=scale, h_out=ho)
                    else:
                        ops.linear(x, Ws[i % copies], n=n, out=y, swiglu=sw, rowscale=rs)

            loop()
            torch.cuda.synchronize()
            graph = torch.cuda.CUDAGraph()
            with torch.cuda.graph(graph):
                loop()
            graph.replay()
            us = timed(lambda i: graph.replay(), 3) / iters * 1e3
            del graph
            wb = N * K * 2
            out[f"{name}_n{n}"] = {"us": round(us, 2), "weight_MB": round(wb / 1e6, 2),
                                   "GBs": round(wb / (us * 1e-6) / 1e9, 1),
                                   "form": "split-K slices + folded norm pair's row kernel" if split
                                   else "one launch, row-scaled"}
        del Ws
    torch.cuda.empty_cache()
    res["extra"]["linears_bs32_rows"] = out
    log(f"linrows: {out}")


def bs32_section(args, dev, res, w=None):
    import torch
    from wavefront_decoding_amd import model as M
    from wavefront_decoding_amd.blocks import LoopedBlocksBatch
    from wavefront_decoding_amd.emu import EmulatedAcceptance
    from wavefront_decoding_amd.engine import LoopedModel
    from wavefront_decoding_amd.policy import SsdPolicy
    from wavefront_decoding_amd.scheduler_batch import generate_wavefront_batch, prefill_once

    cfg = M.CONFIGS["looped-2048"]
    B = 32
    g = torch.Generator().manual_seed(0)
    plen = torch.randint(128, 2049, (B,), generator=g).tolist()
    glen = torch.randint(64, 513, (B,), generator=g).tolist()
    if args.quick:
        plen = [p // 4 for p in plen]
        glen = [x // 4 for x in glen]
    prompts = [torch.randint(0, cfg.vocab_size, (p,), generator=g).to(dev) for p in plen]
    w = w if w is not None else M.init_weights(cfg, 0)
    model = LoopedModel(cfg, w, dev, max_seq_len=max(plen) + max(glen) + 16, max_batch=B, use_graphs=not args.eager)
    bb = LoopedBlocksBatch(model, batch_size=B)
    t0 = time.perf_counter()
    pf = prefill_once(bb, prompts)
    log(f"bs32: prefill of {sum(plen)} prompt tokens in {time.perf_counter() - t0:.1f}s")
    policy = SsdPolicy(cfg.T_total, 2)
    out = {}
    generate_wavefront_batch(bb, prompts, [8] * B, policy, [EmulatedAcceptance(0.9, 1000 + b) for b in range(B)],
                             prefilled=pf)
    for alpha in (0.5, 0.7, 0.9):
        emus = [EmulatedAcceptance(alpha, 1000 + b) for b in range(B)]
        bt = generate_wavefront_batch(bb, prompts, glen, policy, emus, prefilled=pf)
        out[str(alpha)] = {"decode_tokens_per_s": round(bt.n_tokens / max(bt.walltime_decode_s, 1e-9), 1),
                           "tokens": bt.n_tokens, "r_ticks": bt.n_r_calls, "r_union_mean": round(bt.r_union_mean, 1),
                           "acceptance": round(bt.acceptance_rate, 3)}
        log(f"bs32: alpha={alpha}: {out[str(alpha)]}")
    res["extra"]["bs32"] = out
    res["extra"]["bs32_workload"] = ("32 sequences, prompts U[128,2048], generation U[64,512] (seed 0), "
                                     "T_total=16, T_draft=2, emulated acceptance seeds 1000+b, prefill excluded")
    # draft-then-verify on the same batch (the reference's exp4 setting: T_draft = 1,
    # draft length 4); its verify sources share slots, so their attention is grouped
    from wavefront_decoding_amd.scheduler_batch import generate_dtv_batch
    emus = [EmulatedAcceptance(0.9, 1000 + b) for b in range(B)]
    bt = generate_dtv_batch(bb, prompts, glen, SsdPolicy(cfg.T_total, 1), 4, emus, prefilled=pf)
    res["extra"]["bs32_dtv_alpha0.9_Tdraft1_dl4"] = {
        "decode_tokens_per_s": round(bt.n_tokens / max(bt.walltime_decode_s, 1e-9), 1), "tokens": bt.n_tokens,
        "r_ticks": bt.n_r_calls, "r_union_mean": round(bt.r_union_mean, 1), "acceptance": round(bt.acceptance_rate, 3)}
    log(f"bs32: DtV {res['extra']['bs32_dtv_alpha0.9_Tdraft1_dl4']}")
    del model, bb, pf
    torch.cuda.empty_cache()


def attn_section(args, dev, res):
    """The wavefront attention op alone: C2's shapes (16 heads x 64, W=8,
    L in {1k, 4k, 16k}), one layer-tick of the 2048-d model at bs=1 (8 rows,
    16 x 128 heads, prefixes 512..778 keys: the headline's shape) and at bs=32
    (112 ragged rows, 128..2527 keys). The bs=1 tick is also reported as a
    roofline object (the kernel the north-star target names)."""
    out = {}
    for L in (1024, 4096, 16384):
        us, by = attn_bench(dev, 8, 16, 16, 64, [L - 7 + i for i in range(8)])
        out[f"op_L{L}"] = {"us": round(us, 2), "MB": round(by / 1e6, 2), "GBs": round(by / us / 1e3, 1),
                           "frac": round(by / us / 1e3 / HBM_PEAK_GBS, 4)}
    shapes = {"decode_2048d_layer_tick": [512 + 38 * i for i in range(8)],
              "decode_2048d_bs32_tick": [128 + (i * 977) % 2400 for i in range(112)]}
    for name, lens in shapes.items():
        us, by = attn_bench(dev, len(lens), 16, 16, 128, lens, iters=24 if len(lens) <= 16 else 8)
        out[name] = {"us": round(us, 2), "MB": round(by / 1e6, 2), "GBs": round(by / us / 1e3, 1),
                     "frac": round(by / us / 1e3 / HBM_PEAK_GBS, 4)}
    res["extra"]["wavefront_attention"] = out
    t = out["decode_2048d_layer_tick"]
    res["roofline"] = {
        "bound": "hbm", "achieved": t["GBs"], "peak": HBM_PEAK_GBS, "unit": "GB/s", "frac": t["frac"],
        "traffic": None, "kernel": "wfd::attn_split_kernel<bf16_t, 128, 1, 1, 8, 32> (2048-d model, one bs=1 "
                                   "layer tick: 8 rows x 16 heads x Dh 128, prefixes 512..778 keys, one key split "
                                   "and two column halves each: 256 workgroups)",
        "bytes_per_launch": int(t["MB"] * 1e6), "avg_launch_us": t["us"]}
    _attach_traffic(res["roofline"], "wavefront_attention_c3_tick_traffic.json")
    log(f"attn: {out}")
    _calibration_copy(dev)


def attnkeys_section(args, dev, res):
    """Opt-in (`--only attnkeys`): the bs=1 tick's attention launch (8 rows x
    16 heads x Dh 128, two column halves: 256 workgroups) with every row at
    the same key count, from 1 key up, and one row alone. The 1-key launch is
    the launch's fixed part (dispatch, the row-table and first K/V loads, the
    wave merge, the store); each further round of 8 waves x 32-key tiles
    adds its bytes at the rate the chip streams them."""
    out = {}
    for L in (1, 32, 64, 128, 256, 512, 650, 1024):
        us, by = attn_bench(dev, 8, 16, 16, 128, [L] * 8)
        out[f"tick8_L{L}"] = {"us": round(us, 2), "GBs": round(by / us / 1e3, 1)}
    for L in (1, 256, 650, 1024):
        us, by = attn_bench(dev, 1, 16, 16, 128, [L])
        out[f"row1_L{L}"] = {"us": round(us, 2), "GBs": round(by / us / 1e3, 1)}
    res["extra"]["attention_key_sweep"] = out
    log(f"attnkeys: {out}")


def linsweep_section(args, dev, res):
    """Opt-in (`--only linsweep`): the few-row linear's time against its
    weight bytes -- a plain 2048-input bf16 linear over 4096..8192 output
    columns at 1 and 8 rows, each timed like the n=8 shapes (HIP events
    around graph replays of 24 launches over rotating weight copies). The
    fit time = fixed part + bytes / rate separates the per-launch fixed part
    from the streaming rate."""
    import torch
    from wavefront_decoding_amd import ops

    g = torch.Generator(device=dev).manual_seed(2)
    K, iters = 2048, 24
    out, pts = {}, {1: [], 8: []}
    for N in (4096, 5120, 6144, 7168, 8192):
        copies = max(2, math.ceil(2 * MALL_BYTES / (N * K * 2)) + 1)
        Ws = [ops.pack_linear((0.02 * torch.randn(N, K, device=dev, generator=g)).to(torch.bfloat16))
              for _ in range(copies)]
        for n in (1, 8):
            x = torch.randn(n, K + 32, device=dev, generator=g).to(torch.bfloat16)[:, :K]
            y = torch.empty(n, N, device=dev, dtype=torch.bfloat16)

            def loop(Ws=Ws, x=x, y=y, n=n):
                for i in range(iters):
                    ops.linear(x, Ws[i % len(Ws)], n=n, out=y)

            loop()
            torch.cuda.synchronize()
            graph = torch.cuda.CUDAGraph()
            with torch.cuda.graph(graph):
                loop()
            graph.replay()
            us = timed(lambda i: graph.replay(), 3) / iters * 1e3
            del graph
            out[f"N{N}_n{n}"] = round(us, 2)
            pts[n].append((N * K * 2, us))
        del Ws
    for n, p in pts.items():  # least-squares line us = a + bytes / rate
        xs, ys = [b for b, _ in p], [u for _, u in p]
        mx, my = sum(xs) / len(xs), sum(ys) / len(ys)
        slope = sum((a - mx) * (b - my) for a, b in zip(xs, ys)) / sum((a - mx) ** 2 for a in xs)
        out[f"fit_n{n}"] = {"fixed_us": round(my - slope * mx, 2), "rate_GBs": round(1e-3 / slope, 1)}
    res["extra"]["linear_bytes_sweep"] = out
    log(f"linsweep: {out}")
    torch.cuda.empty_cache()


def attnoverlap_section(args, dev, res):
    """Opt-in (`--only attnoverlap`): how much of one bs=1 layer's Wqkv +
    attention pair a form that overlaps them could hide, at the headline's
    layer tick (8 rows; Wqkv 6144 x 2048 with the folded norm pair's row scale
    from group sums, RoPE and the slot append; attention over 512..778-key
    prefixes, 16 heads x 128). Per iteration of a captured graph, timed with
    HIP events: the Wqkv launch alone, the attention launch alone, the two in
    order on one stream (the dependent pair the decode runs), the attention
    alone on a side branch (the fork / join's own cost), and the two on
    parallel branches of the graph (the attention reads q and a KV set that
    the concurrent Wqkv does not write). Weight copies and KV sets rotate over
    > 512 MB. The parallel figure bounds any overlapped form from below: such
    a form must still wait for its rows' q before the first QK^T."""
    import torch
    from wavefront_decoding_amd import model as M
    from wavefront_decoding_amd import ops

    c = M.CONFIGS["looped-2048"]
    n, H, Hkv, Dh, D = 8, c.n_heads, c.n_kv_heads, c.head_dim, c.d_model
    lens = [512 + 38 * i for i in range(n)]
    S = max(lens) + 1
    g = torch.Generator(device=dev).manual_seed(3)
    per = (H + 2 * Hkv) * Dh * D * 2 + n * S * Hkv * Dh * 2 * 2
    ns = max(3, math.ceil(2 * MALL_BYTES / per) + 1)
    Ws = [ops.pack_linear((0.02 * torch.randn((H + 2 * Hkv) * Dh, D, device=dev, generator=g)).to(torch.bfloat16))
          for _ in range(ns)]
    kv = [(torch.randn(n, Hkv, S, Dh, device=dev, generator=g).to(torch.bfloat16),
           torch.randn(n, Hkv, S, Dh, device=dev, generator=g).to(torch.bfloat16)) for _ in range(ns)]
    x = torch.randn(n, D + 32, device=dev, generator=g).to(torch.bfloat16)[:, :D]
    part = torch.rand(n * ops.FOLD_SLOTS * 2, device=dev, generator=g) + 0.5
    rs = ops.RowScale(D=D, eps=c.norm_eps, two=True, part=part)
    pos = torch.tensor([L - 1 for L in lens], dtype=torch.int32, device=dev)
    kl = torch.tensor(lens, dtype=torch.int32, device=dev)
    rb = torch.tensor([i * S for i in range(n)], dtype=torch.int64, device=dev)
    fr = rb + pos.to(torch.int64)
    ang = torch.rand(S, Dh // 2, device=dev, generator=g) * 6.28
    cos_t, sin_t = torch.cos(ang).contiguous(), torch.sin(ang).contiguous()
    q = torch.empty(n, H, Dh, device=dev, dtype=torch.bfloat16)
    q_prev = torch.randn(n, H, Dh, device=dev, generator=g).to(torch.bfloat16)
    o = torch.empty_like(q)
    ws = ops.attn_workspace(n, H, Dh, max(lens), dev)
    iters = 24

    def wqkv(i):
        kc, vc = kv[(i + 1) % ns]
        ops.linear_qkv_rope_append(x, Ws[i % ns], pos, cos_t, sin_t, fr, kc, vc, H, Hkv, Dh, n=n, q_out=q,
                                   rowscale=rs)

    def attn(i, qq):
        kc, vc = kv[i % ns]
        ops.attn_decode(qq, kc, vc, rb, kl, kv_len_max=max(lens), out=o, workspace=ws)

    side = torch.cuda.Stream()

    def run(mode):
        cur = torch.cuda.current_stream()
        for i in range(iters):
            if mode == "wqkv":
                wqkv(i)
            elif mode == "attn":
                attn(i, q_prev)
            elif mode == "serial":
                wqkv(i)
                attn(i, q)
            elif mode == "fork_attn":  # the attention alone on the side branch: the fork / join's own cost
                side.wait_stream(cur)
                with torch.cuda.stream(side):
                    attn(i, q_prev)
                cur.wait_stream(side)
            else:  # two branches of the graph, joined at the end of every iteration
                side.wait_stream(cur)
                with torch.cuda.stream(side):
                    attn(i, q_prev)
                wqkv(i)
                cur.wait_stream(side)

    out = {}
    for mode in ("wqkv", "attn", "serial", "fork_attn", "parallel"):
        run(mode)
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            run(mode)
        graph.replay()
        out[f"{mode}_us"] = round(timed(lambda i: graph.replay(), 3) / iters * 1e3, 2)
        del graph
    out["overlap_bound_us"] = round(out["serial_us"] - out["parallel_us"], 2)
    # the same bound with the fork / join's own cost taken out of the parallel pair
    out["overlap_bound_net_us"] = round(out["serial_us"] - (out["parallel_us"] - (out["fork_attn_us"] - out["attn_us"])),
                                        2)
    res["extra"]["attention_overlap"] = out
    log(f"attnoverlap: {out}")
    del Ws, kv
    torch.cuda.empty_cache()


def gqa_section(args, dev, res):
    """Long-context GQA decode: one R tick for 4 sequences x W=16 rows over a
    32k random-filled prompt cache (prefill of 4 x 32k prompts is out of scope)."""
    import torch
    from wavefront_decoding_amd import model as M
    from wavefront_decoding_amd.engine import LoopedModel

    cfg = M.CONFIGS["looped-2048-gqa"]
    B, ctx, W = 4, 32768, 16
    us, by = attn_bench(dev, B * W, 16, 4, 128, [ctx + i for i in range(B * W)], iters=10)
    res["extra"]["gqa_attention"] = {"us": round(us, 1), "GB": round(by / 1e9, 3), "GBs": round(by / us / 1e3, 1),
                                     "frac": round(by / us / 1e3 / HBM_PEAK_GBS, 4)}
    log(f"gqa attention: {res['extra']['gqa_attention']}")
    if args.quick:
        return
    model = LoopedModel(cfg, M.init_weights(cfg, 0), dev, max_seq_len=ctx + 128 + 16, max_batch=B)
    cache = model.create_cache(B)
    g = torch.Generator(device=dev).manual_seed(2)
    for t in (cache.flat_k, cache.flat_v):
        for chunk in torch.split(t.view(-1), 1 << 28):
            chunk.normal_(generator=g)
    seqs = [b for b in range(B) for _ in range(W)]
    pos = [ctx + W - 1 - j for _ in range(B) for j in range(W)]
    steps = [2 * j for _ in range(B) for j in range(W)]
    tick = lambda i: model.core_union(cache, seqs, pos, steps)  # noqa: E731
    timed(tick, 1)
    ms = timed(tick, 5)
    kv = sum(p + 1 for p in pos) * cfg.n_kv_heads * cfg.head_dim * 2 * 2 * cfg.n_core
    res["extra"]["gqa_decode_tick"] = {"ms": round(ms, 3), "kv_GB": round(kv / 1e9, 2),
                                       "note": "B=4 x W=16 rows at depths 0,2,..,30; 32k random-filled context"}
    log(f"gqa tick: {ms:.2f} ms")
    del model, cache
    torch.cuda.empty_cache()


def prefill_section(args, dev, res):
    """Causal prefill attention on MFMA (bf16): one prompt per call, all heads,
    timed with HIP events; TFLOP/s counts 4*H*Dh flops per (query, key) pair
    of the causal triangle (QK^T and PV), against 2.5 PFLOP/s dense bf16. Also
    the whole-model prefill of the bs=1 prompt."""
    import torch
    from wavefront_decoding_amd import model as M
    from wavefront_decoding_amd import ops
    from wavefront_decoding_amd.engine import LoopedModel

    out = {}
    for name, H, Hkv, Dh, L in [("mha_L2048", 16, 16, 128, 2048), ("gqa_L32768", 16, 4, 128, 32768)]:
        g = torch.Generator(device=dev).manual_seed(0)
        K = torch.randn(1, Hkv, L, Dh, device=dev, generator=g).to(torch.bfloat16)
        V = torch.randn(1, Hkv, L, Dh, device=dev, generator=g).to(torch.bfloat16)
        q = torch.randn(L, H, Dh, device=dev, generator=g).to(torch.bfloat16)
        rb = torch.zeros(1, dtype=torch.int64, device=dev)
        qs = torch.tensor([0, L], dtype=torch.int32, device=dev)
        p0 = torch.zeros(1, dtype=torch.int32, device=dev)
        o = torch.empty_like(q)
        call = lambda i: ops.attn_prefill(q, K, V, rb, qs, p0, max_seg_len=L, out=o)  # noqa: E731
        call(0)
        torch.cuda.synchronize()
        iters = 5 if L > 8192 else 40
        us = timed(call, iters) * 1e3
        flops = 4.0 * H * Dh * L * (L + 1) / 2
        out[name] = {"us": round(us, 1), "TFLOPs": round(flops / us / 1e6, 1),
                     "frac_of_bf16_peak": round(flops / us / 1e6 / MFMA_BF16_PEAK_TFLOPS, 4)}
        del K, V, q, o
    res["extra"]["prefill_attention"] = out
    cfg = M.CONFIGS["looped-2048"]
    m = LoopedModel(cfg, M.init_weights(cfg, 0), dev, max_seq_len=640, max_batch=1)
    cache = m.create_cache(1)
    ids = torch.randint(0, cfg.vocab_size, (512,), generator=torch.Generator().manual_seed(0)).tolist()
    for _ in range(2):
        m.prefill_seq(cache, 0, ids)
    torch.cuda.synchronize()
    # HIP events around 5 back-to-back calls (the stream's span per call) ...
    res["extra"]["prefill_bs1_prompt_ms"] = round(timed(lambda i: m.prefill_seq(cache, 0, ids), 5), 2)
    # ... and the host's wall time of 5 calls, each synchronized
    walls = []
    for _ in range(5):
        t0 = time.perf_counter()
        m.prefill_seq(cache, 0, ids)
        torch.cuda.synchronize()
        walls.append((time.perf_counter() - t0) * 1e3)
    res["extra"]["prefill_bs1_prompt_wall_ms"] = {"median": round(sorted(walls)[2], 2), "min": round(min(walls), 2),
                                                  "max": round(max(walls), 2)}
    log(f"prefill: {out}; bs1 prompt (512 tokens, 68 layer passes) {res['extra']['prefill_bs1_prompt_ms']} ms "
        f"(HIP events, 5 calls); wall {res['extra']['prefill_bs1_prompt_wall_ms']}")
    del m, cache
    torch.cuda.empty_cache()


def c5_section(args, dev, res):
    """The long-context configuration end to end: the GQA looped model (16 q /
    4 kv heads, 4-layer core x 32), 4 sequences of 32768 uniform-random prompt
    tokens prefilled on the GPU (MFMA causal attention), then 128 new tokens
    each by WFD with T_draft = 2 (wavefront width 16) at emulated alpha = 0.9."""
    import torch
    from wavefront_decoding_amd import model as M
    from wavefront_decoding_amd.blocks import LoopedBlocksBatch
    from wavefront_decoding_amd.emu import EmulatedAcceptance
    from wavefront_decoding_amd.engine import LoopedModel
    from wavefront_decoding_amd.policy import SsdPolicy
    from wavefront_decoding_amd.scheduler_batch import generate_wavefront_batch, prefill_once

    cfg = M.CONFIGS["looped-2048-gqa"]
    B, ctx, N = 4, 32768, 128
    g = torch.Generator().manual_seed(0)
    prompts = [torch.randint(0, cfg.vocab_size, (ctx,), generator=g).to(dev) for _ in range(B)]
    model = LoopedModel(cfg, M.init_weights(cfg, 0), dev, max_seq_len=ctx + N + 16, max_batch=B,
                        use_graphs=not args.eager)
    bb = LoopedBlocksBatch(model, batch_size=B)
    t0 = time.perf_counter()
    pf = prefill_once(bb, prompts)
    prefill_s = time.perf_counter() - t0
    log(f"c5: prefill of {B} x {ctx} tokens in {prefill_s:.1f} s")
    policy = SsdPolicy(cfg.T_total, 2)
    generate_wavefront_batch(bb, prompts, [4] * B, policy, [EmulatedAcceptance(0.9, 1000 + b) for b in range(B)],
                             prefilled=pf)  # warm-up (graph capture)
    bt = generate_wavefront_batch(bb, prompts, N, policy, [EmulatedAcceptance(0.9, 1000 + b) for b in range(B)],
                                  prefilled=pf)
    res["extra"]["c5_long_context"] = {
        "decode_tokens_per_s": round(bt.n_tokens / max(bt.walltime_decode_s, 1e-9), 1), "tokens": bt.n_tokens,
        "r_ticks": bt.n_r_calls, "r_union_mean": round(bt.r_union_mean, 1), "acceptance": round(bt.acceptance_rate, 3),
        "prefill_s": round(prefill_s, 2), "kv_cache_GB": round(pf.cache.nbytes / 1e9, 1),
        "workload": "GQA 16q/4kv looped model, B=4 x 32768-token prompts, 128 new tokens each, T_total=32, "
                    "T_draft=2 (W=16), emulated alpha 0.9; decode rate excludes prefill"}
    log(f"c5: {res['extra']['c5_long_context']}")
    del model, bb, pf
    torch.cuda.empty_cache()


def roofline_section(args, dev, res):
    """Dominant kernel of the decode tick: the weight-stream linear. The
    headline figure is its largest stream, the gate|up projection with the
    SwiGLU epilogue, at the bs=1 wavefront width (8 rows)."""
    from wavefront_decoding_amd import model as M

    lin = linear_roofline(dev, M.CONFIGS["looped-2048"], 8)
    us, by = lin["fc_swiglu"]
    ach = by / (us * 1e-6) / 1e9
    rl = {"bound": "hbm", "achieved": round(ach, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
          "frac": round(ach / HBM_PEAK_GBS, 4), "traffic": None,
          "kernel": "wfd::linear_wide_kernel<bf16_t, bf16_t, 1, 1, false, 8> (gate|up 11264x2048 + SwiGLU, n=8 rows)",
          "bytes_per_launch": int(by), "avg_launch_us": round(us, 2)}
    _attach_traffic(rl, "linear_swiglu_n8_traffic.json")
    res["extra"]["roofline_linear"] = rl
    res["extra"]["linear_shapes_n8"] = {k: {"us": round(u, 2), "MB": round(b / 1e6, 2),
                                            "GBs": round(b / (u * 1e-6) / 1e9, 1)} for k, (u, b) in lin.items()}
    log(f"roofline: fc+SwiGLU linear {ach:.0f} GB/s over {us:.2f} us avg launch; shapes "
        f"{res['extra']['linear_shapes_n8']}")
    _calibration_copy(dev)


def _attach_traffic(rl: dict, name: str) -> None:
    """HBM bytes per launch of the roofline kernel at its shape, from the
    committed rocprofv3 FETCH_SIZE / WRITE_SIZE passes (a counter run cannot
    time itself), when the profile names the same kernel."""
    tpath = os.path.join(REPO, "profiles", name)
    if os.path.exists(tpath):
        with open(tpath) as f:
            t = json.load(f)
        if t.get("kernel", "") and rl["kernel"].startswith(t["kernel"]):
            rl["traffic"] = t["traffic_bytes"]
            rl["traffic_source"] = t["source"]


def _calibration_copy(dev) -> None:
    """A plain device copy of known size (256 MiB read + 256 MiB written):
    the scale for the HBM byte counters (FETCH_SIZE / WRITE_SIZE) read in the
    same run."""
    import torch

    a = torch.empty(256 << 20, dtype=torch.uint8, device=dev)
    b = torch.empty_like(a)
    for _ in range(3):
        b.copy_(a)
    torch.cuda.synchronize()
    del a, b


def _cpu_model() -> str:
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return platform.processor() or platform.machine()


def _threads() -> int:
    try:
        from threadpoolctl import threadpool_info
        return max(i["num_threads"] for i in threadpool_info())
    except Exception:  # threadpoolctl missing: numpy's BLAS defaults to one thread per core
        return os.cpu_count()


def cpu_section(args, res, w=None):
    """The oracle (numpy float32, this host's cores) on bounded samples of the
    workloads (reported baselines, not optimisation targets):
      C3 (the cpu_baseline object): greedy WFD of the 2048-d model over a
          random-filled 512-token prompt cache (the oracle prefill of
          512 x 68 layer passes is skipped);
      C1: the whole tiny configuration, 128-token prompt prefill and 64 WFD tokens;
      C4: one 112-row R tick of the 2048-d model, timed on 8 of its rows;
      C5: one 64-row R tick of the GQA model at 32k context, timed on 2 rows."""
    import numpy as np

    from oracle import scheduler as osched
    from oracle import state_init
    from oracle.looped_lm import OracleBatchBlocks, OracleLM
    from wavefront_decoding_amd import model as M

    threads = _threads()
    cpu = f"BLAS threads {threads} of {os.cpu_count()} cpus; cpu={_cpu_model()}"
    cfg = M.CONFIGS["looped-2048"]
    w = w if w is not None else M.init_weights(cfg, 0)
    wn = M.weights_numpy(w)
    L, N = 512, 16
    s0t = lambda p: M.initial_state_tokens(cfg, [p])[0].numpy()  # noqa: E731
    lm = OracleLM(cfg, wn, L + N + 8, 1, s0t, None)
    rng = np.random.default_rng(0)
    lm.Kc[:, :, :L] = rng.standard_normal(lm.Kc[:, :, :L].shape, dtype=np.float32)
    lm.Vc[:, :, :L] = rng.standard_normal(lm.Vc[:, :, :L].shape, dtype=np.float32)

    class Warm(OracleBatchBlocks):
        def prefill(self, prompts):
            logits = np.zeros((1, cfg.vocab_size), dtype=np.float32)
            logits[0, 7] = 1.0
            return self._Cache(), logits

    t0 = time.perf_counter()
    r = osched.wfd_batch(Warm(lm), [[0] * L], N, cfg.T_total, 2)
    dt = time.perf_counter() - t0
    toks = len(r.per_seq[0].tokens) - 1  # the first token comes from the (skipped) prefill
    res["cpu_baseline"] = {"value": round(toks / dt, 4), "unit": "tokens/s", "cores": threads, "kind": "port",
                           "sample": (f"oracle greedy WFD decode of {toks} tokens (T_total=16, T_draft=2, "
                                      f"{r.n_r_calls} R ticks, real argmax acceptance) on the 2048-d model in float32 "
                                      f"over a random-filled 512-token prompt cache; {dt:.1f} s; {cpu}")}
    log(f"cpu: {res['cpu_baseline']}")
    del lm
    legs = {}
    # C1: tiny fp32, whole configuration
    tc = M.CONFIGS["tiny"]
    tw = M.weights_numpy(M.init_weights(tc, 0))
    ids = np.random.default_rng(0).integers(0, tc.vocab_size, 128).tolist()
    t0 = time.perf_counter()
    tlm = OracleLM(tc, tw, 256, 1, lambda p: state_init.s0_token(tc.d_model, tc.state_std, tc.emb_scale, 0, p),
                   lambda n: state_init.s0_prefill(tc.d_model, tc.state_std, tc.emb_scale, 0, n))
    tr = osched.wfd_single(OracleBatchBlocks(tlm), ids, 64, tc.T_total, 2)
    legs["c1_full_run"] = {"seconds": round(time.perf_counter() - t0, 2), "tokens": len(tr.tokens),
                           "note": "tiny fp32 oracle: 128-token prompt prefill + 64 WFD tokens (T_draft 2)"}
    # C4: one R tick of a 112-row union, 8 rows timed
    lens = [128 + (i * 977) % 2400 for i in range(112)]
    lm = OracleLM(cfg, wn, max(lens) + 1, 1, None, None)
    sample = list(range(0, 112, 14))
    for i in sample:  # random K/V in the slots these rows read
        for l in range(cfg.n_core):
            sl = lm.slot_core(i % cfg.T_total, l)
            lm.Kc[sl, 0, : lens[i]] = rng.standard_normal(lm.Kc[sl, 0, : lens[i]].shape, dtype=np.float32)
            lm.Vc[sl, 0, : lens[i]] = rng.standard_normal(lm.Vc[sl, 0, : lens[i]].shape, dtype=np.float32)
    st = rng.standard_normal((2, cfg.d_model), dtype=np.float32)
    t0 = time.perf_counter()
    for i in sample:
        lm.core(0, lens[i] - 1, i % cfg.T_total, st[0], st[1])
    per_row = (time.perf_counter() - t0) / len(sample)
    legs["c4_r_tick"] = {"seconds_per_tick": round(per_row * 112, 3), "rows_timed": len(sample),
                         "note": "2048-d oracle, one R tick of a 112-row ragged union (prefixes 128..2527), "
                                 "extrapolated from the rows timed"}
    del lm
    # C5: GQA, 32k context: the oracle holds only the 4 core slots of one depth
    gc = M.CONFIGS["looped-2048-gqa"].with_(T_total=1)
    gw = M.weights_numpy(M.init_weights(gc, 0))
    ctx = 32768
    lm = OracleLM(gc, gw, ctx + 16, 1, None, None)
    for l in range(gc.n_core):
        sl = lm.slot_core(0, l)
        lm.Kc[sl, 0, :ctx] = rng.standard_normal(lm.Kc[sl, 0, :ctx].shape, dtype=np.float32)
        lm.Vc[sl, 0, :ctx] = rng.standard_normal(lm.Vc[sl, 0, :ctx].shape, dtype=np.float32)
    t0 = time.perf_counter()
    for j in range(2):
        lm.core(0, ctx + j, 0, st[0], st[1])
    per_row = (time.perf_counter() - t0) / 2
    legs["c5_r_tick"] = {"seconds_per_tick": round(per_row * 64, 2), "rows_timed": 2,
                         "note": "GQA 16q/4kv oracle over a random-filled 32k context, one R tick of "
                                 "B=4 x W=16 rows extrapolated from the rows timed"}
    del lm
    res["extra"]["cpu_legs"] = {"threads": threads, "cpu": _cpu_model(), **legs}
    log(f"cpu legs: {res['extra']['cpu_legs']}")


def main():
    args = parse()
    if args.gpus != 1:
        print(json.dumps({"error": "this build runs on one GPU only; multi-GPU sharding is a design note "
                                   "(no collectives are built)", "n_gpus": args.gpus}))
        sys.exit(2)
    import torch

    import __graft_entry__

    __graft_entry__.load_package()
    from wavefront_decoding_amd import _lib

    _lib.load()
    dev = torch.device("cuda:0")
    only = set(filter(None, args.only.split(",")))
    want = lambda s: not only or s in only  # noqa: E731
    res = {
        "metric": "decode tokens/s bs=1 & bs=32 (looped LM); wavefront-attn HBM GB/s vs peak",
        "value": None, "unit": "tokens/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": None, "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "bf16",
        "data": "synthetic (random-init weights N(0,0.02) seed 0, uniform random prompts seed 0)",
        "config": {"workload": "looped-2048 bf16 bs=1 greedy WFD decode (d=2048, 16x128 heads, SwiGLU 5632, "
                               "2 prelude + 4-layer core x 16 loops + 2 coda, V=32000): 512-token prompt, "
                               "256 new tokens, T_total=16, T_draft=2 (W=8), real argmax acceptance, tokens "
                               "checked identical to sequential decode; step = one 256-token decode, prefill excluded",
                   "batch": 1, "prompt_len": 512, "new_tokens": 256, "T_total": 16, "T_draft": 2,
                   "acceptance": "greedy (argmax compare on the device)"},
        "roofline": None, "cpu_baseline": None, "extra": {},
    }
    w = None
    if want("bs1"):
        w = bs1_section(args, dev, res)
    if want("roofline"):
        roofline_section(args, dev, res)
    if want("attn"):
        attn_section(args, dev, res)
    if want("linrows"):
        linrows_section(args, dev, res)
    if want("bs32") and not args.quick:
        bs32_section(args, dev, res, w)
    if want("prefill"):
        prefill_section(args, dev, res)
    if want("c5") and not args.quick:
        c5_section(args, dev, res)
    if want("gqa"):
        gqa_section(args, dev, res)
    if "foldlin" in only:  # opt-in only: not part of the default run
        foldlin_section(args, dev, res)
    if "tick" in only:  # opt-in only: not part of the default run
        tick_section(args, dev, res)
    if "linsweep" in only:  # opt-in only: not part of the default run
        linsweep_section(args, dev, res)
    if "attnoverlap" in only:  # opt-in only: not part of the default run
        attnoverlap_section(args, dev, res)
    if "attnkeys" in only:  # opt-in only: not part of the default run
        attnkeys_section(args, dev, res)
    if want("cpu") and not args.no_cpu:
        cpu_section(args, res, w)
    print(json.dumps(res))


if __name__ == "__main__":
    main()
