"""Each benchmark configuration's own workload on the GPU, against the oracle
or against sequential decode (GPU).

* C1 (tiny fp32, 128-token prompt, 64 tokens): WFD at T_draft 1 and 2 commits
  the oracle's sequential tokens with the oracle's counters; captured graphs
  and the device token ring give the same tokens and counters as the oracle;
  the emulated-acceptance schedulers meet the reference's empirical-alpha
  gate over 384 tokens and match the oracle's emulated run.
* Accepted drafts under real greedy acceptance: an adapter [c R | I]
  (R the random init block) makes shallow drafts agree with the full depth
  (c = 0: every loop step sees e, so every draft is exact; c = 1 on the tiny
  model: a mix of accepts and rejects); WFD and draft-then-verify still
  commit exactly the sequential tokens, eager and captured.
* C3 (2048-d bf16, 512-token prompt): greedy WFD with T_draft = 2 (W = 8) for
  all 256 tokens commits exactly the sequential tokens, eager and captured, on
  the random-init model (drafts rejected) and on the accepting variant.
* C4 (2048-d bf16, B = 32, prompts U[128, 2048], generation U[64, 512]): the
  reference's batch gates (experiments/exp4_emu/verify_batch.py:88-141) over
  the whole workload: each sequence's tokens and counters equal its solo run
  (emulated alpha = 0.9 and 0.5), replicas of one prompt commit the same
  tokens, alpha = 0 next to alpha = 1 leaves the alpha = 1 sequence
  untouched, batch prefill equals single-sequence prefill, AR R calls =
  (N - 1) T_total, and real greedy batch WFD equals lockstep sequential
  decode; one ragged 256-row R tick (multi-split prefixes, grouped rows)
  against the oracle.
* C5 (GQA 16 q / 4 kv, Dh 128): decode attention over 32k-key prefixes
  (33 splits + the combine) against the oracle, and one R tick of the GQA
  model (16 rows at depths 0..30) against the oracle.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import kernels as ok
from oracle import scheduler as osched
from oracle import state_init
from oracle.looped_lm import OracleBatchBlocks, OracleLM
from tests.conftest import rel_err
from wavefront_decoding_amd import model as M
from wavefront_decoding_amd import ops
from wavefront_decoding_amd.blocks import LoopedBlocks, LoopedBlocksBatch
from wavefront_decoding_amd.emu import EmulatedAcceptance
from wavefront_decoding_amd.engine import LoopedModel
from wavefront_decoding_amd.policy import SsdPolicy
from wavefront_decoding_amd.scheduler import generate_draft_then_verify, generate_wavefront_dynamic
from wavefront_decoding_amd.scheduler_emu import generate_dtv_emu, generate_wavefront_emu
from wavefront_decoding_amd.scheduler_batch import ar_generate_batch, generate_wavefront_batch, prefill_once

pytestmark = pytest.mark.gpu

TINY = M.CONFIGS["tiny"]
C3 = M.CONFIGS["looped-2048"]
GQA = M.CONFIGS["looped-2048-gqa"]
MINI_BF16 = M.LoopedLMConfig("mini-bf16", 4096, 512, 4, 4, 128, 1536, 1, 2, 1, 8)


def _prompt(L, seed=0, V=4096):
    return torch.randint(0, V, (L,), generator=torch.Generator().manual_seed(seed))


def _round(a, cfg):
    return torch.from_numpy(a).to(cfg.torch_dtype).float().numpy()


def _oracle(cfg, w, S, B=1):
    wn = M.weights_numpy(w)
    s0t = lambda p: _round(state_init.s0_token(cfg.d_model, cfg.state_std, cfg.emb_scale, 0, p), cfg)  # noqa: E731
    s0p = lambda L: _round(state_init.s0_prefill(cfg.d_model, cfg.state_std, cfg.emb_scale, 0, L), cfg)  # noqa: E731
    return OracleBatchBlocks(OracleLM(cfg, wn, S, B, s0t, s0p))


def accepting(cfg, w, c: float) -> dict:
    """The same weights with adapter [c R | I]: R the random block acting on
    s, identity on e. c = 0 makes every loop step's input e, so the hidden
    state (and the draft) is the same at every depth."""
    D = cfg.d_model
    ad = w["adapter"].clone()
    ad[:, D:] = torch.eye(D)
    ad[:, :D] *= c
    return dict(w, adapter=ad.to(cfg.torch_dtype).float())


# ---------------------------------------------------------------------------
# C1: tiny fp32, 128-token prompt, 64 tokens
# ---------------------------------------------------------------------------
@pytest.fixture(scope="module")
def tiny_w():
    return M.init_weights(TINY, 0)


@pytest.mark.parametrize("graphs", [False, True])
@pytest.mark.parametrize("T_draft", [1, 2])
def test_c1_wfd_64_tokens_match_oracle(gpu, tiny_w, T_draft, graphs):
    ids = _prompt(128)
    N = 64
    print(f"[C1] T_draft={T_draft} graphs={graphs}", flush=True)
    blocks = LoopedBlocks(LoopedModel(TINY, tiny_w, gpu, max_seq_len=256, use_graphs=graphs))
    toks, trace = generate_wavefront_dynamic(blocks, ids.to(gpu), N, SsdPolicy(TINY.T_total, T_draft))
    oc = osched.wfd_single(_oracle(TINY, tiny_w, 256), ids.tolist(), N, TINY.T_total, T_draft)
    assert toks == oc.tokens and len(toks) == N
    assert trace.counters() == {k: getattr(oc, k) for k in trace.counters()}
    assert toks == osched.ar_single(_oracle(TINY, tiny_w, 256), ids.tolist(), N, TINY.T_total)


@pytest.mark.parametrize("alpha", [0.5, 0.8])
def test_emulated_alpha_gate_tiny(gpu, tiny_w, alpha):
    """The reference's emulated-acceptance gate (experiments/exp4_emu/
    verify_step1.py:84-95) on the device path: 384 tokens of
    generate_wavefront_emu and generate_dtv_emu (draft length 4) on the tiny
    model, T_total 4, T_draft 1, seed 7: the empirical acceptance is within
    0.06 of alpha; the WFD run's tokens and counters equal the oracle's
    emulated run, draw for draw."""
    ids = _prompt(128)
    blocks = LoopedBlocks(LoopedModel(TINY, tiny_w, gpu, max_seq_len=128 + 400, use_graphs=True))
    policy = SsdPolicy(TINY.T_total, 1)
    print(f"[emu gate] alpha={alpha}", flush=True)
    emu = EmulatedAcceptance(alpha, 7)
    toks, tr = generate_wavefront_emu(blocks, ids.to(gpu), 384, policy, emu=emu)
    assert len(toks) == 384 and abs(emu.empirical_rate - alpha) < 0.06, emu.empirical_rate
    oemu = osched.Emu(alpha, 7)
    oc = osched.wfd_single(_oracle(TINY, tiny_w, 128 + 400), ids.tolist(), 384, TINY.T_total, 1, emu=oemu)
    assert toks == oc.tokens
    assert tr.counters() == {k: getattr(oc, k) for k in tr.counters()}
    assert (emu.n_draws, emu.n_accepts) == (oemu.n_draws, oemu.n_accepts)
    emu = EmulatedAcceptance(alpha, 7)
    toks, tr = generate_dtv_emu(blocks, ids.to(gpu), 384, policy, 4, emu=emu)
    assert len(toks) == 384 and abs(emu.empirical_rate - alpha) < 0.06, emu.empirical_rate


def test_graph_batch_and_token_ring_match_oracle(gpu, tiny_w):
    """Captured batch WFD with ids kept in the device token ring (emulated
    acceptance) against the oracle's batch restatement: tokens, per-sequence
    counters and union sizes."""
    P = [_prompt(40, 4), _prompt(25, 5), _prompt(33, 6)]
    bb = LoopedBlocksBatch(LoopedModel(TINY, tiny_w, gpu, max_seq_len=128, max_batch=3, use_graphs=True))
    emus = [EmulatedAcceptance(0.6, 1000 + b) for b in range(3)]
    bt = generate_wavefront_batch(bb, [p.to(gpu) for p in P], [12, 9, 15], SsdPolicy(TINY.T_total, 2), emus)
    res = osched.wfd_batch(_oracle(TINY, tiny_w, 128, B=3), [p.tolist() for p in P], [12, 9, 15], TINY.T_total, 2,
                           [osched.Emu(0.6, 1000 + b) for b in range(3)])
    for b in range(3):
        assert bt.per_seq[b].tokens == res.per_seq[b].tokens
        assert bt.per_seq[b].counters() == {k: getattr(res.per_seq[b], k) for k in bt.per_seq[b].counters()}
    assert (bt.n_r_calls, bt.r_union_total, bt.r_union_max) == (res.n_r_calls, res.r_union_total, res.r_union_max)


# ---------------------------------------------------------------------------
# accepted drafts under real greedy acceptance
# ---------------------------------------------------------------------------
@pytest.mark.parametrize("graphs", [False, True])
def test_accepted_and_rejected_drafts_tiny(gpu, tiny_w, graphs):
    """c = 1 on the tiny model: some drafts accepted, some rejected; tokens
    and counters equal the oracle's, tokens equal sequential decode."""
    w = accepting(TINY, tiny_w, 1.0)
    ids = _prompt(32)
    blocks = LoopedBlocks(LoopedModel(TINY, w, gpu, max_seq_len=128, use_graphs=graphs))
    toks, tr = generate_wavefront_dynamic(blocks, ids.to(gpu), 30, SsdPolicy(TINY.T_total, 2))
    assert tr.n_drafts_accepted > 0 and tr.n_drafts_rejected > 0, tr.counters()
    oc = osched.wfd_single(_oracle(TINY, w, 128), ids.tolist(), 30, TINY.T_total, 2)
    assert toks == oc.tokens
    assert tr.counters() == {k: getattr(oc, k) for k in tr.counters()}
    ar, _ = blocks.ar_generate(ids.to(gpu), 30)
    assert toks == ar


@pytest.mark.parametrize("graphs", [False, True])
def test_accepted_drafts_bf16_wfd_and_dtv_lossless(gpu, graphs):
    """c = 0 on a bf16 model with the 2048-d head shape: every draft is
    accepted (WFD keeps its speculative rows and commits them), draft-then-
    verify commits every draft plus the bonus tokens; both equal sequential."""
    w = accepting(MINI_BF16, M.init_weights(MINI_BF16, 0), 0.0)
    blocks = LoopedBlocks(LoopedModel(MINI_BF16, w, gpu, max_seq_len=256, use_graphs=graphs))
    ids = _prompt(90, 3).to(gpu)
    ar, _ = blocks.ar_generate(ids, 40)
    for T_draft in (1, 2):
        toks, tr = generate_wavefront_dynamic(blocks, ids, 40, SsdPolicy(MINI_BF16.T_total, T_draft))
        assert toks == ar, T_draft
        assert tr.n_drafts_accepted == tr.n_drafts_proposed > 0 and tr.n_drafts_rejected == 0
    toks, tr = generate_draft_then_verify(blocks, ids, 40, SsdPolicy(MINI_BF16.T_total, 1), 3)
    assert toks == ar
    assert tr.n_drafts_accepted == tr.n_drafts_proposed > 0


class _HostCompare:
    """The same blocks without device-side comparison or token handles: the
    batch scheduler then reads every argmax back and compares on the host."""

    def __init__(self, inner):
        self._inner = inner

    def __getattr__(self, name):
        if name in ("resolve_tokens", "reset_token_ring", "device_accept"):
            raise AttributeError(name)
        return getattr(self._inner, name)


@pytest.mark.parametrize("graphs", [False, True])
def test_device_greedy_verify_matches_host_compare(gpu, tiny_w, graphs):
    """Greedy batch WFD with the accept decision made on the device (one flag
    per verify row, ids kept in the token ring) commits the tokens and counters
    of the host comparison and of the oracle, over accepts and rejects."""
    w = accepting(TINY, tiny_w, 1.0)
    P = [_prompt(32), _prompt(21, 5), _prompt(40, 6)]
    N = [30, 17, 25]
    res = []
    for host in (False, True):
        bb = LoopedBlocksBatch(LoopedModel(TINY, w, gpu, max_seq_len=128, max_batch=3, use_graphs=graphs))
        bt = generate_wavefront_batch(_HostCompare(bb) if host else bb, [p.to(gpu) for p in P], N,
                                      SsdPolicy(TINY.T_total, 2))
        res.append([(t.tokens, t.counters()) for t in bt.per_seq])
    assert res[0] == res[1]
    acc = sum(c["n_drafts_accepted"] for _, c in res[0])
    rej = sum(c["n_drafts_rejected"] for _, c in res[0])
    assert acc > 0 and rej > 0, (acc, rej)
    oc = osched.wfd_batch(_oracle(TINY, w, 128, B=3), [p.tolist() for p in P], N, TINY.T_total, 2)
    assert [t for t, _ in res[0]] == [t.tokens for t in oc.per_seq]


# ---------------------------------------------------------------------------
# C3: the 2048-d model, 512-token prompt, greedy WFD at W = 8
# ---------------------------------------------------------------------------
@pytest.fixture(scope="module")
def w2048():
    return M.init_weights(C3, 0)


@pytest.mark.parametrize("variant", ["random_init", "accepting"])
def test_c3_greedy_wfd_is_lossless(gpu, w2048, variant):
    """All 256 tokens of greedy WFD (T_total 16, T_draft 2) from the
    512-token prompt equal sequential looped decode, eager and captured."""
    w = w2048 if variant == "random_init" else accepting(C3, w2048, 0.0)
    ids = _prompt(512, 0, C3.vocab_size).to(gpu)
    N = 256
    ref = None
    for graphs in (False, True):
        print(f"[C3] {variant} graphs={graphs}", flush=True)
        blocks = LoopedBlocks(LoopedModel(C3, w, gpu, max_seq_len=512 + N + 16, use_graphs=graphs))
        ar, _ = blocks.ar_generate(ids, N)
        toks, tr = generate_wavefront_dynamic(blocks, ids, N, SsdPolicy(C3.T_total, 2))
        assert toks == ar and len(toks) == N
        if variant == "accepting":
            assert tr.n_drafts_accepted == tr.n_drafts_proposed > 0
        ref = ar if ref is None else ref
        assert ar == ref  # eager and captured decode agree
        # the batch scheduler at B = 1 with the verify on the device (the bench's path)
        bb = LoopedBlocksBatch(blocks.model, batch_size=1)
        bt = generate_wavefront_batch(bb, [ids], N, SsdPolicy(C3.T_total, 2))
        assert bt.per_seq[0].tokens == ar
        assert bt.per_seq[0].counters() == tr.counters()
        del blocks, bb
        torch.cuda.empty_cache()


# ---------------------------------------------------------------------------
# C4: the 2048-d model at B = 32, prompts U[128, 2048], generation U[64, 512]
# (seed 0): the workload the bs=32 benchmark decodes
# ---------------------------------------------------------------------------
B4 = 32


def c4_workload(seed: int = 0):
    """(prompt lengths, generation lengths, prompts) of the B = 32 workload."""
    g = torch.Generator().manual_seed(seed)
    plen = torch.randint(128, 2049, (B4,), generator=g).tolist()
    glen = torch.randint(64, 513, (B4,), generator=g).tolist()
    prompts = [torch.randint(0, C3.vocab_size, (p,), generator=g) for p in plen]
    return plen, glen, prompts


@pytest.fixture(scope="module")
def c4(gpu, w2048):
    plen, glen, prompts = c4_workload()
    prompts = [p.to(gpu) for p in prompts]
    model = LoopedModel(C3, w2048, gpu, max_seq_len=max(plen) + max(glen) + 16, max_batch=B4, use_graphs=True)
    bb = LoopedBlocksBatch(model, batch_size=B4)
    print(f"[C4] prefill of {sum(plen)} prompt tokens ({min(plen)}-{max(plen)} per sequence)", flush=True)
    pf = prefill_once(bb, prompts)
    yield model, bb, pf, prompts, glen
    del model, bb, pf
    torch.cuda.empty_cache()


@pytest.mark.parametrize("alpha", [0.9, 0.5])
def test_c4_batch_equals_solo_runs(gpu, c4, alpha):
    """Emulated acceptance (seeds 1000 + b): every sequence of the 32-wide
    batch commits its solo run's tokens with its solo run's counters, over
    the whole generation (64-512 tokens after a 128-2048-token prompt)."""
    model, bb, pf, prompts, glen = c4
    policy = SsdPolicy(C3.T_total, 2)
    print(f"[C4] batch of 32, alpha={alpha}", flush=True)
    bt = generate_wavefront_batch(bb, prompts, glen, policy, [EmulatedAcceptance(alpha, 1000 + b) for b in range(B4)],
                                  prefilled=pf)
    assert bt.r_union_max > 100  # the sequences' waves really shared unions
    assert [len(t.tokens) for t in bt.per_seq] == glen
    solo_blocks = LoopedBlocksBatch(model, batch_size=1)
    for b in range(B4):
        solo = generate_wavefront_batch(solo_blocks, [prompts[b]], [glen[b]], policy,
                                        [EmulatedAcceptance(alpha, 1000 + b)])
        assert bt.per_seq[b].tokens == solo.per_seq[0].tokens, b
        assert bt.per_seq[b].counters() == solo.per_seq[0].counters(), b
    print(f"[C4] alpha={alpha}: {bt.n_tokens} tokens, {bt.n_r_calls} R ticks, acceptance "
          f"{bt.acceptance_rate:.3f}", flush=True)


def test_c4_greedy_batch_equals_sequential(gpu, c4):
    """Real greedy acceptance (decided on the device) over the ragged 32-wide
    batch commits exactly the lockstep sequential decode's tokens for every
    sequence's whole generation; AR R calls = (N - 1) T_total."""
    model, bb, pf, prompts, glen = c4
    print("[C4] greedy batch WFD vs lockstep sequential decode", flush=True)
    wfd = generate_wavefront_batch(bb, prompts, glen, SsdPolicy(C3.T_total, 2), prefilled=pf)
    ar = ar_generate_batch(bb, prompts, glen, prefilled=pf)
    assert [t.tokens for t in wfd.per_seq] == [t.tokens for t in ar.per_seq]
    for t, n in zip(ar.per_seq, glen):
        assert t.n_r_calls == (n - 1) * C3.T_total and len(t.tokens) == n
    print(f"[C4] greedy: {wfd.n_tokens} tokens, {wfd.n_r_calls} R ticks, acceptance {wfd.acceptance_rate:.3f}",
          flush=True)


def test_c4_replicas_isolation_and_prefill(gpu, c4):
    """Replicas of one prompt commit identical tokens and counters; an
    alpha = 0 neighbour leaves an alpha = 1 sequence's run unchanged; batch
    prefill logits equal the single-sequence prefill's."""
    model, bb, pf, prompts, glen = c4
    policy = SsdPolicy(C3.T_total, 1)
    bb4 = LoopedBlocksBatch(model, batch_size=4)
    bt = generate_wavefront_batch(bb4, [prompts[0]] * 4, 40, policy, [EmulatedAcceptance(1.0, 11) for _ in range(4)])
    assert all(t.tokens == bt.per_seq[0].tokens and t.counters() == bt.per_seq[0].counters() for t in bt.per_seq)
    bb1 = LoopedBlocksBatch(model, batch_size=1)
    solo = generate_wavefront_batch(bb1, [prompts[1]], 40, policy, [EmulatedAcceptance(1.0, 31)])
    bb2 = LoopedBlocksBatch(model, batch_size=2)
    mix = generate_wavefront_batch(bb2, [prompts[1]] * 2, 40, policy,
                                   [EmulatedAcceptance(0.0, 99), EmulatedAcceptance(1.0, 31)])
    assert solo.per_seq[0].counters() == mix.per_seq[1].counters()
    assert solo.per_seq[0].tokens == mix.per_seq[1].tokens
    t0 = mix.per_seq[0]
    assert t0.n_drafts_proposed > 0 and t0.n_drafts_accepted == 0 and len(t0.tokens) == 40
    _, lb = bb2.prefill([prompts[2], prompts[2]])
    _, ls = LoopedBlocks(model).prefill(prompts[2], C3.T_total, 2)
    assert rel_err(lb[0].cpu().numpy(), ls.cpu().numpy()) <= 1e-6


def test_c4_ragged_r_tick_matches_oracle(gpu, w2048):
    """One union R tick of the B = 32 workload: 256 rows, each sequence at a
    position inside its own generation (key prefixes 178-2381, the shortest
    prompt's first wave to the longest sequence's last token; most rows span
    2-3 of the attention's 1024-key splits), over random K/V. 28 sequences carry a WFD wave (8 rows at depths 0, 2, .., 14); 4
    carry draft-then-verify-like rows (4 rows at one depth, adjacent, so the
    attention groups them, next to 4 rows at other depths). Rows of every
    kind are compared with the fp32 oracle's core fed the same bf16 values:
    <= 2e-2."""
    plen, glen, _ = c4_workload()
    S = max(plen) + max(glen) + 16
    model = LoopedModel(C3, w2048, gpu, max_seq_len=S, max_batch=B4, use_graphs=True)
    cache = model.create_cache(B4)
    g = torch.Generator(device=gpu).manual_seed(44)
    for t in (cache.flat_k, cache.flat_v):
        t.copy_(torch.randn(t.shape, generator=g, device=gpu).to(torch.bfloat16))
    # sequence b's newest row sits k_b / 11 of the way through its generation:
    # the shortest prompt at its start, the longest prompt + generation at its end
    k = [(b * 7) % 12 for b in range(B4)]
    k[int(np.argmin(plen))] = 0
    k[int(np.argmax(np.add(plen, glen)))] = 11
    seqs, pos, steps = [], [], []
    for b in range(B4):
        p = plen[b] + 7 + (glen[b] - 8) * k[b] // 11
        if b % 8 == 7:
            d = (b // 8) * 3
            rows = [(p + i, d) for i in range(4)] + [(p - 1 - i, d + 1 + i) for i in range(4)]
        else:
            rows = [(p - i, 2 * i) for i in range(8)]
        for q, d in rows:
            seqs.append(b)
            pos.append(q)
            steps.append(d)
    assert len(seqs) == 256 and max(steps) < C3.T_total and max(pos) < S - 1
    assert min(pos) + 1 == min(plen) + 1 and max(pos) + 1 == max(np.add(plen, glen))
    pool_rows = [model.pool_row(b, q) for b, q in zip(seqs, pos)]
    assert len(set(pool_rows)) == 256
    gh = torch.Generator().manual_seed(45)
    state = torch.randn(256, 2 * C3.d_model, generator=gh).to(torch.bfloat16)
    model.pool[pool_rows] = state.to(gpu)
    tick = model._tick
    prm = model._tick_params(cache)
    t32, t64 = model._table_scratch(1)
    grouped = tick.plan_pass(t32, 0, t64, 0, prm, "R", seqs, pos, steps, -1, -1, -1)[3]
    assert grouped  # the adjacent same-depth rows share their prefix reads
    print("[C4] ragged R tick, 256 rows", flush=True)
    model.core_union(cache, seqs, pos, steps)
    got = model.pool[pool_rows, : C3.d_model].float().cpu().numpy()
    lm = OracleLM(C3, M.weights_numpy(w2048), S, 1, None, None)
    st = state.float().numpy()
    # the longest and shortest prefixes, grouped rows, each depth of a wave
    check = sorted({int(np.argmax(pos)), int(np.argmin(pos)), 7 * 8, 7 * 8 + 1, 7 * 8 + 3, 7 * 8 + 6, 15 * 8 + 2,
                    3 * 8 + 0, 3 * 8 + 7, 12 * 8 + 4, 20 * 8 + 5, 31 * 8 + 3})
    for i in check:
        b, d = seqs[i], steps[i]
        # the oracle's one sequence gets sequence b's slots of this depth as the
        # tick left them (other rows' appends included, as the GPU read them)
        for l in range(C3.n_core):
            sl = model.slot_core(d, l)
            lm.Kc[sl, 0] = cache.K[sl, b].float().cpu().numpy()
            lm.Vc[sl, 0] = cache.V[sl, b].float().cpu().numpy()
        ref = lm.core(0, pos[i], d, st[i, : C3.d_model], st[i, C3.d_model:])
        err = rel_err(got[i], ref)
        assert err <= 2e-2, (i, b, pos[i], steps[i], err)
    del model, cache
    torch.cuda.empty_cache()


# ---------------------------------------------------------------------------
# C5: GQA 16 q / 4 kv heads, 32k context
# ---------------------------------------------------------------------------
def test_c5_attention_32k_matches_oracle(gpu):
    """8 decode rows over two 32k-key slots in the engine's head-major block
    layout: 33 splits per row plus the split combine, against the oracle."""
    S = 32800
    lens = [32768, 32769, 32770, 32775, 32700, 30000, 32799, 31744]
    g = torch.Generator().manual_seed(32)
    K = torch.randn(2 * S, 4, 128, generator=g).to(torch.bfloat16)
    V = torch.randn(2 * S, 4, 128, generator=g).to(torch.bfloat16)
    q = torch.randn(8, 16, 128, generator=g).to(torch.bfloat16)
    rb = torch.tensor([(i % 2) * S for i in range(8)], dtype=torch.int64)
    kl = torch.tensor(lens, dtype=torch.int32)
    blocks = lambda t: t.view(2, S, 4, 128).permute(0, 2, 1, 3).contiguous()  # noqa: E731
    print("[C5] attention 32k", flush=True)
    out = ops.attn_decode(q.to(gpu), blocks(K).to(gpu), blocks(V).to(gpu), rb.to(gpu), kl.to(gpu), kv_len_max=S)
    assert ops.attn_workspace_bytes(8, 16, 128, S) > 0
    ref = ok.attention_rows(q.float().numpy(), K.float().numpy(), V.float().numpy(), rb.numpy(), kl.numpy())
    assert rel_err(out.float().cpu().numpy(), ref) <= 2e-2


def test_c5_gqa_core_tick_matches_oracle(gpu):
    """One R tick of the GQA looped model (16 rows = W at depths 0, 2, ..., 30
    of one sequence, random K/V prefixes at a reduced 2k context) against the
    fp32 oracle fed the same bf16 values: <= 2e-2."""
    cfg = GQA
    w = M.init_weights(cfg, 0)
    S = 2048
    model = LoopedModel(cfg, w, gpu, max_seq_len=S, max_batch=1)
    cache = model.create_cache(1)
    g = torch.Generator().manual_seed(5)
    for t in (cache.flat_k, cache.flat_v):
        t.copy_(torch.randn(t.shape, generator=g).to(torch.bfloat16))
    pos = [2000 - i for i in range(16)]
    steps = [2 * i for i in range(16)]
    rows = [model.pool_row(0, p) for p in pos]
    state = torch.randn(16, 2 * cfg.d_model, generator=g).to(torch.bfloat16)
    model.pool[rows] = state.to(gpu)
    print("[C5] GQA core tick", flush=True)
    model.core_union(cache, [0] * 16, pos, steps)
    got = model.pool[rows, : cfg.d_model].float().cpu().numpy()
    lm = OracleLM(cfg, M.weights_numpy(w), S, 1, None, None)
    lm.Kc[:] = cache.K.float().cpu().numpy()
    lm.Vc[:] = cache.V.float().cpu().numpy()
    st = state.float().numpy()
    ref = np.stack([lm.core(0, pos[i], steps[i], st[i, : cfg.d_model], st[i, cfg.d_model:]) for i in range(16)])
    assert rel_err(got, ref) <= 2e-2
    del model, cache
    torch.cuda.empty_cache()
