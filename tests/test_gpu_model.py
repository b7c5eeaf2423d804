"""End-to-end parity of the HIP decode path against the oracle (GPU).

* tiny fp32 looped LM (d=256, 4x64 heads, SwiGLU 1024, 1 + 2x4 + 1 layers,
  V=4096, N(0,0.02) seed 0, 128-token prompt): prefill logits within 1e-4 of
  the oracle; WFD (T_draft 1 and 2) and sequential decode commit the oracle's
  tokens; batch WFD over ragged prompts matches per-sequence decode; the
  emulated-acceptance batch trace equals the oracle's.
* bf16: WFD tokens are bit-identical to sequential decode on the GPU
  (lossless), and one R tick over a mixed-depth union equals each row run
  alone, bit for bit; one R tick of the 2048-d model matches the oracle
  within 2e-2.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import scheduler as osched
from oracle import state_init
from oracle.looped_lm import OracleBatchBlocks, OracleLM
from tests.conftest import rel_err
from wavefront_decoding_amd import model as M
from wavefront_decoding_amd.blocks import LoopedBlocks, LoopedBlocksBatch
from wavefront_decoding_amd.emu import EmulatedAcceptance
from wavefront_decoding_amd.engine import LoopedModel
from wavefront_decoding_amd.policy import SsdPolicy
from wavefront_decoding_amd.scheduler import generate_wavefront_dynamic
from wavefront_decoding_amd.scheduler_batch import ar_generate_batch, generate_dtv_batch, generate_wavefront_batch

pytestmark = pytest.mark.gpu

TINY = M.CONFIGS["tiny"]
# a small bf16 looped LM with the 2048-d model's head shape (Dh = 128) for fast lossless checks
MINI_BF16 = M.LoopedLMConfig("mini-bf16", 4096, 512, 4, 4, 128, 1536, 1, 2, 1, 8)
MINI_GQA = M.LoopedLMConfig("mini-gqa", 4096, 512, 4, 1, 128, 1536, 1, 2, 1, 8)


def _prompt(L, seed=0, V=4096, B=None):
    g = torch.Generator().manual_seed(seed)
    return torch.randint(0, V, (L,) if B is None else (B, L), generator=g)


def _round(a: np.ndarray, cfg) -> np.ndarray:
    return torch.from_numpy(a).to(cfg.torch_dtype).float().numpy()


def _oracle(cfg, w, S, B=1):
    """Oracle blocks with the oracle's own s0 recipe, rounded through the run
    dtype exactly as the GPU table is."""
    wn = M.weights_numpy(w)
    s0t = lambda p: _round(state_init.s0_token(cfg.d_model, cfg.state_std, cfg.emb_scale, 0, p), cfg)  # noqa: E731
    s0p = lambda L: _round(state_init.s0_prefill(cfg.d_model, cfg.state_std, cfg.emb_scale, 0, L), cfg)  # noqa: E731
    return OracleBatchBlocks(OracleLM(cfg, wn, S, B, s0t, s0p))


@pytest.fixture(scope="module")
def tiny(gpu):
    w = M.init_weights(TINY, 0)
    return w, LoopedModel(TINY, w, gpu, max_seq_len=256, max_batch=3)


def test_state_tables_match_oracle_recipe():
    for p in (0, 7, 300):
        np.testing.assert_array_equal(M.initial_state_tokens(TINY, [p])[0].numpy(),
                                      state_init.s0_token(256, 0.02, 1.0, 0, p))


def test_tiny_prefill_logits_match_oracle(tiny):
    w, model = tiny
    ids = _prompt(128)
    print("[tiny] prefill 128", flush=True)
    blocks = LoopedBlocks(model)
    state, logits = blocks.prefill(ids.to(model.device), TINY.T_total, 2)
    ob = _oracle(TINY, w, 256)
    _, ref = ob.prefill([ids.tolist()])
    assert rel_err(logits.cpu().numpy(), ref[0]) <= 1e-4


@pytest.mark.parametrize("dtype", ["float32", "bfloat16"])
def test_prompt_pass_library_gemm_matches_kernels(gpu, dtype):
    """The prompt pass with library GEMMs (the default) against the same pass
    on the packed linear kernels: the same slot caches and last-position logits
    up to the GEMMs' summation order (rows that are computed once and never
    compared bit for bit with decode rows), and the oracle agrees."""
    import dataclasses
    cfg = dataclasses.replace(TINY, dtype=dtype)
    w = M.init_weights(cfg, 0)
    ids = _prompt(100).tolist()
    outs = []
    for dense in (True, False):
        m = LoopedModel(cfg, w, gpu, max_seq_len=128, max_batch=1, dense_prompt=dense)
        cache = m.create_cache(1)
        logits = m.prefill_seq(cache, 0, ids)
        torch.cuda.synchronize()
        outs.append((logits.float().cpu().numpy(), cache.flat_k.float().cpu().numpy(),
                     cache.flat_v.float().cpu().numpy()))
    tol = 1e-4 if dtype == "float32" else 5e-2  # bf16: roundings of the two GEMM orders compound over the loop
    for a, b in zip(outs[0], outs[1]):
        assert rel_err(a, b) <= tol
    if dtype == "float32":
        ref = _oracle(cfg, w, 128).prefill([ids])[1][0]
        assert rel_err(outs[0][0], ref) <= tol


@pytest.mark.parametrize("T_draft", [1, 2])
def test_tiny_wfd_matches_oracle_and_sequential(tiny, T_draft):
    w, model = tiny
    ids = _prompt(128)
    N = 40
    blocks = LoopedBlocks(model)
    print(f"[tiny] wfd T_draft={T_draft} N={N}", flush=True)
    toks, trace = generate_wavefront_dynamic(blocks, ids.to(model.device), N, SsdPolicy(TINY.T_total, T_draft))
    ar, _ = blocks.ar_generate(ids.to(model.device), N)
    assert toks == ar
    oc = osched.wfd_single(_oracle(TINY, w, 256), ids.tolist(), N, TINY.T_total, T_draft)
    assert toks == oc.tokens
    assert trace.counters() == {k: getattr(oc, k) for k in trace.counters()}


def test_tiny_batch_ragged_matches_single(tiny):
    w, model = tiny
    P = [_prompt(60, 1), _prompt(23, 2), _prompt(100, 3)]
    N = [14, 9, 11]
    bb = LoopedBlocksBatch(model, batch_size=3)
    print("[tiny] batch ragged", flush=True)
    bt = generate_wavefront_batch(bb, [p.to(model.device) for p in P], N, SsdPolicy(TINY.T_total, 2))
    ar = ar_generate_batch(bb, [p.to(model.device) for p in P], N)
    single = LoopedBlocks(model)
    for b in range(3):
        solo, _ = single.ar_generate(P[b].to(model.device), N[b])
        assert bt.per_seq[b].tokens == solo == ar.per_seq[b].tokens
    assert bt.r_union_max > 3  # several sequences and depths shared unions


def test_tiny_emulated_batch_trace_matches_oracle(tiny):
    w, model = tiny
    P = [_prompt(30, 4), _prompt(30, 5)]
    bb = LoopedBlocksBatch(model, batch_size=2)
    emus = [EmulatedAcceptance(0.5, 1000 + b) for b in range(2)]
    bt = generate_wavefront_batch(bb, [p.to(model.device) for p in P], 12, SsdPolicy(TINY.T_total, 2), emus)
    oe = [osched.Emu(0.5, 1000 + b) for b in range(2)]
    res = osched.wfd_batch(_oracle(TINY, w, 256, B=2), [p.tolist() for p in P], 12, TINY.T_total, 2, oe)
    for b in range(2):
        assert bt.per_seq[b].tokens == res.per_seq[b].tokens
        assert bt.per_seq[b].counters() == {k: getattr(res.per_seq[b], k) for k in bt.per_seq[b].counters()}
    assert (bt.n_r_calls, bt.r_union_total) == (res.n_r_calls, res.r_union_total)


@pytest.mark.parametrize("cfg", [MINI_BF16, MINI_GQA], ids=lambda c: c.name)
def test_bf16_wfd_is_lossless(gpu, cfg):
    w = M.init_weights(cfg, 0)
    model = LoopedModel(cfg, w, gpu, max_seq_len=512, max_batch=1)
    blocks = LoopedBlocks(model)
    ids = _prompt(200, 7).to(gpu)
    print(f"[{cfg.name}] lossless", flush=True)
    ar, _ = blocks.ar_generate(ids, 48)
    for T_draft in (1, 2, 4):
        toks, tr = generate_wavefront_dynamic(blocks, ids, 48, SsdPolicy(cfg.T_total, T_draft))
        assert toks == ar, T_draft


@pytest.mark.parametrize("graphs", [True, False])
def test_greedy_flags_after_runs_that_never_read_them(gpu, graphs):
    """The C passes' accept flags land in mapped host memory that every C
    launch rewrites. Runs that never read them (emulated acceptance,
    sequential decode) leave launches in flight; a greedy run on the same
    engine right after must still see its own flags: its tokens equal
    sequential decode's, and equal a greedy run on a fresh engine, with the
    same counters."""
    cfg = MINI_BF16
    w = M.init_weights(cfg, 0)
    P = [_prompt(60, 11, V=cfg.vocab_size), _prompt(45, 12, V=cfg.vocab_size)]
    pol = SsdPolicy(cfg.T_total, 2)

    def greedy(bb):
        bt = generate_wavefront_batch(bb, [p.to(gpu) for p in P], [20, 16], pol)
        return [t.tokens for t in bt.per_seq], [t.counters() for t in bt.per_seq]

    print(f"[flags after unread runs] graphs={graphs}", flush=True)
    fresh = greedy(LoopedBlocksBatch(LoopedModel(cfg, w, gpu, max_seq_len=128, max_batch=2, use_graphs=graphs), 2))
    bb = LoopedBlocksBatch(LoopedModel(cfg, w, gpu, max_seq_len=128, max_batch=2, use_graphs=graphs), 2)
    emus = [EmulatedAcceptance(0.8, 7000 + b) for b in range(2)]
    generate_wavefront_batch(bb, [p.to(gpu) for p in P], [20, 16], pol, emus)  # flags written, never read
    seq = ar_generate_batch(bb, [p.to(gpu) for p in P], [20, 16])           # and again
    after = greedy(bb)
    assert after == fresh
    assert after[0] == [t.tokens for t in seq.per_seq]


@pytest.mark.parametrize("graphs", [True, False])
def test_token_ring_exhaustion_falls_back_to_ids(gpu, graphs):
    """A token ring too small for a generation: once it is full, C passes
    return plain ids (their argmax lands in the trash slot) and the greedy
    verify compares against a mix of handles and ids; tokens and counters
    equal those of a run whose ring never fills."""
    cfg = MINI_BF16
    w = M.init_weights(cfg, 0)
    P = [_prompt(50, 21, V=cfg.vocab_size), _prompt(37, 22, V=cfg.vocab_size)]
    pol = SsdPolicy(cfg.T_total, 2)
    out = []
    for ring_len in (1 << 20, 9):
        print(f"[token ring] graphs={graphs} ring_len={ring_len}", flush=True)
        m = LoopedModel(cfg, w, gpu, max_seq_len=128, max_batch=2, use_graphs=graphs, ring_len=ring_len)
        full = []
        run = m.run_passes

        def counted(cache, passes):
            res = run(cache, passes)
            if any(k == "C" and len(pos) for k, _, pos, _ in passes):
                full.append(m.last_c_handles is None)
            return res

        m.run_passes = counted
        bt = generate_wavefront_batch(LoopedBlocksBatch(m, 2), [p.to(gpu) for p in P], [18, 14], pol)
        out.append(([t.tokens for t in bt.per_seq], [t.counters() for t in bt.per_seq], bt.n_r_calls))
        # the large ring never fills; the small one fills and C passes fall back to ids
        assert any(full) == (ring_len == 9) and not all(full)
    assert out[0] == out[1]


def test_rollback_reappend_reproduces_committed_cache_rows(gpu):
    """Slot-cache append and rollback: greedy WFD on random-init weights
    rejects almost every draft, so rows of rejected tokens are dropped and
    rewritten by the gold token at the same positions. Over every committed
    position that has been through the whole model, every slot's K and V
    rows then equal those of sequential decode bit for bit (the invariant of
    reference kv_cache.py:158-165 with reads bounded by the query's position)."""
    cfg = MINI_BF16
    model = LoopedModel(cfg, M.init_weights(cfg, 0), gpu, max_seq_len=512, max_batch=1)
    blocks = LoopedBlocks(model)
    ids = _prompt(200, 11).to(gpu)
    N = 40
    print("[rollback] sequential", flush=True)
    ar, _ = blocks.ar_generate(ids, N)
    cache = blocks._cache
    end = 200 + N - 1  # the last token is committed but not yet run through the model
    K0, V0 = cache.K[:, 0, :end].clone(), cache.V[:, 0, :end].clone()
    print("[rollback] WFD", flush=True)
    toks, tr = generate_wavefront_dynamic(blocks, ids, N, SsdPolicy(cfg.T_total, 2))
    assert toks == ar and tr.n_rollback_events > 0
    assert torch.equal(cache.K[:, 0, :end], K0) and torch.equal(cache.V[:, 0, :end], V0)


def test_core_tick_row_invariant(gpu):
    """One R tick over a mixed-depth union equals each row ticked alone, bit for bit."""
    cfg = MINI_BF16
    model = LoopedModel(cfg, M.init_weights(cfg, 1), gpu, max_seq_len=256, max_batch=1)
    cache = model.create_cache(1)
    g = torch.Generator().manual_seed(3)
    cache.flat_k.copy_(torch.randn(cache.flat_k.shape, generator=g).to(cache.flat_k.dtype))
    cache.flat_v.copy_(torch.randn(cache.flat_v.shape, generator=g).to(cache.flat_v.dtype))
    pos = [100, 99, 98, 97, 96, 95]
    steps = [5, 4, 3, 2, 1, 0]
    rows = [model.pool_row(0, p) for p in pos]
    model.pool.copy_(torch.randn(model.pool.shape, generator=g).to(model.pool.dtype))
    init = model.pool.clone()
    model.core_union(cache, [0] * 6, pos, steps)
    union = model.pool[rows].clone()
    for i in range(6):
        model.pool.copy_(init)
        model.core_union(cache, [0], [pos[i]], [steps[i]])
        assert torch.equal(model.pool[rows[i]], union[i]), i


@pytest.mark.parametrize("cfg", [MINI_BF16, M.CONFIGS["looped-2048"]], ids=lambda c: c.name)
def test_split_k_projections_same_bits(gpu, cfg):
    """proj, the MLP down projection and the adapter split over K (slice sums
    reduced in the next norm) give the bits of the one-launch linears: an R
    tick over 40 mixed-depth rows of 4 sequences (distinct pool rows) and a C
    pass over the same rows, with the split path on (its default row range)
    and off."""
    w = M.init_weights(cfg, 2)
    B, n = 4, 40
    model = LoopedModel(cfg, w, gpu, max_seq_len=64, max_batch=B, max_rows=64)
    assert model.split_rows[0] <= n <= model.split_rows[1]
    cache = model.create_cache(B)
    g = torch.Generator().manual_seed(6)
    kv = torch.randn(2, *cache.flat_k.shape, generator=g).to(cache.flat_k.dtype).to(gpu)
    seqs = [i // 10 for i in range(n)]
    pos = [60 - i % 10 for i in range(n)]
    steps = [i % cfg.T_total for i in range(n)]
    rows = [model.pool_row(b, p) for b, p in zip(seqs, pos)]
    assert len(set(rows)) == n
    model.pool.copy_(torch.randn(model.pool.shape, generator=g).to(model.pool.dtype))
    init = model.pool.clone()
    out = {}
    for split in (True, False):
        print(f"[split-K model] {cfg.name} split={split}", flush=True)
        model.split_rows = (17, 512) if split else (1 << 30, 1 << 30)
        model.pool.copy_(init)
        cache.flat_k.copy_(kv[0])
        cache.flat_v.copy_(kv[1])
        model.core_union(cache, seqs, pos, steps)
        logits, _ = model.coda_union(cache, seqs, pos)
        out[split] = (model.pool[rows].clone(), logits.clone())
    assert torch.equal(out[True][0], out[False][0])
    assert torch.equal(out[True][1], out[False][1])


def test_2048_core_tick_matches_oracle(gpu):
    """One R tick of the 2048-d bf16 model (8 rows, depths 0..14, slot prefixes
    of random K/V) against the fp32 oracle fed the same bf16 values: <= 2e-2."""
    cfg = M.CONFIGS["looped-2048"]
    w = M.init_weights(cfg, 0)
    S = 640
    model = LoopedModel(cfg, w, gpu, max_seq_len=S, max_batch=1)
    cache = model.create_cache(1)
    g = torch.Generator().manual_seed(4)
    kv = torch.randn(2, *cache.flat_k.shape, generator=g).to(torch.bfloat16)
    cache.flat_k.copy_(kv[0])
    cache.flat_v.copy_(kv[1])
    pos = [600 - i for i in range(8)]
    steps = [2 * i for i in range(8)]
    rows = [model.pool_row(0, p) for p in pos]
    state = torch.randn(8, 2 * cfg.d_model, generator=g).to(torch.bfloat16)
    model.pool[rows] = state.to(gpu)
    print("[2048] core tick", flush=True)
    model.core_union(cache, [0] * 8, pos, steps)
    got = model.pool[rows, : cfg.d_model].float().cpu().numpy()
    lm = OracleLM(cfg, M.weights_numpy(w), S, 1, None, None)
    K = cache.K.float().cpu().numpy()
    V = cache.V.float().cpu().numpy()
    lm.Kc[:] = K
    lm.Vc[:] = V
    st = state.float().numpy()
    ref = np.stack([lm.core(0, pos[i], steps[i], st[i, : cfg.d_model], st[i, cfg.d_model:]) for i in range(8)])
    assert rel_err(got, ref) <= 2e-2


@pytest.mark.parametrize("cfg", [TINY, MINI_BF16], ids=lambda c: c.name)
def test_graph_mode_matches_eager(gpu, cfg):
    """Captured decode passes (fixed tables refreshed per replay, padded rows
    aimed at trash rows) commit exactly the eager tokens and counters; the
    graphs replay many times with eager work and host syncs in between."""
    w = M.init_weights(cfg, 2)
    ids = _prompt(90, 11, V=cfg.vocab_size).to(gpu)
    eager = LoopedBlocks(LoopedModel(cfg, w, gpu, max_seq_len=200, max_batch=1))
    graph = LoopedBlocks(LoopedModel(cfg, w, gpu, max_seq_len=200, max_batch=1, use_graphs=True))
    for T_draft in (1, 2):
        a, ta = generate_wavefront_dynamic(eager, ids, 30, SsdPolicy(cfg.T_total, T_draft))
        b, tb = generate_wavefront_dynamic(graph, ids, 30, SsdPolicy(cfg.T_total, T_draft))
        assert a == b and ta.counters() == tb.counters(), T_draft
    assert len(graph.model._graphs) >= 3
    ar_e, _ = eager.ar_generate(ids, 12)
    ar_g, _ = graph.ar_generate(ids, 12)
    assert ar_e == ar_g


def test_graph_mode_batch_emulated(gpu):
    cfg = TINY
    w = M.init_weights(cfg, 0)
    P = [_prompt(40, 4), _prompt(25, 5), _prompt(33, 6)]
    res = []
    for graphs in (False, True):
        bb = LoopedBlocksBatch(LoopedModel(cfg, w, gpu, max_seq_len=128, max_batch=3, use_graphs=graphs))
        emus = [EmulatedAcceptance(0.7, 1000 + b) for b in range(3)]
        bt = generate_wavefront_batch(bb, [p.to(gpu) for p in P], [10, 14, 7], SsdPolicy(cfg.T_total, 2), emus)
        res.append([(s.tokens, s.counters()) for s in bt.per_seq])
    assert res[0] == res[1]


class _NoHandles:
    """The same blocks without token handles: the schedulers then read every
    argmax back as it is produced (the reference's behaviour)."""

    def __init__(self, inner):
        self._inner = inner

    def __getattr__(self, name):
        if name in ("resolve_tokens", "reset_token_ring"):
            raise AttributeError(name)
        return getattr(self._inner, name)


@pytest.mark.parametrize("graphs", [False, True])
def test_token_handles_match_eager_ids(gpu, graphs):
    """Keeping sampled ids on the device (token ring + handles, no host read
    per commit) gives the same tokens and counters as reading every id back,
    for emulated WFD and for sequential batch decode."""
    cfg = TINY
    w = M.init_weights(cfg, 0)
    P = [_prompt(40, 4), _prompt(25, 5), _prompt(33, 6)]
    res = []
    for handles in (True, False):
        bb = LoopedBlocksBatch(LoopedModel(cfg, w, gpu, max_seq_len=128, max_batch=3, use_graphs=graphs))
        blk = bb if handles else _NoHandles(bb)
        emus = [EmulatedAcceptance(0.6, 2000 + b) for b in range(3)]
        bt = generate_wavefront_batch(blk, [p.to(gpu) for p in P], [12, 9, 15], SsdPolicy(cfg.T_total, 2), emus)
        ar = ar_generate_batch(blk, [p.to(gpu) for p in P], [6, 8, 5])
        res.append(([(t.tokens, t.counters()) for t in bt.per_seq], [t.tokens for t in ar.per_seq]))
        assert all(v >= 0 for t in bt.per_seq for v in t.tokens)
    assert res[0] == res[1]


@pytest.mark.parametrize("cfg", [TINY, MINI_BF16, MINI_GQA], ids=lambda c: c.name)
def test_dtv_is_lossless(gpu, cfg):
    """Draft-then-verify (single sequence and batch, ragged) commits exactly
    the sequential tokens: every committed token is a full-depth argmax and
    every kernel is row-invariant, so verify rows equal sequential rows bit
    for bit."""
    from wavefront_decoding_amd.scheduler import generate_draft_then_verify

    w = M.init_weights(cfg, 0)
    model = LoopedModel(cfg, w, gpu, max_seq_len=256, max_batch=3)
    blocks = LoopedBlocks(model)
    ids = _prompt(70, 8, V=cfg.vocab_size).to(gpu)
    print(f"[{cfg.name}] dtv lossless", flush=True)
    ar, _ = blocks.ar_generate(ids, 24)
    for T_draft, K in ((1, 3), (2, 2), (4, 1)):
        toks, tr = generate_draft_then_verify(blocks, ids, 24, SsdPolicy(cfg.T_total, T_draft), K)
        assert toks == ar, (T_draft, K)
        assert tr.n_drafts_proposed > 0
    P = [_prompt(40, 4, V=cfg.vocab_size), _prompt(25, 5, V=cfg.vocab_size), _prompt(33, 6, V=cfg.vocab_size)]
    N = [11, 7, 13]
    bb = LoopedBlocksBatch(model, batch_size=3)
    bt = generate_dtv_batch(bb, [p.to(gpu) for p in P], N, SsdPolicy(cfg.T_total, 2), 3)
    ab = ar_generate_batch(bb, [p.to(gpu) for p in P], N)
    assert [t.tokens for t in bt.per_seq] == [t.tokens for t in ab.per_seq]


def test_dtv_token_handles_match_eager_ids(gpu):
    """Emulated-acceptance DtV keeps every id on the device (drafts feed the
    next source's prelude as ring handles) and still commits the ids an
    eager read-back run commits."""
    cfg = TINY
    w = M.init_weights(cfg, 0)
    P = [_prompt(40, 4), _prompt(25, 5), _prompt(33, 6)]
    res = []
    for handles in (True, False):
        bb = LoopedBlocksBatch(LoopedModel(cfg, w, gpu, max_seq_len=128, max_batch=3))
        blk = bb if handles else _NoHandles(bb)
        emus = [EmulatedAcceptance(0.6, 3000 + b) for b in range(3)]
        bt = generate_dtv_batch(blk, [p.to(gpu) for p in P], [12, 9, 15], SsdPolicy(cfg.T_total, 2), 3, emus)
        res.append([(t.tokens, t.counters()) for t in bt.per_seq])
        assert all(v >= 0 for t in bt.per_seq for v in t.tokens)
    assert res[0] == res[1]


def test_grouped_attention_keeps_tokens(gpu):
    """Engines with and without same-slot attention groups (draft-then-verify
    sources, a coda's verifies + draft) commit the same tokens and counters,
    eager and captured."""
    cfg = MINI_BF16
    w = M.init_weights(cfg, 0)
    P = [_prompt(40, 4, V=cfg.vocab_size), _prompt(25, 5, V=cfg.vocab_size)]
    res = []
    for grouped, graphs in ((False, False), (True, False), (True, True)):
        m = LoopedModel(cfg, w, gpu, max_seq_len=128, max_batch=2, use_graphs=graphs, group_attention=grouped)
        m.group_min_workgroups = 0  # group even these small unions
        bb = LoopedBlocksBatch(m, batch_size=2)
        emus = [EmulatedAcceptance(0.7, 4000 + b) for b in range(2)]
        dt = generate_dtv_batch(bb, [p.to(gpu) for p in P], [14, 10], SsdPolicy(cfg.T_total, 1), 4, emus)
        emus = [EmulatedAcceptance(0.7, 5000 + b) for b in range(2)]
        wf = generate_wavefront_batch(bb, [p.to(gpu) for p in P], [14, 10], SsdPolicy(cfg.T_total, 2), emus)
        res.append(([(t.tokens, t.counters()) for t in dt.per_seq], [(t.tokens, t.counters()) for t in wf.per_seq]))
    assert res[0] == res[1] == res[2]
