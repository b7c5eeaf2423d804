"""The numpy looped LM under the oracle schedulers (CPU): losslessness and
batch behaviour on the tiny fp32 config (d=256, 4x64 heads, 1 + 2x4 + 1
layers, V=4096, random init N(0, 0.02) seed 0, 128-token prompt)."""
from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import scheduler as osched
from oracle import state_init
from oracle.looped_lm import OracleBatchBlocks, OracleLM
from wavefront_decoding_amd import model as M

CFG = M.CONFIGS["tiny"]


def make_oracle(cfg=CFG, S=256, B=1, seed=0):
    w = M.weights_numpy(M.init_weights(cfg, seed))
    s0t = lambda p: state_init.s0_token(cfg.d_model, cfg.state_std, cfg.emb_scale, 0, p)  # noqa: E731
    s0p = lambda L: state_init.s0_prefill(cfg.d_model, cfg.state_std, cfg.emb_scale, 0, L)  # noqa: E731
    return OracleBatchBlocks(OracleLM(cfg, w, S, B, s0t, s0p))


def prompt(B=1, L=128, seed=0):
    g = torch.Generator().manual_seed(seed)
    return torch.randint(0, CFG.vocab_size, (B, L), generator=g)


def test_state_init_matches_product_recipe():
    for p in (0, 5, 1000):
        np.testing.assert_array_equal(state_init.s0_token(256, 0.02, 1.0, 3, p),
                                      M.initial_state_tokens(CFG, [p], state_seed=3)[0].numpy())
    np.testing.assert_array_equal(state_init.s0_prefill(256, 0.02, 1.0, 0, 7), M.initial_state_prefill(CFG, 7).numpy())
    a = state_init.s0_token(256, 0.02, 1.0, 0, 11)
    assert np.abs(a).max() <= 3 * 0.02 + 1e-7 and 0.01 < a.std() < 0.03


def test_prompt_state_stream_is_prefix_consistent():
    """The engine draws the prompt's initial loop state once for the longest
    prompt and slices it: rows [0, L) of any longer draw must be the draw of
    length L, at the 2048-d model's width too."""
    for cfg in (CFG, M.CONFIGS["looped-2048"]):
        long = M.initial_state_prefill(cfg, 3000, state_seed=2)
        for L in (1, 2, 7, 512, 1999, 3000):
            assert torch.equal(M.initial_state_prefill(cfg, L, state_seed=2), long[:L]), (cfg.name, L)


@pytest.mark.parametrize("T_draft", [1, 2])
def test_oracle_wfd_equals_sequential(T_draft):
    ids = prompt()[0].tolist()
    ar = osched.ar_single(make_oracle(), ids, 24, CFG.T_total)
    c = osched.wfd_single(make_oracle(), ids, 24, CFG.T_total, T_draft)
    assert c.tokens == ar
    assert c.n_drafts_proposed > 0
    assert c.n_r_calls < (24 - 1) * CFG.T_total or T_draft == CFG.T_total


def test_oracle_batch_wfd_equals_sequential_and_isolated():
    P = prompt(B=2, L=40, seed=1)
    rows = [P[0].tolist(), P[1].tolist()[:25]]                  # ragged prompts
    res = osched.wfd_batch(make_oracle(B=2), rows, [12, 7], CFG.T_total, 2)
    for b in range(2):
        solo = osched.ar_single(make_oracle(), rows[b], [12, 7][b], CFG.T_total)
        assert res.per_seq[b].tokens == solo


def test_oracle_replica_symmetry():
    P = prompt(B=1, L=30, seed=2)[0].tolist()
    res = osched.wfd_batch(make_oracle(B=3), [P, P, P], 10, CFG.T_total, 2)
    t0 = res.per_seq[0]
    for s in res.per_seq[1:]:
        assert s.tokens == t0.tokens and s.n_r_calls == t0.n_r_calls and s.n_drafts_accepted == t0.n_drafts_accepted
