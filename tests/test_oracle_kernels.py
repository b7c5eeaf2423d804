"""Pin the oracle's per-op math against library routines and closed forms (CPU).

Each check is chosen so that a plausible slip in the oracle (a dropped scale,
a wrong sign, a transposed operand, an off-by-one cutoff, a wrong GQA map)
fails it; test_oracle_mutations.py plants such slips to prove it.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import kernels as ok


def _sdpa_ref(q, K, V, kv_len):
    """torch SDPA over the first kv_len keys with an explicit boolean mask that
    also hides the keys past kv_len (library routine, float64)."""
    H, Dh = q.shape
    S, Hkv, _ = K.shape
    qt = torch.from_numpy(q).double().view(1, H, 1, Dh)
    kt = torch.from_numpy(K).double().permute(1, 0, 2).unsqueeze(0)
    vt = torch.from_numpy(V).double().permute(1, 0, 2).unsqueeze(0)
    if Hkv != H:
        kt = kt.repeat_interleave(H // Hkv, dim=1)
        vt = vt.repeat_interleave(H // Hkv, dim=1)
    mask = (torch.arange(S) < kv_len).view(1, 1, 1, S)
    return F.scaled_dot_product_attention(qt, kt, vt, attn_mask=mask)[0, :, 0, :].numpy()


@pytest.mark.parametrize("H,Hkv,Dh,S,kv_len", [(4, 4, 64, 50, 37), (16, 4, 128, 300, 300), (8, 2, 64, 20, 1),
                                                (2, 1, 64, 700, 513)])
def test_attention_matches_sdpa(H, Hkv, Dh, S, kv_len):
    rng = np.random.default_rng(0)
    q = rng.standard_normal((H, Dh))
    K = rng.standard_normal((S, Hkv, Dh))
    V = rng.standard_normal((S, Hkv, Dh))
    got = ok.attention(q, K, V, kv_len)
    ref = _sdpa_ref(q, K, V, kv_len)
    np.testing.assert_allclose(got, ref, rtol=1e-10, atol=1e-12)


def test_attention_special_cases():
    rng = np.random.default_rng(1)
    q = rng.standard_normal((4, 64))
    K = rng.standard_normal((10, 4, 64))
    V = rng.standard_normal((10, 4, 64))
    # kv_len = 1: the single value row comes back unchanged.
    np.testing.assert_allclose(ok.attention(q, K, V, 1), V[0], rtol=1e-12)
    # identical keys: uniform weights -> mean of the visible values.
    Ke = np.repeat(K[:1], 10, axis=0)
    np.testing.assert_allclose(ok.attention(q, Ke, V, 7), V[:7].mean(axis=0), rtol=1e-10)
    # GQA == MHA with repeated K/V.
    q8 = rng.standard_normal((8, 64))
    K2 = rng.standard_normal((10, 2, 64))
    V2 = rng.standard_normal((10, 2, 64))
    gqa = ok.attention(q8, K2, V2, 9)
    mha = ok.attention(q8, np.repeat(K2, 4, axis=1), np.repeat(V2, 4, axis=1), 9)
    np.testing.assert_allclose(gqa, mha, rtol=1e-12)
    # keys past kv_len are never read.
    K3, V3 = K.copy(), V.copy()
    K3[5:] = 1e6
    V3[5:] = np.nan
    np.testing.assert_allclose(ok.attention(q, K3, V3, 5), ok.attention(q, K, V, 5), rtol=1e-12)


def test_attention_rows_flat_layout():
    rng = np.random.default_rng(2)
    B, S, n_slots, Hkv, Dh = 3, 16, 4, 2, 64
    K = rng.standard_normal((n_slots, B, S, Hkv, Dh))
    V = rng.standard_normal((n_slots, B, S, Hkv, Dh))
    q = rng.standard_normal((5, 4, Dh))
    trip = [(0, 0, 3), (3, 2, 15), (1, 1, 0), (2, 0, 9), (3, 1, 7)]  # (slot, seq, pos)
    rb = [(sl * B + b) * S for sl, b, _ in trip]
    kl = [p + 1 for _, _, p in trip]
    got = ok.attention_rows(q, K.reshape(-1, Hkv, Dh), V.reshape(-1, Hkv, Dh), rb, kl)
    for i, (sl, b, p) in enumerate(trip):
        np.testing.assert_allclose(got[i], ok.attention(q[i], K[sl, b], V[sl, b], p + 1), rtol=1e-12)


def test_rmsnorm_matches_torch():
    rng = np.random.default_rng(3)
    x = rng.standard_normal((5, 256))
    w = rng.standard_normal(256)
    ref = F.rms_norm(torch.from_numpy(x), (256,), torch.from_numpy(w), eps=1e-6).numpy()
    np.testing.assert_allclose(ok.rmsnorm(x, w, 1e-6), ref, rtol=1e-12)


def test_rope_is_complex_rotation():
    cos, sin = ok.rope_tables(64, 16, 10000.0)
    rng = np.random.default_rng(4)
    x = rng.standard_normal((3, 16))
    for pos in (0, 1, 17, 63):
        got = ok.rope(x, pos, cos.astype(np.float64), sin.astype(np.float64))
        theta = 10000.0 ** (-np.arange(8) * 2.0 / 16)
        z = (x[:, 0::2] + 1j * x[:, 1::2]) * np.exp(1j * pos * theta)
        ref = np.empty_like(x)
        ref[:, 0::2], ref[:, 1::2] = z.real, z.imag
        np.testing.assert_allclose(got, ref, rtol=2e-6, atol=2e-6)
        np.testing.assert_allclose(np.linalg.norm(got, axis=1), np.linalg.norm(x, axis=1), rtol=1e-6)
    # relative-position property: <rope(q, m), rope(k, n)> depends on m - n only
    q, k = rng.standard_normal(16), rng.standard_normal(16)
    c64, s64 = cos.astype(np.float64), sin.astype(np.float64)
    d1 = ok.rope(q[None], 20, c64, s64)[0] @ ok.rope(k[None], 13, c64, s64)[0]
    d2 = ok.rope(q[None], 50, c64, s64)[0] @ ok.rope(k[None], 43, c64, s64)[0]
    assert abs(d1 - d2) < 1e-5


def test_swiglu_matches_torch():
    rng = np.random.default_rng(5)
    g, u = rng.standard_normal(100), rng.standard_normal(100)
    ref = (F.silu(torch.from_numpy(g)) * torch.from_numpy(u)).numpy()
    np.testing.assert_allclose(ok.swiglu(g, u), ref, rtol=1e-12)


def test_linear_rows_match_matmul():
    rng = np.random.default_rng(6)
    x = rng.standard_normal((4, 32))
    W = rng.standard_normal((48, 32))
    np.testing.assert_allclose(ok.linear(x, W), x @ W.T, rtol=1e-12)
