"""The reference's attention-backend API (wavefront_decoding_amd.attention)
against the oracle (GPU).

Each entry point is called with the argument layout the reference's callers
use (src/decoding/fa4_attention.py:191-342): packed varlen segments with
cu_seqlens, dense (B, T, H, Dh) batches, the coda's per-query cutoff, and the
q1 padded form. Tolerance: max relative error 2e-2 (bf16) / 1e-4 (fp32).
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import kernels as ok
from tests.conftest import rel_err
from wavefront_decoding_amd import attention as A

pytestmark = pytest.mark.gpu

TOL = {torch.bfloat16: 2e-2, torch.float32: 1e-4}


def _np(t):
    return t.detach().float().cpu().numpy().astype(np.float64)


def _varlen_ref(q, k, v, cu_q, cu_k, causal):
    """Oracle: each segment's rows over the segment's keys, bottom-right causal
    per segment when asked (rows with no keys are zero)."""
    qn, kn, vn = _np(q), _np(k), _np(v)
    out = np.zeros_like(qn)
    for s in range(len(cu_q) - 1):
        q0, q1, k0, k1 = cu_q[s], cu_q[s + 1], cu_k[s], cu_k[s + 1]
        ql, kl = q1 - q0, k1 - k0
        for r in range(ql):
            n = max(kl - ql + r + 1, 0) if causal else kl
            out[q0 + r] = ok.attention(qn[q0 + r], kn[k0:k1], vn[k0:k1], n)
    return out


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("H,Hkv,Dh", [(16, 16, 128), (16, 4, 128), (4, 4, 64)])
def test_attn_varlen_matches_oracle(gpu, dtype, causal, H, Hkv, Dh):
    """Packed segments of ragged query and key lengths, including one with
    fewer keys than queries (its first rows have no keys under causal) and a
    long one that spans several key splits."""
    seg = [(1, 700), (5, 5), (3, 1), (8, 2500), (1, 1), (4, 33)]  # (q_len, k_len)
    cu_q = np.concatenate([[0], np.cumsum([a for a, _ in seg])]).astype(np.int32)
    cu_k = np.concatenate([[0], np.cumsum([b for _, b in seg])]).astype(np.int32)
    g = torch.Generator().manual_seed(H * 7 + Dh + causal)
    q = torch.randn(int(cu_q[-1]), H, Dh, generator=g).to(dtype)
    k = torch.randn(int(cu_k[-1]), Hkv, Dh, generator=g).to(dtype)
    v = torch.randn(int(cu_k[-1]), Hkv, Dh, generator=g).to(dtype)
    print(f"[attn_varlen] dtype={dtype} causal={causal} H={H} Hkv={Hkv} Dh={Dh}", flush=True)
    out = A.attn_varlen(q.to(gpu), k.to(gpu), v.to(gpu), torch.from_numpy(cu_q).to(gpu),
                        torch.from_numpy(cu_k).to(gpu), max(a for a, _ in seg), max(b for _, b in seg), causal=causal)
    ref = _varlen_ref(q, k, v, cu_q, cu_k, causal)
    assert rel_err(_np(out), ref) <= TOL[dtype]
    if causal:  # rows with no keys come back as zeros
        assert torch.count_nonzero(out[cu_q[2]: cu_q[2] + 2].float()) == 0


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_attn_varlen_q1_padded_matches_oracle(gpu, dtype):
    lens = [1, 64, 300, 1025, 7]
    cu_k = np.concatenate([[0], np.cumsum(lens)]).astype(np.int32)
    g = torch.Generator().manual_seed(5)
    q = torch.randn(len(lens), 16, 128, generator=g).to(dtype)
    k = torch.randn(int(cu_k[-1]), 16, 128, generator=g).to(dtype)
    v = torch.randn(int(cu_k[-1]), 16, 128, generator=g).to(dtype)
    out = A.attn_varlen_q1_padded(q.to(gpu), k.to(gpu), v.to(gpu), torch.from_numpy(cu_k).to(gpu), max(lens))
    ref = _varlen_ref(q, k, v, np.arange(len(lens) + 1), cu_k, False)
    assert rel_err(_np(out), ref) <= TOL[dtype]


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("B,Tq,Tk,H,Hkv,Dh", [(2, 200, 200, 16, 4, 128), (3, 7, 150, 4, 4, 64),
                                             (1, 1, 300, 16, 16, 128), (2, 40, 20, 4, 2, 64)])
def test_attn_dense_matches_oracle(gpu, dtype, causal, B, Tq, Tk, H, Hkv, Dh):
    """Bottom-right causal (or full) dense attention over (B, T, H, Dh)
    batches: bf16 prompts go through the MFMA prefill kernel, the rest through
    the decode kernel; Tq > Tk leaves the first rows without keys (zeros)."""
    g = torch.Generator().manual_seed(B * 100 + Tq + Tk)
    q = torch.randn(B, Tq, H, Dh, generator=g).to(dtype)
    k = torch.randn(B, Tk, Hkv, Dh, generator=g).to(dtype)
    v = torch.randn(B, Tk, Hkv, Dh, generator=g).to(dtype)
    out = A.attn_dense(q.to(gpu), k.to(gpu), v.to(gpu), causal=causal)
    qn, kn, vn = _np(q), _np(k), _np(v)
    ref = np.zeros_like(qn)
    for b in range(B):
        for j in range(Tq):
            n = max(Tk - Tq + j + 1, 0) if (causal and Tq > 1) else Tk
            ref[b, j] = ok.attention(qn[b, j], kn[b], vn[b], n)
    assert out.shape == q.shape
    assert rel_err(_np(out), ref) <= TOL[dtype]


def test_attn_cutoff_multi_matches_oracle(gpu):
    """The coda's verify + draft rows at disjoint positions on one slot."""
    g = torch.Generator().manual_seed(9)
    qpos = [510, 517, 600]
    Tk = max(qpos) + 1
    q = torch.randn(1, 3, 16, 128, generator=g).to(torch.bfloat16)
    k = torch.randn(1, Tk, 16, 128, generator=g).to(torch.bfloat16)
    v = torch.randn(1, Tk, 16, 128, generator=g).to(torch.bfloat16)
    for pos in (qpos, torch.tensor(qpos, device=gpu)):
        out = A.attn_cutoff_multi(q.to(gpu), k.to(gpu), v.to(gpu), pos)
        ref = np.stack([ok.attention(_np(q)[0, j], _np(k)[0], _np(v)[0], p + 1) for j, p in enumerate(qpos)])
        assert rel_err(_np(out)[0], ref) <= 2e-2


def test_compute_qkv_matches_oracle(gpu):
    """Fused Wqkv projection + interleaved-pair RoPE at given positions."""
    from wavefront_decoding_amd.model import rope_tables

    class Attn:
        n_head, n_kv_head, head_dim = 4, 2, 64

    g = torch.Generator().manual_seed(2)
    B, T, C = 2, 5, 256
    N = (4 + 2 * 2) * 64
    Attn.Wqkv = (0.05 * torch.randn(N, C, generator=g)).to(gpu)
    x = torch.randn(B, T, C, generator=g).to(gpu)
    cos, sin = rope_tables(64, 64, 10000.0)
    pos = torch.tensor([3, 4, 9, 10, 40], dtype=torch.int32)
    q, k, v = A.compute_qkv(Attn, x, (cos.to(gpu), sin.to(gpu), pos.to(gpu)))
    qkv = _np(x).reshape(B * T, C) @ _np(Attn.Wqkv).T
    oc, os_ = ok.rope_tables(64, 64)
    for r in range(B * T):
        p = int(pos[r % T])
        qr = ok.rope(qkv[r, :256].reshape(4, 64), p, oc, os_)
        kr = ok.rope(qkv[r, 256:384].reshape(2, 64), p, oc, os_)
        assert rel_err(_np(q).reshape(B * T, 4, 64)[r], qr) <= 1e-4
        assert rel_err(_np(k).reshape(B * T, 2, 64)[r], kr) <= 1e-4
        assert rel_err(_np(v).reshape(B * T, 2, 64)[r], qkv[r, 384:].reshape(2, 64)) <= 1e-4


@pytest.mark.parametrize("dtype,H,Hkv,Dh", [(torch.bfloat16, 16, 16, 128), (torch.bfloat16, 16, 4, 128),
                                            (torch.float32, 4, 2, 64)])
def test_compute_qkv_reference_form(gpu, dtype, H, Hkv, Dh):
    """The reference's call form (src/decoding/fa4_attention.py:128-152):
    separate bias-free c_q / c_k / c_v nn.Linear projections and complex
    freqs_cis shaped (1, T, 1, Dh/2). q and k are the projections rotated as
    complex numbers (x[2j] + i x[2j+1]) * freqs[t, j], v the plain projection
    (numpy, float64); the fused-Wqkv form gives the same bits; use_rope =
    False returns the plain projections; a weight changed in place is seen."""
    g = torch.Generator().manual_seed(H + Hkv + Dh)
    B, T, C = 2, 7, 512

    class Attn(torch.nn.Module):
        def __init__(self):
            super().__init__()
            self.n_head, self.n_kv_head, self.head_dim = H, Hkv, Dh
            self.c_q = torch.nn.Linear(C, H * Dh, bias=False)
            self.c_k = torch.nn.Linear(C, Hkv * Dh, bias=False)
            self.c_v = torch.nn.Linear(C, Hkv * Dh, bias=False)

    attn = Attn()
    with torch.no_grad():
        for m in (attn.c_q, attn.c_k, attn.c_v):
            m.weight.copy_(0.05 * torch.randn(m.weight.shape, generator=g))
    attn = attn.to(device=gpu, dtype=dtype)
    x = torch.randn(B, T, C, generator=g).to(device=gpu, dtype=dtype)
    ang = torch.rand(T, Dh // 2, generator=g, dtype=torch.float64) * 6.0
    freqs = torch.polar(torch.ones_like(ang), ang).to(torch.complex64).view(1, T, 1, Dh // 2)

    def reference(x, attn):
        xs = _np(x).reshape(B * T, C)
        qs = xs @ _np(attn.c_q.weight).T
        ks = xs @ _np(attn.c_k.weight).T
        vs = xs @ _np(attn.c_v.weight).T
        f = freqs.view(T, Dh // 2).to(torch.complex128).numpy()

        def rot(a, heads):
            a = a.reshape(B, T, heads, Dh // 2, 2)
            z = (a[..., 0] + 1j * a[..., 1]) * f[None, :, None, :]
            return np.stack([z.real, z.imag], axis=-1).reshape(B, T, heads, Dh)

        return rot(qs, H), rot(ks, Hkv), vs.reshape(B, T, Hkv, Dh)

    q, k, v = A.compute_qkv(attn, x, freqs, None, None)
    rq, rk, rv = reference(x, attn)
    tol = TOL[dtype]
    assert rel_err(_np(q), rq) <= tol and rel_err(_np(k), rk) <= tol and rel_err(_np(v), rv) <= tol

    class Fused:
        n_head, n_kv_head, head_dim = H, Hkv, Dh
        Wqkv = torch.cat([attn.c_q.weight, attn.c_k.weight, attn.c_v.weight]).detach().contiguous()

    q2, k2, v2 = A.compute_qkv(Fused, x, freqs)
    assert torch.equal(q2, q) and torch.equal(k2, k) and torch.equal(v2, v)

    class NoRope:
        class rope_settings:
            use_rope = False
        clip_qkv = None
        qk_bias = False
        qk_norm = False

    q3, k3, v3 = A.compute_qkv(attn, x, freqs, None, NoRope)
    xs = _np(x).reshape(B * T, C)
    assert rel_err(_np(q3).reshape(B * T, -1), xs @ _np(attn.c_q.weight).T) <= tol
    assert rel_err(_np(k3).reshape(B * T, -1), xs @ _np(attn.c_k.weight).T) <= tol
    assert torch.equal(v3, v)

    with torch.no_grad():
        attn.c_k.weight.mul_(-1)  # in place: the packed copy must be rebuilt
    q4, k4, v4 = A.compute_qkv(attn, x, freqs)
    assert torch.equal(q4, q) and torch.equal(v4, v) and torch.equal(k4, -k)
