"""Folded RMSNorm pairs (include/wfd.h, wfd_prep_t): the residual stream and
the next linear's operand prepared in a linear's epilogue (wfd_linear_prep)
or by the row kernel (wfd_norm_prep, from rows or from split-K slices), and
the consumer's row scale taken from group sums or precomputed (GPU).

* Every form gives the same bits: r, A, s_a, the consumer's outputs (plain,
  SwiGLU through the 8-wave few-row kernel, QKV-RoPE-append, the lm_head
  group argmax) and the block's last norm, at 1-16 rows and, for the row
  kernel and the many-row consumers, at 17-96 rows.
* Against the oracle: the consumer's output equals linear(norm_b(norm_a(
  y + x_res))) computed in float64 (2e-2 bf16, 1e-4 fp32), for a pair with
  and without its first norm, with and without a residual.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import kernels as ok
from tests.conftest import rel_err
from wavefront_decoding_amd import ops

pytestmark = pytest.mark.gpu

TOL = {torch.bfloat16: 2e-2, torch.float32: 1e-4}


def _np(t):
    return t.detach().float().cpu().numpy().astype(np.float64)


def _case(gpu, dtype, n, D, K, seed):
    g = torch.Generator().manual_seed(seed)
    mk = lambda *s, sc=1.0: (sc * torch.randn(*s, generator=g)).to(dtype).to(gpu)  # noqa: E731
    return dict(x=mk(n, K), W=mk(D, K, sc=0.02), r_in=mk(n, D), s_in=(0.5 + torch.rand(n, generator=g)).to(gpu),
                w_in=mk(D, sc=0.1) + 1, wa=mk(D, sc=0.1) + 1, wb=mk(D, sc=0.1) + 1)


def _reference(c, eps, res: bool, two: bool):
    """float64: y = x W^T rounded as the linear stores it; r = round(y + x_res);
    h = norm_b(norm_a(r)) (norm_a absent: h = norm_b(r))."""
    dt = c["x"].dtype
    rnd = lambda a: torch.from_numpy(a).to(dt).double().numpy()  # noqa: E731
    y = rnd(_np(c["x"]) @ _np(c["W"]).T)
    if res:
        xr = rnd(_np(c["r_in"]) * _np(c["s_in"])[:, None] * _np(c["w_in"])[None, :])
        r = rnd(y + xr)
    else:
        r = y
    if two:
        r = ok.rmsnorm(r, _np(c["wa"]), eps)
    return r, ok.rmsnorm(r, _np(c["wb"]), eps)


def _row_forms(c, n, D, dtype, eps, res, two):
    """The row kernel from the one-launch linear's rows and from split-K slices,
    each also writing norm a's output h (the many-row residual stream)."""
    out = []
    kw = dict(r_in=c["r_in"], s_in=c["s_in"], w_in=c["w_in"]) if res else {}
    for split in (False, True):
        r = torch.empty(n, D, dtype=dtype, device=c["x"].device)
        A = torch.empty_like(r)
        sc = torch.empty(n, dtype=torch.float32, device=r.device)
        sa = torch.full((n,), -1.0, dtype=torch.float32, device=r.device)
        if split:
            part = torch.empty(4 * n * D, dtype=torch.float32, device=r.device)
            S = ops.linear_partials(c["x"], c["W"], part, n=n)
            src = dict(part=part, nslices=S)
        else:
            src = dict(a=ops.linear(c["x"], c["W"], n=n))
        h = torch.empty_like(r)
        ops.norm_prep(n=n, D=D, dtype=dtype, eps=eps, r_out=r, a_out=A, wa=c["wa"] if two else None, wb=c["wb"],
                      two=two, scale_out=sc, s_out=sa, h_out=h, **kw, **src)
        out.append((r, A, sc, sa, h))
    return out


@pytest.mark.parametrize("dtype,D,K", [(torch.bfloat16, 2048, 2048), (torch.bfloat16, 2048, 5632),
                                       (torch.bfloat16, 512, 1024), (torch.bfloat16, 128, 256),
                                       (torch.float32, 256, 1024)])
@pytest.mark.parametrize("res,two", [(True, True), (False, False), (True, False)])
def test_prep_forms_same_bits_and_match_oracle(gpu, dtype, D, K, res, two):
    eps = 1e-6
    for n in (1, 3, 8, 16):
        c = _case(gpu, dtype, n, D, K, n + K)
        print(f"[fold] dtype={dtype} D={D} K={K} res={res} two={two} n={n}", flush=True)
        kw = dict(r_in=c["r_in"], s_in=c["s_in"], w_in=c["w_in"]) if res else {}
        r1 = torch.empty(n, D, dtype=dtype, device=gpu)
        A1 = torch.empty_like(r1)
        gp = torch.full((n * ops.FOLD_SLOTS * 2,), float("nan"), dtype=torch.float32, device=gpu)
        ops.linear_prep(c["x"], c["W"], n=n, r_out=r1, a_out=A1, wa=c["wa"] if two else None, wb=c["wb"], part=gp,
                        **kw)
        hf = torch.empty_like(r1)  # norm a alone, from r (the block's last-norm form)
        ops.norm_prep(n=n, D=D, dtype=dtype, eps=eps, a=r1, wa=c["wa"] if two else None, h_out=hf, two=two)
        for r2, A2, sc2, sa2, h2 in _row_forms(c, n, D, dtype, eps, res, two):
            assert torch.equal(r1, r2) and torch.equal(A1, A2) and torch.equal(h2, hf)
        # consumers: group sums (few rows) against precomputed scales
        W2 = (0.02 * torch.randn(1024, D, generator=torch.Generator().manual_seed(7))).to(dtype).to(gpu)
        sa1 = torch.full((n,), -1.0, dtype=torch.float32, device=gpu)
        y1 = ops.linear(A1, W2, n=n, rowscale=ops.RowScale(D=D, eps=eps, two=two, part=gp, s_out=sa1))
        y2 = ops.linear(A2, W2, n=n, rowscale=ops.RowScale(D=D, eps=eps, two=two, scale=sc2))
        assert torch.equal(y1, y2) and torch.equal(sa1, sa2)
        if not two:
            assert torch.all(sa1 == 1.0)
        rr, h = _reference(c, eps, res, two)
        assert rel_err(_np(y1), h @ _np(W2).T) <= TOL[dtype]
        if two:
            assert rel_err(_np(hf), rr) <= TOL[dtype]
        else:  # no norm a: s_a = 1 and h = r
            assert torch.equal(hf, r1)


@pytest.mark.parametrize("dtype,D", [(torch.bfloat16, 2048), (torch.bfloat16, 512), (torch.float32, 256)])
def test_consumers_same_bits_at_any_row_count(gpu, dtype, D):
    """A row's outputs do not depend on n: rows prepared and consumed at 1-16
    rows (group sums, few-row kernels -- SwiGLU at 704 tiles takes the 8-wave
    form) equal the same rows inside 17-96-row launches (split slices, row
    kernel, precomputed scales, many-row kernels), for plain, SwiGLU and the
    lm_head group argmax."""
    eps = 1e-6
    N = 96
    c = _case(gpu, dtype, N, D, D, 3)
    F = 5632 if D == 2048 else 1024
    g = torch.Generator().manual_seed(11)
    Wfc = ops.pack_linear((0.02 * torch.randn(2 * F, D, generator=g)).to(dtype).to(gpu), swiglu=True)
    Wlm = (0.02 * torch.randn(4096, D, generator=g)).to(dtype).to(gpu)

    def run(rows):
        n = len(rows)
        idx = torch.tensor(rows, device=gpu)
        cc = {k: (v[idx] if k in ("x", "r_in", "s_in") else v) for k, v in c.items()}
        r = torch.empty(n, D, dtype=dtype, device=gpu)
        A = torch.empty_like(r)
        if n <= 16:
            gp = torch.empty(n * ops.FOLD_SLOTS * 2, dtype=torch.float32, device=gpu)
            ops.linear_prep(cc["x"], cc["W"], n=n, r_in=cc["r_in"], s_in=cc["s_in"], w_in=cc["w_in"], r_out=r,
                            a_out=A, wa=cc["wa"], wb=cc["wb"], part=gp)
            rs = ops.RowScale(D=D, eps=eps, two=True, part=gp)
        else:
            (r, A, sc, _, _), _ = _row_forms(cc, n, D, dtype, eps, True, True)
            rs = ops.RowScale(D=D, eps=eps, two=True, scale=sc)
        u = ops.linear(A, Wfc, n=n, swiglu=True, rowscale=rs)
        lg = ops.linear(A, Wlm, n=n, out_dtype=torch.float32, rowscale=rs)
        ids = ops.argmax(lg, n=n)
        if n <= 16 and dtype == torch.bfloat16:
            G = ops.linear_argmax_groups(n, Wlm)
            lg2, pv, pi = ops.linear_argmax(A, Wlm, n=n, rowscale=rs)
            assert torch.equal(lg2[:n], lg[:n])
            assert torch.equal(ops.argmax_groups(pv, pi, G, n=n), ids)
        return r, A, u, lg, ids

    big = run(list(range(N)))
    for rows in ([5], [0, 7, 9], list(range(40, 56)), list(range(30, 60))):
        print(f"[fold rows] dtype={dtype} rows={rows[:4]}.. n={len(rows)}", flush=True)
        small = run(rows)
        for a, b in zip(small, big):
            assert torch.equal(a[: len(rows)], b[rows]), rows


@pytest.mark.parametrize("n", [1, 8, 40])
def test_final_norm_and_qkv_consumer(gpu, n):
    """The block's last norm written to a row table (from the few-row
    producer's r rows and from split slices: same bits, against float64), and
    the QKV-RoPE-append consumer with a row scale (group sums or
    precomputed) equal to the unscaled kernel fed the normalized rows within
    the bf16 tolerance."""
    D, H, Hkv, Dh, eps = 2048, 16, 16, 128, 1e-6
    dtype = torch.bfloat16
    c = _case(gpu, dtype, n, D, D, 21 + n)
    rows = torch.randperm(64, generator=torch.Generator().manual_seed(n))[:n].to(torch.int32).to(gpu)
    out = []
    for split in ((False, True) if n > 16 else (False,)):
        h = torch.zeros(64, D, dtype=dtype, device=gpu)
        if split:
            part = torch.empty(4 * n * D, dtype=torch.float32, device=gpu)
            S = ops.linear_partials(c["x"], c["W"], part, n=n)
            ops.norm_prep(n=n, D=D, dtype=dtype, eps=eps, part=part, nslices=S, r_in=c["r_in"], s_in=c["s_in"],
                          w_in=c["w_in"], wa=c["wa"], h_out=h, h_rows=rows)
        else:
            r = torch.empty(n, D, dtype=dtype, device=gpu)
            if n <= 16:
                ops.linear_prep(c["x"], c["W"], n=n, r_in=c["r_in"], s_in=c["s_in"], w_in=c["w_in"], r_out=r,
                                a_out=torch.empty_like(r), wb=c["wa"],
                                part=torch.empty(n * ops.FOLD_SLOTS * 2, dtype=torch.float32, device=gpu))
            else:
                (r, _, _, _, _), _ = _row_forms(c, n, D, dtype, eps, True, True)
            ops.norm_prep(n=n, D=D, dtype=dtype, eps=eps, a=r, wa=c["wa"], h_out=h, h_rows=rows)
        out.append(h)
    assert all(torch.equal(o, out[0]) for o in out)
    hr, _ = _reference(c, eps, True, True)
    assert rel_err(_np(out[0][rows.long()]), hr) <= 2e-2
    # QKV consumer: scaled operand vs the plain kernel on the normalized rows
    g = torch.Generator().manual_seed(5)
    Wq = (0.02 * torch.randn((H + 2 * Hkv) * Dh, D, generator=g)).to(dtype).to(gpu)
    from wavefront_decoding_amd.model import rope_tables
    cos, sin = [t.to(gpu) for t in rope_tables(256, Dh, 10000.0)]
    pos = torch.randint(0, 256, (n,), generator=g).to(torch.int32).to(gpu)
    fr = torch.arange(n, dtype=torch.int64, device=gpu)
    r = torch.empty(n, D, dtype=dtype, device=gpu)
    A = torch.empty_like(r)
    if n <= 16:
        gp = torch.empty(n * ops.FOLD_SLOTS * 2, dtype=torch.float32, device=gpu)
        ops.linear_prep(c["x"], c["W"], n=n, r_in=c["r_in"], s_in=c["s_in"], w_in=c["w_in"], r_out=r, a_out=A,
                        wa=c["wa"], wb=c["wb"], part=gp)
        rs = ops.RowScale(D=D, eps=eps, two=True, part=gp)
    else:
        (r, A, sc, _, _), _ = _row_forms(c, n, D, dtype, eps, True, True)
        rs = ops.RowScale(D=D, eps=eps, two=True, scale=sc)
    kc = torch.zeros(n, Hkv, Dh, dtype=dtype, device=gpu)
    vc = torch.zeros_like(kc)
    q = ops.linear_qkv_rope_append(A, Wq, pos, cos, sin, fr, kc, vc, H, Hkv, Dh, n=n, rowscale=rs)
    _, hb = _reference(c, eps, True, True)
    hb_t = torch.from_numpy(hb).to(dtype).to(gpu)
    kc2, vc2 = torch.zeros_like(kc), torch.zeros_like(vc)
    q2 = ops.linear_qkv_rope_append(hb_t, Wq, pos, cos, sin, fr, kc2, vc2, H, Hkv, Dh, n=n)
    for a, b in ((q, q2), (kc, kc2), (vc, vc2)):
        assert rel_err(_np(a), _np(b)) <= 2e-2
