"""Kernel-level parity of libwfd.so against the CPU oracle (GPU).

Tolerances (max|gpu - oracle| / max|oracle|): 2e-2 for bf16, 1e-4 for fp32.
Integer/index work (slot append rows, argmax ids) must be bit-exact, and every
kernel must be row-invariant (a row's bits do not depend on the batch).
"""
from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from oracle import kernels as ok
from tests.conftest import rel_err
from wavefront_decoding_amd import ops

pytestmark = pytest.mark.gpu

TOL = {torch.bfloat16: 2e-2, torch.float32: 1e-4}


def _np(t: torch.Tensor) -> np.ndarray:
    return t.detach().float().cpu().numpy().astype(np.float64)


def _attn_case(dev, dtype, n, H, Hkv, Dh, lens, S=None, seed=0):
    g = torch.Generator().manual_seed(seed)
    S = S or max(lens) + 3
    n_slots = n + 1
    K = torch.randn(n_slots * S, Hkv, Dh, generator=g).to(dtype)
    V = torch.randn(n_slots * S, Hkv, Dh, generator=g).to(dtype)
    q = torch.randn(n, H, Dh, generator=g).to(dtype)
    # query i reads slot (i+1) % n_slots -- a different slot per query
    rb = torch.tensor([((i + 1) % n_slots) * S for i in range(n)], dtype=torch.int64)
    kl = torch.tensor(lens, dtype=torch.int32)
    return q, K, V, rb, kl


def _blocks(t: torch.Tensor, S: int) -> torch.Tensor:
    """Token-major cache (nblk*S, Hkv, Dh) -> head-major blocks (nblk, Hkv, S, Dh)."""
    return t.view(-1, S, t.shape[1], t.shape[2]).permute(0, 2, 1, 3).contiguous()


def _rows(t: torch.Tensor) -> torch.Tensor:
    """Head-major blocks (nblk, Hkv, S, Dh) -> token-major rows (nblk*S, Hkv, Dh)."""
    return t.permute(0, 2, 1, 3).reshape(-1, t.shape[1], t.shape[3])


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("H,Hkv,Dh,lens", [
    (16, 16, 64, [1017 + i for i in range(8)]),      # wavefront attention op, W=8, L=1024
    (16, 16, 128, [512 + i for i in range(8)]),      # 2048-d model decode tick
    (16, 4, 128, [3000, 2999, 1, 256, 257, 255, 64, 65]),  # GQA 16/4 + split/tile edges
    (4, 4, 64, [1, 2, 63, 64, 65, 129]),             # tiny model heads
])
def test_attn_decode_matches_oracle(gpu, dtype, H, Hkv, Dh, lens):
    """Both cache layouts, against the oracle; the head-major block layout
    gives the token-major result bit for bit (only addresses differ)."""
    n = len(lens)
    S = max(lens) + 3
    q, K, V, rb, kl = _attn_case(gpu, dtype, n, H, Hkv, Dh, lens, S=S)
    print(f"[attn] dtype={dtype} n={n} H={H} Hkv={Hkv} Dh={Dh} lens={lens}", flush=True)
    out = ops.attn_decode(q.to(gpu), K.to(gpu), V.to(gpu), rb.to(gpu), kl.to(gpu), kv_len_max=max(lens))
    outb = ops.attn_decode(q.to(gpu), _blocks(K, S).to(gpu), _blocks(V, S).to(gpu), rb.to(gpu), kl.to(gpu),
                           kv_len_max=max(lens))
    torch.cuda.synchronize()
    ref = ok.attention_rows(_np(q), _np(K), _np(V), rb.numpy(), kl.numpy())
    err = rel_err(_np(out), ref)
    assert err <= TOL[dtype], err
    assert torch.equal(out, outb)


@pytest.mark.parametrize("L", [4096, 16384])
def test_attn_decode_long_prefix(gpu, L):
    lens = [L - 7 + i for i in range(8)]
    S = L + 3
    q, K, V, rb, kl = _attn_case(gpu, torch.bfloat16, 8, 16, 16, 64, lens, S=S, seed=L)
    out = ops.attn_decode(q.to(gpu), _blocks(K, S).to(gpu), _blocks(V, S).to(gpu), rb.to(gpu), kl.to(gpu),
                          kv_len_max=L)
    ref = ok.attention_rows(_np(q), _np(K), _np(V), rb.numpy(), kl.numpy())
    assert rel_err(_np(out), ref) <= 2e-2


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("H,Hkv,Dh", [(16, 16, 128), (16, 4, 128), (4, 4, 64)])
def test_attn_decode_row_invariant(gpu, dtype, H, Hkv, Dh):
    """A query's output bits do not depend on the other queries, the batch
    size, or kv_len_max (the grid bound): alone (each (split, head, row)
    split over two workgroups by output columns), among 8 rows and among 64
    rows (one workgroup each at 16 kv heads)."""
    lens = [700, 33, 1500, 256, 1, 900, 511, 1024]
    q, K, V, rb, kl = _attn_case(gpu, dtype, 8, H, Hkv, Dh, lens, S=1803, seed=7 + Hkv + Dh)
    K, V = _blocks(K, 1803), _blocks(V, 1803)
    q, K, V, rb, kl = (t.to(gpu) for t in (q, K, V, rb, kl))
    print(f"[attn row-invariant] dtype={dtype} H={H} Hkv={Hkv} Dh={Dh}", flush=True)
    full = ops.attn_decode(q, K, V, rb, kl, kv_len_max=1500)  # 2 x Hkv x 8 workgroups (x2 column parts at Hkv 4)
    for i in range(8):
        one = ops.attn_decode(q[i:i + 1].contiguous(), K, V, rb[i:i + 1], kl[i:i + 1], kv_len_max=lens[i] + 300)
        assert torch.equal(one[0], full[i]), i
    # the same 8 queries repeated over 64 rows: 2 x Hkv x 64 workgroups
    big = ops.attn_decode(q.repeat(8, 1, 1), K, V, rb.repeat(8), kl.repeat(8), kv_len_max=1500)
    for r in range(64):
        assert torch.equal(big[r], full[r % 8]), r
    ref = ok.attention_rows(_np(q), _np(_rows(K)), _np(_rows(V)), rb.cpu().numpy(), kl.cpu().numpy())
    assert rel_err(_np(full), ref) <= TOL[dtype]


@pytest.mark.parametrize("blocks", [False, True])
@pytest.mark.parametrize("H,Hkv,Dh,segs", [
    (16, 16, 128, [(0, 200)]),                          # one 2048-d-model prompt
    (16, 4, 128, [(0, 64), (0, 65), (37, 100)]),        # GQA, tile edges, a segment after a cached prefix
    (4, 4, 64, [(0, 1), (5, 3), (0, 130), (120, 70)]),  # tiny heads, 1-row and ragged segments
    (16, 16, 64, [(0, 257), (300, 1)]),                 # a lone query over a 300-key prefix
    (16, 16, 128, [(0, 1000), (0, 63), (64, 64)]),      # many tiles per key stream, odd and even tile counts
    (16, 16, 64, [(0, 2100), (10, 300)]),               # one key stream (> 2048 rows at 16 heads) beside two
])
def test_attn_prefill_matches_oracle(gpu, H, Hkv, Dh, segs, blocks):
    """MFMA causal prefill: segment (pos0, len) on its own slot, each row
    attending keys [0, its position]; against the oracle, and both cache
    layouts give the same bits. A segment takes one or two key streams by its
    own length, so each segment's rows equal its rows launched alone."""
    dtype = torch.bfloat16
    g = torch.Generator().manual_seed(len(segs) * 31 + Dh)
    S = max(p0 + n for p0, n in segs) + 5
    n_slots = len(segs) + 1
    K = torch.randn(n_slots * S, Hkv, Dh, generator=g).to(dtype)
    V = torch.randn(n_slots * S, Hkv, Dh, generator=g).to(dtype)
    n = sum(ln for _, ln in segs)
    q = torch.randn(n, H, Dh, generator=g).to(dtype)
    seg_rb = torch.tensor([(s + 1) * S for s in range(len(segs))], dtype=torch.int64)
    qs = torch.tensor(np.cumsum([0] + [ln for _, ln in segs]), dtype=torch.int32)
    p0 = torch.tensor([p for p, _ in segs], dtype=torch.int32)
    rb = torch.cat([torch.full((ln,), int(seg_rb[s])) for s, (_, ln) in enumerate(segs)])
    kl = torch.cat([torch.arange(p + 1, p + ln + 1) for p, ln in segs]).to(torch.int32)
    print(f"[prefill] H={H} Hkv={Hkv} Dh={Dh} segs={segs} blocks={blocks}", flush=True)
    Kd, Vd = (_blocks(K, S), _blocks(V, S)) if blocks else (K, V)
    mx = max(ln for _, ln in segs)
    out = ops.attn_prefill(q.to(gpu), Kd.to(gpu), Vd.to(gpu), seg_rb.to(gpu), qs.to(gpu), p0.to(gpu), max_seg_len=mx)
    other = ops.attn_prefill(q.to(gpu), (K if blocks else _blocks(K, S)).to(gpu),
                             (V if blocks else _blocks(V, S)).to(gpu), seg_rb.to(gpu), qs.to(gpu), p0.to(gpu),
                             max_seg_len=mx)
    torch.cuda.synchronize()
    ref = ok.attention_rows(_np(q), _np(K), _np(V), rb.numpy(), kl.numpy())
    assert rel_err(_np(out), ref) <= 2e-2
    assert torch.equal(out, other)
    if len(segs) > 1:  # each segment alone: the same bits
        for i, (pp, ln) in enumerate(segs):
            alone = ops.attn_prefill(q[qs[i]:qs[i + 1]].to(gpu), Kd.to(gpu), Vd.to(gpu), seg_rb[i:i + 1].to(gpu),
                                     torch.tensor([0, ln], dtype=torch.int32, device=gpu), p0[i:i + 1].to(gpu),
                                     max_seg_len=ln)
            assert torch.equal(alone, out[qs[i]:qs[i + 1]]), i
    # per-row agreement with the decode kernel on the same rows (different arithmetic, same math)
    dec = ops.attn_decode(q.to(gpu), K.to(gpu), V.to(gpu), rb.to(gpu), kl.to(gpu), kv_len_max=int(kl.max()))
    assert rel_err(_np(out), _np(dec)) <= 2e-2


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("H,Hkv,Dh", [(16, 16, 128), (16, 8, 64), (16, 4, 128), (4, 4, 64)])
def test_attn_decode_grouped_rows_same_bits(gpu, dtype, H, Hkv, Dh):
    """Rows that share a slot, grouped (one prefix read per group), give the
    ungrouped rows' bits exactly -- ragged lengths inside a group, groups that
    straddle the 1024- and 2048-key split edges, a 1-row group, and the oracle
    agrees."""
    gmax = ops.attn_group_max_rows(H, Hkv)
    g = torch.Generator().manual_seed(H * 3 + Hkv + Dh)
    groups = [[700, 701, 702, 650], [50], [2040, 2048, 2049, 3000, 10, 2100, 1, 4100][:gmax], [2047, 2048][:gmax],
              [1023, 1024, 1025, 1026][:gmax]]
    S = 4200
    n_slots = len(groups) + 1
    K = torch.randn(n_slots * S, Hkv, Dh, generator=g).to(dtype)
    V = torch.randn(n_slots * S, Hkv, Dh, generator=g).to(dtype)
    lens = [ln for grp in groups for ln in grp[:gmax]]
    rb = torch.tensor([(gi + 1) * S for gi, grp in enumerate(groups) for _ in grp[:gmax]], dtype=torch.int64)
    first = np.cumsum([0] + [len(grp[:gmax]) for grp in groups]).tolist()
    n = len(lens)
    gf = torch.tensor(first + [n] * (n + 1 - len(first)), dtype=torch.int32)
    q = torch.randn(n, H, Dh, generator=g).to(dtype)
    kl = torch.tensor(lens, dtype=torch.int32)
    print(f"[attn grouped] dtype={dtype} H={H} Hkv={Hkv} Dh={Dh} groups={first}", flush=True)
    Kb, Vb = _blocks(K, S).to(gpu), _blocks(V, S).to(gpu)
    args = (q.to(gpu), Kb, Vb, rb.to(gpu), kl.to(gpu))
    plain = ops.attn_decode(*args, kv_len_max=max(lens))
    grouped = ops.attn_decode(*args, kv_len_max=max(lens), group_first=gf.to(gpu))
    torch.cuda.synchronize()
    assert torch.equal(plain, grouped)
    ref = ok.attention_rows(_np(q), _np(K), _np(V), rb.numpy(), kl.numpy())
    assert rel_err(_np(grouped), ref) <= TOL[dtype]


def test_attn_decode_kv_len_device_data(gpu):
    """Lengths are read from device memory at launch time: changing them in place changes the result."""
    q, K, V, rb, kl = _attn_case(gpu, torch.bfloat16, 2, 16, 16, 128, [600, 600], S=2048)
    q, K, V, rb, kl = (t.to(gpu) for t in (q, K, V, rb, kl))
    a = ops.attn_decode(q, K, V, rb, kl, kv_len_max=2048).clone()
    kl.fill_(900)
    b = ops.attn_decode(q, K, V, rb, kl, kv_len_max=2048)
    ref = ok.attention_rows(_np(q), _np(K), _np(V), rb.cpu().numpy(), [900, 900])
    assert rel_err(_np(b), ref) <= 2e-2
    assert (a.float() - b.float()).abs().max().item() > 1e-3


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("n,N,K", [(1, 2048, 2048), (8, 6144, 2048), (17, 64, 5632), (40, 512, 4096),
                                   (300, 256, 1024), (3, 32000, 256), (16, 96, 6144), (5, 48, 8192)])
def test_linear_matches_oracle(gpu, dtype, n, N, K):
    if K % ops.linear_k_multiple(dtype):
        pytest.skip("K not a multiple of the kernel granularity")
    g = torch.Generator().manual_seed(n * 7 + N)
    x = torch.randn(n, K, generator=g).to(dtype)
    W = (0.02 * torch.randn(N, K, generator=g)).to(dtype)
    print(f"[linear] dtype={dtype} n={n} N={N} K={K}", flush=True)
    y = ops.linear(x.to(gpu), W.to(gpu))
    ref = ok.linear(_np(x), _np(W))
    assert rel_err(_np(y), ref) <= TOL[dtype]


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_linear_swiglu_fp32_out_and_row_gather(gpu, dtype):
    g = torch.Generator().manual_seed(11)
    n, F_, K = 9, 96, 512
    pool = torch.randn(20, K + 64, generator=g).to(dtype)
    rows = torch.tensor([3, 17, 0, 5, 5, 12, 19, 1, 8], dtype=torch.int32)
    W = (0.05 * torch.randn(2 * F_, K, generator=g)).to(dtype)
    y = ops.linear(pool.to(gpu), W.to(gpu), x_rows=rows.to(gpu), swiglu=True)
    xs = _np(pool)[rows.numpy(), :K]
    gu = ok.linear(xs, _np(W))
    ref = ok.swiglu(gu[:, :F_], gu[:, F_:])
    assert rel_err(_np(y), ref) <= TOL[dtype]
    if dtype == torch.bfloat16:
        y32 = ops.linear(pool.to(gpu), W.to(gpu), x_rows=rows.to(gpu), out_dtype=torch.float32)
        assert y32.dtype == torch.float32
        assert rel_err(_np(y32), gu) <= 1e-4 * 10  # fp32 out of bf16 inputs: only accumulation-order error


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("N", [384, 4096, 4112, 11280])
def test_linear_row_invariant(gpu, dtype, N):
    """Row m of y is bit-identical for every batch size and position in the
    batch, whichever kernel a row count selects. N = 24, 256, 257 and 705
    column tiles: at 300 rows, the LDS-pipelined stream kernel with 1 and 2
    tiles per workgroup, then weights shared through LDS 2 or 4 tiles per
    workgroup (2 at 33-64 rows for 257 tiles; both with a ragged tail);
    gathered rows at 3 and 40 rows; x
    read at a row pitch of K + 64 bytes (the engine's activation buffers)."""
    g = torch.Generator().manual_seed(5)
    K = 2048
    print(f"[linear row invariance] dtype={dtype} N={N}", flush=True)
    X = torch.randn(300, K, generator=g).to(dtype).to(gpu)
    W = (0.02 * torch.randn(N, K, generator=g)).to(dtype).to(gpu)
    full = ops.linear(X, W)
    assert rel_err(_np(full), ok.linear(_np(X), _np(W))) <= TOL[dtype]
    for n in (1, 5, 16, 17, 33, 64, 65, 300):
        part = ops.linear(X[:n].contiguous(), W)
        assert torch.equal(part, full[:n]), n
    pitched = torch.empty(300, K + 64 // X.element_size(), dtype=dtype, device=gpu)[:, :K]
    pitched.copy_(X)
    for n in (5, 64, 300):
        assert torch.equal(ops.linear(pitched, W, n=n), full[:n]), n
    rows = torch.tensor([299, 0, 150], dtype=torch.int32, device=gpu)
    gathered = ops.linear(X, W, x_rows=rows)
    assert torch.equal(gathered, full[rows.long()])
    rows = torch.randperm(300, generator=g)[:40].to(torch.int32).to(gpu)
    gathered = ops.linear(X, W, x_rows=rows)
    assert torch.equal(gathered, full[rows.long()])
    sw = torch.cat([W, W.flip(0)])
    a = ops.linear(X[:1].contiguous(), sw, swiglu=True)
    b = ops.linear(X, sw, swiglu=True)
    assert torch.equal(a[0], b[0])


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("N,K", [(2048, 2048), (2048, 5632), (2048, 4096), (256, 1024), (512, 384), (128, 128)])
def test_linear_split_k_same_bits(gpu, dtype, N, K):
    """Split-K projections: the slice sums of linear_partials, added in slice
    order in fp32 and rounded, equal the one-launch linear bit for bit (1 to 4
    slices: K = 128 .. 5632; 2 and 4 tiles per workgroup; row blocks with 1 to
    64 rows), over contiguous and gathered rows; the norm that
    reduces them (add_rmsnorm_split) equals linear + add_rmsnorm, including
    the kept linear rows (a_out), and matches the oracle."""
    if K % ops.linear_k_multiple(dtype):
        pytest.skip("K not a multiple of the kernel granularity")
    g = torch.Generator().manual_seed(N + K)
    print(f"[split-K] dtype={dtype} N={N} K={K}", flush=True)
    X = torch.randn(300, K, generator=g).to(dtype).to(gpu)
    Wm = (0.02 * torch.randn(N, K, generator=g)).to(dtype).to(gpu)
    W = ops.pack_linear(Wm)
    r = torch.randn(300, N, generator=g).to(dtype).to(gpu)
    w1 = (1 + 0.1 * torch.randn(N, generator=g)).to(dtype).to(gpu)
    w2 = (1 + 0.1 * torch.randn(N, generator=g)).to(dtype).to(gpu)
    part = torch.empty(4 * 300 * N, dtype=torch.float32, device=gpu)
    S = ops.linear_slices(K, dtype)
    P = K // ops.linear_k_multiple(dtype)
    assert S == -(-P // -(-P // 4))  # ceil(P / Q) slices of Q = ceil(P / 4) chunks
    norm_ok = N % ops.linear_k_multiple(dtype) == 0
    for n, rows in ((1, None), (17, None), (64, None), (113, None), (200, None), (300, None),
                    (40, torch.randperm(300, generator=g)[:40].to(torch.int32).to(gpu))):
        y = ops.linear(X, W, n=n, x_rows=rows)
        assert ops.linear_partials(X, W, part, n=n, x_rows=rows) == S
        sl = part[: S * n * N].view(S, n, N)
        acc = torch.zeros(n, N, dtype=torch.float32, device=gpu)
        for q in range(S):
            acc = acc + sl[q]
        assert torch.equal(acc.to(dtype), y), n
        if not norm_ok:
            continue
        keep = torch.empty(n, N, dtype=dtype, device=gpu)
        x1, h1 = ops.add_rmsnorm_split(part, S, n, w1, 1e-6, dtype=dtype, res=r, w2=w2, a_out=keep)
        x0, h0 = ops.add_rmsnorm(y, w1, 1e-6, res=r, w2=w2, n=n)
        assert torch.equal(keep, y) and torch.equal(x1, x0) and torch.equal(h1, h0), n
        h2 = ops.add_rmsnorm_split(part, S, n, w1, 1e-6, dtype=dtype)
        assert torch.equal(h2, ops.rmsnorm(y, w1, 1e-6, n=n)), n
    # the last case (gathered rows) against the oracle
    assert rel_err(_np(y), ok.linear(_np(X)[rows.long().cpu().numpy()], _np(Wm))) <= TOL[dtype]


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_swiglu_matches_reference(gpu, dtype):
    """silu(gate) * up of [gate | up] rows in fp32, rounded once: against an fp32
    torch reference on the same rounded inputs (bit-exact up to the last
    rounding: one ulp of the element type), with a strided, padded gu."""
    g = torch.Generator().manual_seed(2)
    n, F = 37, 5632 // 4
    gu = (3 * torch.randn(n, 2 * F + 64, generator=g)).to(dtype).to(gpu)[:, :2 * F]
    out = ops.swiglu(gu)
    gf, uf = gu[:, :F].float(), gu[:, F:].float()
    ref = (gf / (1 + torch.exp(-gf)) * uf).to(dtype)
    diff = (out.float() - ref.float()).abs()
    ulp = ref.float().abs() * (2 ** -7 if dtype == torch.bfloat16 else 2 ** -22) + 1e-30
    assert bool((diff <= ulp).all()), float((diff / ulp).max())
    # n rows of a larger buffer; the rows past n are untouched
    buf = torch.full((n + 3, F), 7.0, dtype=dtype, device=gpu)
    ops.swiglu(gu, n=n, out=buf)
    assert torch.equal(buf[:n], out) and bool((buf[n:] == 7).all())


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_add_rmsnorm(gpu, dtype):
    g = torch.Generator().manual_seed(3)
    n, D = 6, 2048
    a = torch.randn(n, D, generator=g).to(dtype)
    r = torch.randn(n, D, generator=g).to(dtype)
    w1 = (1 + 0.1 * torch.randn(D, generator=g)).to(dtype)
    w2 = (1 + 0.1 * torch.randn(D, generator=g)).to(dtype)
    x, h = ops.add_rmsnorm(a.to(gpu), w1.to(gpu), 1e-6, res=r.to(gpu), w2=w2.to(gpu))
    xr = ok.rmsnorm(_np(a) + _np(r), _np(w1), 1e-6)
    assert rel_err(_np(x), xr) <= TOL[dtype]
    hr = ok.rmsnorm(_np(x), _np(w2), 1e-6)  # second norm reads the stored x
    assert rel_err(_np(h), hr) <= TOL[dtype]
    # fused second norm == a separate rmsnorm call on x_out, bit for bit
    h2 = ops.rmsnorm(x, w2.to(gpu), 1e-6)
    assert torch.equal(h, h2)
    # row gather / scatter variants
    pool = torch.zeros(10, D, dtype=dtype, device=gpu)
    rows = torch.tensor([7, 2, 9, 0, 4, 5], dtype=torch.int32, device=gpu)
    ops.add_rmsnorm(a.to(gpu), w1.to(gpu), 1e-6, res=r.to(gpu), x_out=pool, out_rows=rows)
    assert torch.equal(pool[rows.long()], x)
    y = ops.rmsnorm(pool, w1.to(gpu), 1e-6, a_rows=rows)
    assert torch.equal(y, ops.rmsnorm(x, w1.to(gpu), 1e-6))


@pytest.mark.parametrize("dtype,D", [(torch.bfloat16, 512), (torch.bfloat16, 4096), (torch.float32, 256),
                                     (torch.float32, 1984)])
def test_add_rmsnorm_widths(gpu, dtype, D):
    """Widths with fewer than 16 chunks, several rounds of 16 chunks, and a
    ragged last round: against the oracle, and the fused second norm equals a
    separate call on the stored first result."""
    g = torch.Generator().manual_seed(D)
    n = 7
    a = torch.randn(n, D, generator=g).to(dtype).to(gpu)
    r = torch.randn(n, D, generator=g).to(dtype).to(gpu)
    w1 = (1 + 0.1 * torch.randn(D, generator=g)).to(dtype).to(gpu)
    w2 = (1 + 0.1 * torch.randn(D, generator=g)).to(dtype).to(gpu)
    x, h = ops.add_rmsnorm(a, w1, 1e-6, res=r, w2=w2)
    assert rel_err(_np(x), ok.rmsnorm(_np(a) + _np(r), _np(w1), 1e-6)) <= TOL[dtype]
    assert torch.equal(h, ops.rmsnorm(x, w2, 1e-6))
    # rows of different launches agree bit for bit
    assert torch.equal(ops.add_rmsnorm(a[3:4], w1, 1e-6, res=r[3:4]), x[3:4])


@pytest.mark.parametrize("blocks", [False, True])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("H,Hkv,Dh", [(16, 16, 128), (16, 4, 128), (4, 4, 64)])
def test_qkv_rope_append(gpu, dtype, H, Hkv, Dh, blocks):
    g = torch.Generator().manual_seed(H + Hkv)
    n, S = 5, 64
    qkv = torch.randn(n, (H + 2 * Hkv) * Dh, generator=g).to(dtype)
    pos = torch.tensor([0, 63, 7, 31, 1], dtype=torch.int32)
    flat = torch.tensor([5, 100, 64, 0, 127], dtype=torch.int64)
    cos, sin = ok.rope_tables(S, Dh)
    shape = (2, Hkv, 64, Dh) if blocks else (128, Hkv, Dh)  # 128 cache rows either way
    kc = torch.zeros(shape, dtype=dtype, device=gpu)
    vc = torch.zeros(shape, dtype=dtype, device=gpu)
    q = ops.qkv_rope_append(qkv.to(gpu), pos.to(gpu), torch.from_numpy(cos).to(gpu), torch.from_numpy(sin).to(gpu),
                            flat.to(gpu), kc, vc, H, Hkv, Dh)
    if blocks:
        kc, vc = _rows(kc), _rows(vc)
    x = _np(qkv)
    for i in range(n):
        p = int(pos[i])
        qi = x[i, :H * Dh].reshape(H, Dh)
        ki = x[i, H * Dh:(H + Hkv) * Dh].reshape(Hkv, Dh)
        vi = x[i, (H + Hkv) * Dh:].reshape(Hkv, Dh)
        assert rel_err(_np(q[i]), ok.rope(qi, p, cos, sin)) <= TOL[dtype]
        assert rel_err(_np(kc[int(flat[i])]), ok.rope(ki, p, cos, sin)) <= TOL[dtype]
        assert np.array_equal(_np(vc[int(flat[i])]), vi)  # V is copied bit for bit
    written = set(flat.tolist())
    untouched = [r for r in range(128) if r not in written]
    assert kc[untouched].abs().sum().item() == 0 and vc[untouched].abs().sum().item() == 0


@pytest.mark.parametrize("blocks", [False, True])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("H,Hkv,Dh,K", [(16, 16, 128, 2048), (16, 4, 128, 2048), (4, 4, 64, 256)])
@pytest.mark.parametrize("n", [1, 5, 16, 37])
def test_linear_qkv_rope_append_fused(gpu, dtype, H, Hkv, Dh, K, n, blocks):
    """The fused projection + RoPE + append equals linear() then
    qkv_rope_append() bit for bit, in both the wide (n <= 16) and tile regimes,
    with a gathered x, and touches no other cache row."""
    g = torch.Generator().manual_seed(n * 7 + Dh)
    S, rows = 96, 4 * 96
    N = (H + 2 * Hkv) * Dh
    X = torch.randn(n + 3, K, generator=g).to(dtype).to(gpu)
    Wq = (torch.randn(N, K, generator=g) * K ** -0.5).to(dtype).to(gpu)
    xr = torch.randperm(n + 3, generator=g)[:n].to(torch.int32).to(gpu)
    pos = torch.randint(0, S, (n,), generator=g, dtype=torch.int32).to(gpu)
    flat = (torch.randperm(rows, generator=g)[:n]).to(torch.int64).to(gpu)
    cos, sin = (torch.from_numpy(t).to(gpu) for t in ok.rope_tables(S, Dh))
    kc0 = torch.zeros((4, Hkv, S, Dh) if blocks else (rows, Hkv, Dh), dtype=dtype, device=gpu)
    vc0 = torch.zeros_like(kc0)
    qkv = ops.linear(X, Wq, x_rows=xr)
    q0 = ops.qkv_rope_append(qkv, pos, cos, sin, flat, kc0, vc0, H, Hkv, Dh)
    kc1 = torch.zeros_like(kc0)
    vc1 = torch.zeros_like(kc0)
    q1 = ops.linear_qkv_rope_append(X, Wq, pos, cos, sin, flat, kc1, vc1, H, Hkv, Dh, x_rows=xr)
    assert torch.equal(q0, q1)
    assert torch.equal(kc0, kc1) and torch.equal(vc0, vc1)
    if blocks:
        vc1 = _rows(vc1)
    # and against the oracle for one row
    i = n - 1
    ref = ok.linear(_np(X)[int(xr[i])][None], _np(Wq))[0]
    p = int(pos[i])
    assert rel_err(_np(q1[i]), ok.rope(ref[:H * Dh].reshape(H, Dh), p, cos.cpu().numpy(), sin.cpu().numpy())) \
        <= TOL[dtype]
    assert rel_err(_np(vc1[int(flat[i])]), ref[(H + Hkv) * Dh:].reshape(Hkv, Dh)) <= TOL[dtype]


def test_kv_append_exact_rows(gpu):
    """Writes land at exactly the requested flat rows, bit for bit (the analogue
    of experiments/exp5_graph/verify_graph.py gate 1c)."""
    kc = torch.zeros(2048, 16, 128, dtype=torch.bfloat16, device=gpu)
    vc = torch.zeros_like(kc)
    k = torch.randn(3, 16, 128, device=gpu).to(torch.bfloat16)
    v = torch.randn(3, 16, 128, device=gpu).to(torch.bfloat16)
    rows = torch.tensor([700, 701, 702], dtype=torch.int64, device=gpu)
    ops.kv_append(k, v, kc, vc, rows)
    nz = (kc.float().abs().sum(dim=(1, 2)) > 0).nonzero().flatten().tolist()
    assert nz == [700, 701, 702]
    assert torch.equal(kc[700:703], k) and torch.equal(vc[700:703], v)


def test_kv_append_blocks_match_rows(gpu):
    """The head-major block layout receives exactly the token-major rows:
    rows 700-702 of 512-row blocks land in block 1 at positions 188-190, every
    head, and nothing else changes."""
    kc = torch.zeros(4, 16, 512, 128, dtype=torch.bfloat16, device=gpu)
    vc = torch.zeros_like(kc)
    k = torch.randn(3, 16, 128, device=gpu).to(torch.bfloat16)
    v = torch.randn(3, 16, 128, device=gpu).to(torch.bfloat16)
    rows = torch.tensor([700, 701, 702], dtype=torch.int64, device=gpu)
    ops.kv_append(k, v, kc, vc, rows)
    assert torch.equal(kc[1, :, 188:191].transpose(0, 1), k) and torch.equal(vc[1, :, 188:191].transpose(0, 1), v)
    nz = (_rows(kc).float().abs().sum(dim=(1, 2)) > 0).nonzero().flatten().tolist()
    assert nz == [700, 701, 702]


def test_embed_copy_argmax(gpu):
    g = torch.Generator().manual_seed(9)
    table = torch.randn(100, 256, generator=g).to(torch.bfloat16).to(gpu)
    ids = torch.tensor([3, 99, 0, 3], dtype=torch.int64, device=gpu)
    e = ops.embed(ids, table, 1.0)
    assert torch.equal(e, table[ids])
    e2 = ops.embed(ids, table, 2.0)
    assert torch.equal(e2, (table[ids].float() * 2).to(torch.bfloat16))
    dst = torch.zeros(8, 300, dtype=torch.bfloat16, device=gpu)
    ops.copy_rows(table, dst, n=2, width=256, src_rows=torch.tensor([5, 6], dtype=torch.int32, device=gpu),
                  dst_rows=torch.tensor([7, 1], dtype=torch.int32, device=gpu))
    assert torch.equal(dst[7, :256], table[5]) and torch.equal(dst[1, :256], table[6])
    logits = torch.randn(7, 32000, generator=g).to(gpu)
    logits[2, 17] = 100.0
    logits[2, 30000] = 100.0  # tie: first index wins, as torch.argmax
    logits[4, 31000] = float("nan")  # NaN ranks above every number, as torch.argmax: first NaN wins
    logits[4, 20000] = float("nan")
    logits[4, 5] = float("inf")
    logits[5] = float("nan")  # an all-NaN row: id 0
    logits[6] = float("-inf")  # an all -inf row: id 0
    am = ops.argmax(logits)
    assert am.tolist() == logits.argmax(dim=-1).tolist()
    assert am[2].item() == 17 and am[4].item() == 20000 and am[5].item() == 0 and am[6].item() == 0


@pytest.mark.parametrize("dtype,D", [(torch.bfloat16, 2048), (torch.bfloat16, 256), (torch.float32, 256)])
def test_embed_rmsnorm_same_bits_as_three_launches(gpu, dtype, D):
    """The prelude's opening launch -- embed (ids and ring handles), the first
    norm, and the initial-loop-state copy into the wave-state rows -- equals
    embed + rmsnorm + copy_rows bit for bit."""
    g = torch.Generator().manual_seed(D)
    V, n = 300, 6
    table = torch.randn(V, D, generator=g).to(dtype).to(gpu)
    w = (1 + 0.1 * torch.randn(D, generator=g)).to(dtype).to(gpu)
    ring = torch.tensor([7, 250, 3], dtype=torch.int64, device=gpu)
    ids = torch.tensor([5, -2, 299, -1, 0, 7], dtype=torch.int64, device=gpu)  # -2, -1: ring handles
    s0 = torch.randn(40, D, generator=g).to(dtype).to(gpu)
    pos = torch.tensor([3, 9, 0, 39, 12, 5], dtype=torch.int32, device=gpu)
    rows = torch.tensor([4, 0, 9, 2, 7, 5], dtype=torch.int32, device=gpu)
    pad = 64 // table.element_size()
    for scale in (1.0, 45.25):
        print(f"[embed_rmsnorm] dtype={dtype} D={D} scale={scale}", flush=True)
        x0 = ops.embed(ids, table, scale, ring=ring)
        h0 = ops.rmsnorm(x0, w, 1e-6)
        pool0 = torch.zeros(10, 2 * D + pad, dtype=dtype, device=gpu)[:, :2 * D]
        ops.copy_rows(s0, pool0, n=n, width=D, src_rows=pos, dst_rows=rows)
        x1 = torch.empty(n, D, dtype=dtype, device=gpu)
        h1 = torch.empty(n, D + pad, dtype=dtype, device=gpu)[:, :D]
        pool1 = torch.zeros(10, 2 * D + pad, dtype=dtype, device=gpu)[:, :2 * D]
        ops.embed_rmsnorm(ids, table, scale, w, 1e-6, h_out=h1, x_out=x1, ring=ring, copy=(s0, pos, pool1, rows, D))
        assert torch.equal(x1, x0) and torch.equal(h1, h0) and torch.equal(pool1, pool0)
        h2 = torch.empty(n, D, dtype=dtype, device=gpu)
        ops.embed_rmsnorm(ids, table, scale, w, 1e-6, h_out=h2, ring=ring)  # no x_out, no copy
        assert torch.equal(h2, h0)


def test_token_ring_round_trip(gpu):
    """argmax drops ids into ring slots (padding rows aimed at a trash slot);
    embed takes a handle -(slot + 1) from the ring, and plain ids as before."""
    g = torch.Generator().manual_seed(10)
    logits = torch.randn(4, 500, generator=g).to(gpu)
    ring = torch.full((9,), -7, dtype=torch.int64, device=gpu)
    rows = torch.tensor([5, 0, 8, 2], dtype=torch.int32, device=gpu)  # 8 = trash slot
    out = ops.argmax(logits, ring=ring, ring_rows=rows)
    ref = logits.argmax(dim=-1)
    assert torch.equal(out, ref)
    assert ring[5].item() == ref[0].item() and ring[0].item() == ref[1].item() and ring[2].item() == ref[3].item()
    assert ring[1].item() == -7  # untouched
    table = torch.randn(500, 256, generator=g).to(torch.bfloat16).to(gpu)
    ids = torch.tensor([-6, 3, -1, -3], dtype=torch.int64, device=gpu)  # handles of slots 5, 0, 2
    e = ops.embed(ids, table, 1.0, ring=ring)
    want = torch.stack([ref[0], torch.tensor(3, device=gpu), ref[1], ref[3]])
    assert torch.equal(e, table[want])


@pytest.mark.parametrize("N,K", [(32000, 2048), (2048, 2048), (1024, 2048), (8192, 2048), (32000, 4096),
                                 (8192, 6144)])
def test_linear_argmax_groups_same_ids_and_bits(gpu, N, K):
    """lm_head with the column-group argmax: y has the bits of the plain
    linear, and the ids (with ring and accept flags) from the group bests equal
    wfd_argmax over y -- including ties across groups and within one group
    (first index wins), an all-zero row (every logit +0: id 0), NaN logits
    (the first NaN wins, as torch.argmax), and every form of the few-row
    launch: half-tile groups (N <= 4096), 8-wave and 16-wave full tiles
    (N 32000 / 8192), one to three chunks per sub-slice (K 2048 / 4096 / 6144)."""
    g = torch.Generator().manual_seed(N + K)
    W = (0.02 * torch.randn(N, K, generator=g)).to(torch.bfloat16)
    x = torch.randn(16, K, generator=g).to(torch.bfloat16)
    x[2] = 0
    big = 0.05 * x.float() / x.float().norm(dim=1, keepdim=True) * math.sqrt(K)
    j1, j2 = 16 * 3 + 5, N - 16 + 2          # different groups, row 0
    j3, j4 = 16 * 7 + 3, 16 * 7 + 9          # one group, row 1
    W[j1] = W[j2] = big[0].to(torch.bfloat16)
    W[j3] = W[j4] = big[1].to(torch.bfloat16)
    Wp = ops.pack_linear(W.to(gpu))
    xg = x.to(gpu)
    for n in (1, 3, 8, 16):
        G = ops.linear_argmax_groups(n, Wp)
        assert G == (N // 16 if N // 16 > 256 else N // 8)
        ref = ops.linear(xg, Wp, n=n, out_dtype=torch.float32)
        y, pv, pi = ops.linear_argmax(xg, Wp, n=n)
        assert torch.equal(y[:n].view(torch.int32), ref[:n].view(torch.int32))
        ids = ops.argmax_groups(pv, pi, G, n=n)
        want = ops.argmax(ref, n=n)
        assert ids.tolist() == want.tolist() == ref[:n].argmax(dim=-1).tolist()
        if n >= 3:
            assert ids[0].item() == j1 and ids[1].item() == j3 and ids[2].item() == 0
        # ring and greedy accept flags, as wfd_argmax leaves them
        expect = torch.tensor([want[0].item(), -2, (want[-1].item() + 1) % N] + [-(1 << 62)] * (n - 3),
                              dtype=torch.int64, device=gpu)[:n] if n >= 3 else want[:n].clone()
        ring_a = torch.full((9,), -7, dtype=torch.int64, device=gpu)
        ring_a[1] = want[min(1, n - 1)]
        ring_b = ring_a.clone()
        rows = torch.arange(n, dtype=torch.int32, device=gpu) + 2
        fa = torch.full((n,), -5, dtype=torch.int32, device=gpu)
        fb = fa.clone()
        ops.argmax(ref, n=n, ring=ring_a, ring_rows=rows, expect=expect, accept=fa)
        ops.argmax_groups(pv, pi, G, n=n, ring=ring_b, ring_rows=rows, expect=expect, accept=fb)
        assert fa.tolist() == fb.tolist() and torch.equal(ring_a, ring_b)
    # a NaN weight makes its column NaN in every row (x rows are nonzero or 0 * NaN);
    # two such columns in different groups: the first one wins everywhere
    Wn = W.clone()
    Wn[j3, 1] = float("nan")
    Wn[j1, 0] = float("nan")
    Wnp = ops.pack_linear(Wn.to(gpu))
    for n in (1, 8):
        ref = ops.linear(xg, Wnp, n=n, out_dtype=torch.float32)
        y, pv, pi = ops.linear_argmax(xg, Wnp, n=n)
        ids = ops.argmax_groups(pv, pi, ops.linear_argmax_groups(n, Wnp), n=n)
        assert ids.tolist() == ops.argmax(ref, n=n).tolist() == ref[:n].argmax(dim=-1).tolist() == [min(j1, j3)] * n
    with pytest.raises(Exception, match="no column groups"):
        ops.linear_argmax(torch.zeros(17, K, dtype=torch.bfloat16, device=gpu), Wp, n=17)


def test_argmax_accept_flags_into_mapped_host_memory(gpu):
    """The greedy verify flags stored straight into mapped, coherent pinned
    host memory (what the engine polls): the same flags as into a device
    tensor, each written over the -1 the host cleared it to."""
    from wavefront_decoding_amd import _lib

    tick = _lib.load_tick()
    g = torch.Generator().manual_seed(11)
    logits = torch.randn(6, 700, generator=g).to(gpu)
    ref = logits.argmax(dim=-1)
    ring = torch.full((9,), -7, dtype=torch.int64, device=gpu)
    ring[3] = ref[1]
    # expected tokens: a match, a ring handle that matches, a mismatch, "no comparison", a match, a mismatch
    expect = torch.tensor([ref[0].item(), -4, (ref[2].item() + 1) % 700, -(1 << 62), ref[4].item(),
                           (ref[5].item() + 3) % 700], dtype=torch.int64, device=gpu)
    dev_flags = torch.full((6,), -5, dtype=torch.int32, device=gpu)
    ops.argmax(logits, ring=ring, ring_rows=torch.full((6,), 8, dtype=torch.int32, device=gpu), expect=expect,
               accept=dev_flags)
    host, devp = tick.host_alloc(4 * 8)
    try:
        tick.clear_flags(host, 8)
        ops.argmax(logits, ring=ring, ring_rows=torch.full((6,), 8, dtype=torch.int32, device=gpu), expect=expect,
                   accept_mapped=(devp, 8))
        flags = tick.wait_flags(host, 6, 10.0)
        torch.cuda.synchronize()
        assert flags == [True, True, False, False, True, False]
        assert flags == [bool(v) for v in dev_flags.tolist()]
        assert tick.wait_flags(host, 8, 0.0) is None  # flags 6, 7: no row of this launch, still -1
    finally:
        torch.cuda.synchronize()
        tick.host_free(host)


def test_bad_arguments_raise(gpu):
    from wavefront_decoding_amd import _lib

    q = torch.zeros(1, 16, 96, dtype=torch.bfloat16, device=gpu)  # unsupported head_dim
    kc = torch.zeros(8, 16, 96, dtype=torch.bfloat16, device=gpu)
    rb = torch.zeros(1, dtype=torch.int64, device=gpu)
    kl = torch.ones(1, dtype=torch.int32, device=gpu)
    with pytest.raises(_lib.WfdError, match="unsupported"):
        ops.attn_decode(q, kc, kc, rb, kl, kv_len_max=8)
    with pytest.raises(_lib.WfdError):
        ops.linear(torch.zeros(2, 100, device=gpu), torch.zeros(16, 100, device=gpu))
    assert math.isfinite(1.0)


def test_linear_consecutive_shapes(gpu):
    """Back-to-back launches of different widths, depths and row counts (both
    kernel variants) each match the oracle."""
    g = torch.Generator().manual_seed(21)
    for N, K, n in [(2048, 2048, 1), (6144, 2048, 8), (512, 4096, 20), (32000, 256, 2), (2048, 5632, 3),
                    (11264, 2048, 100)]:
        x = torch.randn(n, K, generator=g).to(torch.bfloat16)
        W = (0.02 * torch.randn(N, K, generator=g)).to(torch.bfloat16)
        y = ops.linear(x.to(gpu), W.to(gpu))
        assert rel_err(_np(y), ok.linear(_np(x), _np(W))) <= 2e-2, (N, K, n)
