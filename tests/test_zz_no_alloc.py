"""wfd_attn_decode_noalloc (static scratch, no workspace argument) against
wfd_attn_decode (caller's workspace), both called through the C ABI (GPU).

Two calls in a row on the same device, the second with a smaller input, must
each give the workspace path's output bit for bit (the same kernels; the
static scratch keeps the first call's partials, which the second must not
read). A launch that would need more scratch than the stated maximum is
rejected on the host before any launch. The first call of the process --
the one that resolves the scratch's device address -- may be made while a
graph is being captured.
"""
from __future__ import annotations

import ctypes
import math

import pytest
import torch

from wavefront_decoding_amd import _lib, ops

pytestmark = pytest.mark.gpu

MAX_BYTES = 32 << 20  # WFD_ATTN_NOALLOC_MAX_BYTES


def _case(dev, n, H, Hkv, Dh, lens, seed):
    g = torch.Generator(device=dev).manual_seed(seed)
    S = max(lens) + 2
    K = torch.randn(n + 1, Hkv, S, Dh, generator=g, device=dev).to(torch.bfloat16)
    V = torch.randn(n + 1, Hkv, S, Dh, generator=g, device=dev).to(torch.bfloat16)
    q = torch.randn(n, H, Dh, generator=g, device=dev).to(torch.bfloat16)
    rb = torch.tensor([(i + 1) * S for i in range(n)], dtype=torch.int64, device=dev)
    kl = torch.tensor(lens, dtype=torch.int32, device=dev)
    return q, K, V, rb, kl, S


def _call(lib, fn, q, K, V, rb, kl, S, out, ws=None, kv_max=None):
    n, H, Dh = q.shape
    Hkv = K.shape[1]
    stream = torch.cuda.current_stream().cuda_stream
    kv_max = int(kl.max().item()) if kv_max is None else kv_max
    args = [q.data_ptr(), K.data_ptr(), V.data_ptr(), S, rb.data_ptr(), kl.data_ptr(), None, out.data_ptr(), n, H,
            Hkv, Dh, _lib.BF16, 1.0 / math.sqrt(Dh), kv_max]
    if ws is not None:
        args += [ws.data_ptr(), ws.numel()]
    rc = getattr(lib, fn)(*args, stream)
    _lib.check(rc, fn)


def test_noalloc_first_call_under_graph_capture(gpu):
    """Collected first in this file, so its captured call is the process's
    first call of the entry point (no other test file makes one): the scratch
    address is resolved inside torch's graph capture. Three replays, with
    eager calls of both entry points on other inputs between them (which
    overwrite the scratch), each give the workspace path's bits."""
    lib = _lib.load()
    lens = [3000, 1, 1024, 1025, 4100, 64, 2047, 9]
    q, K, V, rb, kl, S = _case(gpu, 8, 16, 16, 128, lens, 3)
    ws = torch.zeros(ops.attn_workspace_bytes(8, 16, 128, S), dtype=torch.uint8, device=gpu)
    ref = torch.empty_like(q)
    _call(lib, "wfd_attn_decode", q, K, V, rb, kl, S, ref, ws)
    q2, K2, V2, rb2, kl2, S2 = _case(gpu, 3, 16, 16, 128, [5000, 700, 1], 4)
    ws2 = torch.zeros(ops.attn_workspace_bytes(3, 16, 128, S2), dtype=torch.uint8, device=gpu)
    ref2 = torch.empty_like(q2)
    _call(lib, "wfd_attn_decode", q2, K2, V2, rb2, kl2, S2, ref2, ws2)
    got = torch.full_like(q, float("nan"))
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    print("[noalloc] first call inside graph capture (n=8, kv_max=4100)", flush=True)
    with torch.cuda.graph(graph):
        _call(lib, "wfd_attn_decode_noalloc", q, K, V, rb, kl, S, got, kv_max=max(lens))
    for r in range(3):
        got.fill_(float("nan"))
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(got, ref), r
        other = torch.full_like(q2, float("nan"))
        _call(lib, "wfd_attn_decode_noalloc", q2, K2, V2, rb2, kl2, S2, other)
        _call(lib, "wfd_attn_decode", q2, K2, V2, rb2, kl2, S2, torch.empty_like(q2), ws2)
        torch.cuda.synchronize()
        assert torch.equal(other, ref2), r


@pytest.mark.parametrize("H,Hkv", [(16, 16), (16, 4)])
def test_noalloc_matches_workspace_path_twice(gpu, H, Hkv):
    lib = _lib.load()
    cases = [(24, [3000, 1, 1024, 1025, 4100, 64] * 4, 1), (5, [700, 20, 2100, 1, 333], 2)]  # second call smaller
    for n, lens, seed in cases:
        q, K, V, rb, kl, S = _case(gpu, n, H, Hkv, 128, lens[:n], seed)
        print(f"[noalloc] n={n} H={H} Hkv={Hkv} kv_max={max(lens[:n])}", flush=True)
        ws = torch.zeros(ops.attn_workspace_bytes(n, H, 128, S), dtype=torch.uint8, device=gpu)
        ref = torch.empty_like(q)
        _call(lib, "wfd_attn_decode", q, K, V, rb, kl, S, ref, ws)
        got = torch.full_like(q, float("nan"))
        _call(lib, "wfd_attn_decode_noalloc", q, K, V, rb, kl, S, got)
        torch.cuda.synchronize()
        assert torch.equal(got, ref)


def test_noalloc_rejects_launches_beyond_its_scratch(gpu):
    lib = _lib.load()
    # 64 rows x 16 heads x 130 splits x (128 + 2) floats > 32 MiB; rejected before anything launches
    need = ops.attn_workspace_bytes(64, 16, 128, 130 * 1024)
    assert need > MAX_BYTES
    rc = lib.wfd_attn_decode_noalloc(None, None, None, 0, None, None, None, None, 64, 16, 16, 128, _lib.BF16,
                                     0.1, 130 * 1024, None)
    assert rc == -4 and b"static scratch" in lib.wfd_last_error()
    assert ctypes.sizeof(ctypes.c_void_p) == 8
