"""wfd_attn_decode_noalloc (static scratch, no workspace argument) against
wfd_attn_decode (caller's workspace), both called through the C ABI (GPU).

Two calls in a row on the same device, the second with a smaller input, must
each give the workspace path's output bit for bit (the same kernels; the
static scratch keeps the first call's partials, which the second must not
read). A launch that would need more scratch than the stated maximum is
rejected on the host before any launch.
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


def _call(lib, fn, q, K, V, rb, kl, S, out, ws=None):
    n, H, Dh = q.shape
    Hkv = K.shape[1]
    stream = torch.cuda.current_stream().cuda_stream
    args = [q.data_ptr(), K.data_ptr(), V.data_ptr(), S, rb.data_ptr(), kl.data_ptr(), None, out.data_ptr(), n, H,
            Hkv, Dh, _lib.BF16, 1.0 / math.sqrt(Dh), int(kl.max().item())]
    if ws is not None:
        args += [ws.data_ptr(), ws.numel()]
    rc = getattr(lib, fn)(*args, stream)
    _lib.check(rc, fn)


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
