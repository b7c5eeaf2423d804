"""Host-side argument checks of the torch front end (CPU).

Every check below must fire before anything reaches libwfd.so: a buffer that
holds fewer rows than the launch touches would otherwise become an
out-of-bounds device access. The tensors live on the `meta` device (shapes
and strides only) and the CUDA-device check is patched out, so the checks are
exercised without a GPU and without calling the library.
"""
from __future__ import annotations

import pytest
import torch

from wavefront_decoding_amd import _lib, ops


@pytest.fixture(autouse=True)
def _meta_tensors_pass_the_device_check(monkeypatch):
    monkeypatch.setattr(ops, "_need_cuda", lambda *ts: None)

    def no_library():
        raise AssertionError("validation should have rejected the call before the library is loaded")

    monkeypatch.setattr(_lib, "load", no_library)


def _m(*shape, dtype=torch.bfloat16):
    return torch.empty(*shape, dtype=dtype, device="meta")


def _w(N, K, swiglu=False):
    return ops.PackedWeight(_m(N, K), N, K, swiglu)


def test_linear_rejects_short_x_and_out():
    with pytest.raises(_lib.WfdError, match="rows < n"):
        ops.linear(_m(4, 256), _w(32, 256), n=8, out=_m(8, 32))
    with pytest.raises(_lib.WfdError, match="bad out"):
        ops.linear(_m(8, 256), _w(32, 256), n=8, out=_m(4, 32))
    with pytest.raises(_lib.WfdError, match="x_rows"):
        ops.linear(_m(4, 256), _w(32, 256), n=8, x_rows=_m(4, dtype=torch.int32), out=_m(8, 32))


def test_linear_qkv_rope_append_rejects_short_x_and_q_out():
    H, Hkv, Dh = 2, 1, 128
    W = _w((H + 2 * Hkv) * Dh, 256)
    cos = _m(16, Dh // 2, dtype=torch.float32)
    kc = _m(64, Hkv, Dh)
    args = (W, _m(8, dtype=torch.int32), cos, cos, _m(8, dtype=torch.int64), kc, kc, H, Hkv, Dh)
    with pytest.raises(_lib.WfdError, match="rows < n"):
        ops.linear_qkv_rope_append(_m(4, 256), *args, n=8, q_out=_m(8, H, Dh))
    with pytest.raises(_lib.WfdError, match="q_out"):
        ops.linear_qkv_rope_append(_m(8, 256), *args, n=8, q_out=_m(4, H, Dh))


def test_add_rmsnorm_rejects_short_buffers():
    w = _m(256)
    with pytest.raises(_lib.WfdError, match="rows < n"):
        ops.add_rmsnorm(_m(4, 256), w, 1e-6, n=8, x_out=_m(8, 256))
    with pytest.raises(_lib.WfdError, match="x_out"):
        ops.add_rmsnorm(_m(8, 256), w, 1e-6, n=8, x_out=_m(4, 256))
    with pytest.raises(_lib.WfdError, match="h_out"):
        ops.add_rmsnorm(_m(8, 256), w, 1e-6, n=8, w2=w, x_out=_m(8, 256), h_out=_m(4, 256))
    with pytest.raises(_lib.WfdError, match="bad res"):
        ops.add_rmsnorm(_m(8, 256), w, 1e-6, n=8, res=_m(4, 256), x_out=_m(8, 256))
    # a row table on the output side: the table is trusted, the buffer's width is still checked
    with pytest.raises(_lib.WfdError, match="x_out"):
        ops.add_rmsnorm(_m(8, 256), w, 1e-6, n=8, x_out=_m(2, 128), out_rows=_m(8, dtype=torch.int32))


def test_embed_copy_rows_argmax_reject_short_buffers():
    with pytest.raises(_lib.WfdError, match="out"):
        ops.embed(_m(8, dtype=torch.int64), _m(100, 256), out=_m(4, 256))
    with pytest.raises(_lib.WfdError, match="src holds"):
        ops.copy_rows(_m(4, 256), _m(8, 256), n=8, width=256)
    with pytest.raises(_lib.WfdError, match="dst holds"):
        ops.copy_rows(_m(8, 256), _m(4, 256), n=8, width=256)
    with pytest.raises(_lib.WfdError, match="at least `width`"):
        ops.copy_rows(_m(8, 128), _m(8, 256), n=8, width=256)
    with pytest.raises(_lib.WfdError, match="outside the"):
        ops.argmax(_m(4, 100, dtype=torch.float32), n=8)
    with pytest.raises(_lib.WfdError, match="out: int64"):
        ops.argmax(_m(8, 100, dtype=torch.float32), n=8, out=_m(4, dtype=torch.int64))


def test_linear_partials_rejects_short_x_and_part(monkeypatch):
    monkeypatch.setattr(ops, "linear_slices", lambda K, dtype: 4)
    W = _w(256, 512)
    part = _m(4 * 8 * 256, dtype=torch.float32)
    with pytest.raises(_lib.WfdError, match="rows < n"):
        ops.linear_partials(_m(4, 512), W, part, n=8)
    with pytest.raises(_lib.WfdError, match="part"):
        ops.linear_partials(_m(8, 512), W, _m(4 * 8 * 256 - 1, dtype=torch.float32), n=8)
    with pytest.raises(_lib.WfdError, match="part"):
        ops.linear_partials(_m(8, 512), W, _m(4 * 8 * 256), n=8)  # bf16, not fp32
    with pytest.raises(_lib.WfdError, match="x_rows"):
        ops.linear_partials(_m(8, 512), W, part, n=8, x_rows=_m(4, dtype=torch.int32))


def test_add_rmsnorm_split_rejects_short_buffers():
    D, n = 256, 8
    w = _m(D)
    part = _m(4 * n * D, dtype=torch.float32)
    kw = dict(dtype=torch.bfloat16)
    with pytest.raises(_lib.WfdError, match="part"):
        ops.add_rmsnorm_split(_m(4 * n * D - 1, dtype=torch.float32), 4, n, w, 1e-6, **kw)
    with pytest.raises(_lib.WfdError, match="nslices"):
        ops.add_rmsnorm_split(part, 5, n, w, 1e-6, **kw)
    with pytest.raises(_lib.WfdError, match="bad res"):
        ops.add_rmsnorm_split(part, 4, n, w, 1e-6, res=_m(n - 1, D), **kw)
    with pytest.raises(_lib.WfdError, match="bad a_out"):
        ops.add_rmsnorm_split(part, 4, n, w, 1e-6, a_out=_m(n - 1, D), **kw)
    with pytest.raises(_lib.WfdError, match="x_out"):
        ops.add_rmsnorm_split(part, 4, n, w, 1e-6, x_out=_m(n - 1, D), **kw)
    with pytest.raises(_lib.WfdError, match="h_out"):
        ops.add_rmsnorm_split(part, 4, n, w, 1e-6, w2=w, x_out=_m(n, D), h_out=_m(n - 1, D), **kw)

