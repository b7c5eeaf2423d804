"""The C-ABI library loads on a host without a GPU and exports exactly what include/wfd.h declares (CPU)."""
from __future__ import annotations

import ctypes
import os
import re
import subprocess

import pytest
import torch

from wavefront_decoding_amd import _lib, ops

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _declared() -> set[str]:
    text = open(os.path.join(REPO, "include", "wfd.h")).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return set(re.findall(r"\b(wfd_[a-z0-9_]+)\s*\(", text))


def test_header_and_binding_agree():
    assert _declared() == set(_lib.SIGNATURES), _declared() ^ set(_lib.SIGNATURES)


def test_library_loads_and_exports_every_symbol():
    lib = _lib.load()
    for name in _declared():
        assert hasattr(lib, name), name
    out = subprocess.run(["nm", "-D", "--defined-only", _lib.LIB_PATH], capture_output=True, text=True).stdout
    exported = set(re.findall(r"\bT (wfd_[a-z0-9_]+)$", out, flags=re.M))
    assert exported == _declared(), exported ^ _declared()


def test_host_only_entry_points():
    lib = _lib.load()
    assert lib.wfd_abi_version() == 7
    # column groups of the tile argmax: 2000 tiles at <= 16 rows (lm_head), half tiles below 256 tiles,
    # none at 17 rows, for fp32 or for a K the few-row kernel does not take
    assert lib.wfd_linear_argmax_groups(8, 32000, 2048, _lib.BF16) == 2000
    assert lib.wfd_linear_argmax_groups(16, 2048, 2048, _lib.BF16) == 256
    assert lib.wfd_linear_argmax_groups(17, 32000, 2048, _lib.BF16) == 0
    assert lib.wfd_linear_argmax_groups(8, 32000, 2048, _lib.F32) == 0
    assert lib.wfd_linear_argmax_groups(8, 32000, 128 * 49, _lib.BF16) == 0
    rc = lib.wfd_linear_argmax(None, None, 2048, None, None, 32000, 17, 32000, 2048, 1, None, None, None, None)
    assert rc == -2 and b"no column groups" in lib.wfd_last_error()
    rc = lib.wfd_linear_argmax(None, None, 2048, None, None, 32000, 8, 32000, 2048, 1, None, None, None, None)
    assert rc == -1 and b"null pointer" in lib.wfd_last_error()
    # folded norm pairs: the prep epilogue has a few-row form only; the row form checks its shape first
    pp = _lib.PrepArgs()
    rc = lib.wfd_linear_prep(None, None, 2048, None, 17, 2048, 2048, 1, ctypes.addressof(pp), None)
    assert rc == -1 and b"null pointer" in lib.wfd_last_error()
    assert lib.wfd_norm_prep(None, 0, None, 0, 0, ctypes.addressof(pp), 1, 1e-6, None, None, None, None, 0, 1, 4096,
                             1, None) == -1  # D beyond the folded form's 2048
    assert b"at most 2048" in lib.wfd_last_error()
    assert lib.wfd_norm_prep(None, 0, None, 0, 0, ctypes.addressof(pp), 1, 1e-6, None, None, None, None, 0, 0, 2048,
                             1, None) == 0   # no rows: nothing to do
    assert ctypes.sizeof(_lib.RowScaleArgs) == 40 and ctypes.sizeof(_lib.PrepArgs) == 88
    assert lib.wfd_argmax_groups(None, None, 0, None, None, None, 0, None, None, 1, None) == -1
    assert lib.wfd_argmax_groups(None, None, 2000, None, None, None, 0, None, None, 0, None) == 0
    assert lib.wfd_argmax_groups(None, None, 2000, None, None, None, 0, None, None, 1, None) == -1
    assert lib.wfd_swiglu(None, 16, None, 8, 1, 12, 1, None) == -1  # F not a multiple of 8 (bf16)
    assert lib.wfd_swiglu(None, 16, None, 8, 0, 8, 1, None) == 0
    assert [lib.wfd_attn_group_max_rows(16, k) for k in (16, 8, 4, 3)] == [8, 4, 2, 0]
    assert lib.wfd_attn_split_keys() == 1024
    assert lib.wfd_linear_k_multiple(_lib.BF16) == 128 and lib.wfd_linear_k_multiple(_lib.F32) == 64
    # workspace: n*H*splits*(Dh + 2) floats, each array 256-byte aligned
    assert lib.wfd_attn_workspace_bytes(8, 16, 64, 1024) == 8 * 16 * 1 * 64 * 4 + 8 * 16 * 1 * 2 * 4
    # argument validation happens before any device work
    rc = lib.wfd_attn_decode(None, None, None, 0, None, None, None, None, 1, 16, 3, 64, 1, 0.1, 10, None, 0, None)
    assert rc == -1 and b"bad shape" in lib.wfd_last_error()
    # head-major blocks: a query's keys must fit one block
    rc = lib.wfd_attn_decode(None, None, None, 512, None, None, None, None, 1, 16, 16, 64, 1, 0.1, 513, None, 0, None)
    assert rc == -1 and b"kv_block_rows=512" in lib.wfd_last_error()
    assert lib.wfd_kv_append(None, None, None, None, -1, None, 1, 16, 128, 1, None) == -1
    rc = lib.wfd_attn_prefill(None, None, None, 0, None, None, None, None, 1, 10, 16, 3, 64, 1, 0.1, None)
    assert rc == -1 and b"wfd_attn_prefill: bad shape" in lib.wfd_last_error()
    assert lib.wfd_attn_prefill(None, None, None, 0, None, None, None, None, 0, 10, 16, 4, 64, 1, 0.1, None) == 0
    rc = lib.wfd_linear(None, None, 100, None, None, 16, 2, 16, 100, 1, 1, 0, 0, None, None)
    assert rc == -1
    # packing: shape and aliasing are checked on the host
    assert lib.wfd_linear_pack(8, 16, 24, 128, 1, 0, 0, None) == -1      # N not a multiple of 16
    assert lib.wfd_linear_pack(8, 8, 32, 128, 1, 0, 0, None) == -1       # W_packed aliases W
    assert lib.wfd_linear_pack(8, 16, 32, 128, 1, 1, 12, None) == -1     # swiglu pair_off mismatch


@pytest.mark.skipif(torch.cuda.device_count() > 0, reason="made-up device addresses: run only where no GPU is "
                    "visible, so a regressed check cannot launch a kernel on them")
def test_alignment_and_grid_checks_reject_before_launch():
    """Checks whose outcome depends on a pointer's value (16-byte alignment)
    or on the grid bound. The addresses are made up (4096, 8192): rejection
    happens on the host, before any launch."""
    lib = _lib.load()
    # 16-byte loads of x rows and packed weights: pointers and the x pitch are checked
    rc = lib.wfd_linear(4096 + 8, None, 128, 8192, 8192, 16, 2, 16, 128, 1, 1, 0, 0, None, None)
    assert rc == -1 and b"16-byte aligned" in lib.wfd_last_error()
    rc = lib.wfd_linear(4096, None, 132, 8192, 8192, 16, 2, 16, 128, 1, 1, 0, 0, None, None)
    assert rc == -1 and b"16-byte aligned" in lib.wfd_last_error()
    rc = lib.wfd_linear_qkv_rope_append(4096, None, 132, 8192, 2, 128, 16, 16, 16, 8, 16, 16, 16, 16, 0, 1, 1, 16, 1,
                                        None, None)
    assert rc == -1 and b"16-byte aligned" in lib.wfd_last_error()
    assert lib.wfd_attn_decode(None, None, None, 0, None, None, None, None, 0, 16, 16, 64, 1, 0.1, 10, None, 0, None) == 0
    rc = lib.wfd_attn_decode(4096, 4096 + 4, 4096, 0, 16, 16, None, 4096, 1, 16, 16, 64, 1, 0.1, 10, 4096, 1 << 20, None)
    assert rc == -1 and b"16-byte aligned" in lib.wfd_last_error()
    rc = lib.wfd_attn_prefill(4096, 4096, 4096, 0, 16, 16, 16, 4096 + 2, 1, 10, 16, 16, 64, 1, 0.1, None)
    assert rc == -1 and b"16-byte aligned" in lib.wfd_last_error()
    # row pitches below the row width of the folded norm pairs' rows
    pp_short = _lib.PrepArgs(None, 0, None, None, None, 0, 4096, 1024, None, 8192, 12288)  # ld_a 1024 < N 2048
    rc = lib.wfd_linear_prep(4096, None, 2048, 8192, 8, 2048, 2048, 1, ctypes.addressof(pp_short), None)
    assert rc == -1 and b"row pitch" in lib.wfd_last_error()
    pp_norm = _lib.PrepArgs(None, 0, None, None, None, 0, 4096, 2048, None, 8192, None)
    rc = lib.wfd_norm_prep(4096, 1024, None, 0, 0, ctypes.addressof(pp_norm), 0, 1e-6, 4096, None, None, None, 0, 4,
                           2048, 1, None)  # lda 1024 < D 2048
    assert rc == -1 and b"row pitch" in lib.wfd_last_error()
    # one grid row per 128-query tile: at most 65535 of them
    rc = lib.wfd_attn_prefill(4096, 4096, 4096, 0, 16, 16, 16, 4096, 1, 65535 * 128 + 1, 16, 16, 64, 1, 0.1, None)
    assert rc < 0 and b"beyond the grid" in lib.wfd_last_error()


def test_engine_rejects_rows_wider_than_the_folded_norms_take():
    """The decode step folds each RMSNorm pair into the linears, one wave per
    row: d_model up to 16 K chunks (2048 bf16, 1024 fp32). A wider model is
    refused when the engine is built, before anything is allocated."""
    import dataclasses

    from wavefront_decoding_amd import model as M
    from wavefront_decoding_amd.engine import LoopedModel

    assert ops.fold_max_d(torch.bfloat16) == 2048 and ops.fold_max_d(torch.float32) == 1024
    wide = dataclasses.replace(M.CONFIGS["looped-2048"], d_model=4096)
    with pytest.raises(ValueError, match="folded norm pairs"):
        LoopedModel(wide, {}, "cpu", max_seq_len=16)
