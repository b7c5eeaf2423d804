"""Host behaviour of the attention-backend API (CPU): backend selection and
argument errors that are raised before anything is launched."""
from __future__ import annotations

import pytest
import torch

from wavefront_decoding_amd import _lib
from wavefront_decoding_amd import attention as A


def test_backend_names():
    assert A.backend() == "hip"
    for name in ("torch", "fa4", "hip"):  # the reference's fused backends map to the HIP kernels
        A.set_backend(name)
        assert A.backend() == "hip"
    with pytest.raises(ValueError, match="parity reference"):
        A.set_backend("sdpa")
    with pytest.raises(ValueError, match="unknown"):
        A.set_backend("triton")
    assert A.backend() == "hip"


def test_reference_entry_points_exist():
    for name in ("attn_dense", "attn_cutoff_multi", "attn_varlen", "attn_varlen_q1_padded", "set_backend",
                 "backend", "compute_qkv"):
        assert callable(getattr(A, name)), name


def test_shape_errors_before_launch():
    q = torch.empty(1, 3, 4, 64, device="meta")
    with pytest.raises(_lib.WfdError):
        A.attn_dense(q, torch.empty(2, 5, 4, 64, device="meta"), torch.empty(2, 5, 4, 64, device="meta"), causal=True)
    with pytest.raises(AssertionError, match="max\\(qpos\\)\\+1"):
        A.attn_cutoff_multi(q, torch.empty(1, 9, 4, 64, device="meta"), torch.empty(1, 9, 4, 64, device="meta"),
                            [2, 3, 5])
    with pytest.raises(_lib.WfdError, match="not supported"):
        A.compute_qkv(object(), torch.empty(1, 2, 8, device="meta"), (None, None, 0), ve=torch.empty(1))
