"""ctypes binding of libwfd.so (the C ABI declared in include/wfd.h).

torch is imported before the library is opened: libwfd.so links the HIP
runtime by soname (libamdhip64.so.7), and torch's bundled copy carries the
same soname, so loading torch first makes both share one runtime, one device
context and one set of streams.

There is no fallback: if the library is missing or cannot be opened, every
op raises. Build it with `python wavefront-decoding_amd/build.py`.
"""
from __future__ import annotations

import ctypes
import os

import torch  # noqa: F401  (must precede the CDLL load, see module docstring)

LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "libwfd.so")

F32, BF16 = 0, 1
EPI_PLAIN, EPI_SWIGLU = 0, 1
STATUS = {0: "ok", -1: "bad argument", -2: "unsupported", -3: "launch failure", -4: "workspace too small"}

_vp = ctypes.c_void_p
_i32 = ctypes.c_int
_i64 = ctypes.c_int64
_f32 = ctypes.c_float
_sz = ctypes.c_size_t

# name -> (restype, argtypes); the exported surface of include/wfd.h.
SIGNATURES: dict[str, tuple] = {
    "wfd_last_error": (ctypes.c_char_p, []),
    "wfd_abi_version": (_i32, []),
    "wfd_attn_workspace_bytes": (_sz, [_i32, _i32, _i32, _i32]),
    "wfd_attn_split_keys": (_i32, []),
    "wfd_attn_group_max_rows": (_i32, [_i32, _i32]),
    "wfd_attn_decode": (_i32, [_vp, _vp, _vp, _i64, _vp, _vp, _vp, _vp, _i32, _i32, _i32, _i32, _i32, _f32, _i32,
                               _vp, _sz, _vp]),
    "wfd_attn_decode_noalloc": (_i32, [_vp, _vp, _vp, _i64, _vp, _vp, _vp, _vp, _i32, _i32, _i32, _i32, _i32, _f32,
                                       _i32, _vp]),
    "wfd_attn_varlen_rows": (_i32, [_vp, _vp, _i32, _i32, _i32, _vp, _vp, _vp]),
    "wfd_attn_prefill": (_i32, [_vp, _vp, _vp, _i64, _vp, _vp, _vp, _vp, _i32, _i32, _i32, _i32, _i32, _i32, _f32,
                                _vp]),
    "wfd_kv_append": (_i32, [_vp, _vp, _vp, _vp, _i64, _vp, _i32, _i32, _i32, _i32, _vp]),
    "wfd_swiglu": (_i32, [_vp, _i64, _vp, _i64, _i32, _i32, _i32, _vp]),
    "wfd_qkv_rope_append": (_i32, [_vp, _i64, _vp, _vp, _vp, _i32, _vp, _vp, _vp, _vp, _i64, _i32, _i32, _i32,
                                   _i32, _i32, _vp]),
    "wfd_linear_k_multiple": (_i32, [_i32]),
    "wfd_linear_pack": (_i32, [_vp, _vp, _i32, _i32, _i32, _i32, _i32, _vp]),
    "wfd_linear": (_i32, [_vp, _vp, _i64, _vp, _vp, _i64, _i32, _i32, _i32, _i32, _i32, _i32, _i32, _vp, _vp]),
    "wfd_linear_prep": (_i32, [_vp, _vp, _i64, _vp, _i32, _i32, _i32, _i32, _vp, _vp]),
    "wfd_norm_prep": (_i32, [_vp, _i64, _vp, _i64, _i32, _vp, _i32, _f32, _vp, _vp, _vp, _vp, _i64, _i32, _i32, _i32,
                             _vp]),
    "wfd_linear_qkv_rope_append": (_i32, [_vp, _vp, _i64, _vp, _i32, _i32, _vp, _vp, _vp, _i32, _vp, _vp, _vp, _vp,
                                          _i64, _i32, _i32, _i32, _i32, _vp, _vp]),
    "wfd_add_rmsnorm": (_i32, [_vp, _vp, _i64, _vp, _i64, _vp, _vp, _vp, _vp, _i64, _vp, _i64, _i32, _i32, _f32,
                               _i32, _vp]),
    "wfd_linear_slices": (_i32, [_i32, _i32]),
    "wfd_linear_partials": (_i32, [_vp, _vp, _i64, _vp, _vp, _i32, _i32, _i32, _i32, _vp]),
    "wfd_add_rmsnorm_split": (_i32, [_vp, _i64, _i32, _vp, _i64, _vp, _i64, _vp, _vp, _vp, _vp, _i64, _vp, _i64,
                                     _i32, _i32, _f32, _i32, _vp]),
    "wfd_embed": (_i32, [_vp, _vp, _i64, _vp, _f32, _vp, _i64, _i32, _i32, _i32, _i32, _vp]),
    "wfd_embed_rmsnorm": (_i32, [_vp, _vp, _i64, _vp, _f32, _i32, _vp, _vp, _i64, _vp, _i64, _vp, _vp, _i64, _vp,
                                 _vp, _i64, _i32, _i32, _i32, _f32, _i32, _vp]),
    "wfd_copy_rows": (_i32, [_vp, _vp, _i64, _vp, _vp, _i64, _i32, _i32, _i32, _vp]),
    "wfd_argmax": (_i32, [_vp, _i64, _vp, _vp, _vp, _i64, _vp, _vp, _i32, _i32, _vp]),
    "wfd_linear_argmax_groups": (_i32, [_i32, _i32, _i32, _i32]),
    "wfd_linear_argmax": (_i32, [_vp, _vp, _i64, _vp, _vp, _i64, _i32, _i32, _i32, _i32, _vp, _vp, _vp, _vp]),
    "wfd_argmax_groups": (_i32, [_vp, _vp, _i32, _vp, _vp, _vp, _i64, _vp, _vp, _i32, _vp]),
}



class PrepArgs(ctypes.Structure):
    """wfd_prep_t (include/wfd.h): the residual stream and operand of a folded norm pair."""

    _fields_ = [("r_in", _vp), ("ld_in", _i64), ("s_in", _vp), ("w_in", _vp), ("r_out", _vp), ("ld_out", _i64),
                ("a_out", _vp), ("ld_a", _i64), ("wa", _vp), ("wb", _vp), ("part", _vp)]


class RowScaleArgs(ctypes.Structure):
    """wfd_rowscale_t (include/wfd.h): where a linear finds its rows' scales."""

    _fields_ = [("scale", _vp), ("part", _vp), ("D", _i32), ("two", _i32), ("eps", _f32), ("s_out", _vp)]


_LIB: ctypes.CDLL | None = None


class WfdError(RuntimeError):
    pass


def load() -> ctypes.CDLL:
    """Open libwfd.so once and bind every exported signature."""
    global _LIB
    if _LIB is not None:
        return _LIB
    if not os.path.exists(LIB_PATH):
        raise WfdError(
            f"libwfd.so not found at {LIB_PATH}; build it with `python wavefront-decoding_amd/build.py` "
            "(there is no non-HIP fallback)."
        )
    lib = ctypes.CDLL(LIB_PATH)
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    _LIB = lib
    return lib


def load_tick():
    """The _tick extension (csrc/tick.cpp: a decode tick's row tables, upload
    and graph launch). Imported after torch for the same reason as libwfd.so;
    raises if it is not built."""
    import importlib

    try:
        return importlib.import_module(__name__.rsplit(".", 1)[0] + "._tick")
    except ImportError as e:
        raise WfdError(f"the _tick extension is not built ({e}); build it with "
                       "`python wavefront-decoding_amd/build.py`") from e


def check(rc: int, what: str) -> None:
    if rc != 0:
        msg = load().wfd_last_error().decode(errors="replace")
        raise WfdError(f"{what} failed ({STATUS.get(rc, rc)}): {msg}")
