"""The reference's attention-backend API on this library's HIP kernels.

Same names, argument meanings, shapes and masking conventions as
src/decoding/fa4_attention.py (set_backend / backend :107-118, compute_qkv
:128-160, attn_dense :191-232, attn_cutoff_multi :240-291, attn_varlen
:301-317 with its FA varlen convention, attn_varlen_q1_padded :320-342), so a
caller written against that module can import this one instead. Every call
runs a HIP kernel of libwfd.so on torch's current stream:

  attn_dense      bf16 causal with Tq <= Tk (a prompt, bottom-right aligned):
                  the MFMA prefill kernel (wfd_attn_prefill), one segment per
                  batch row; otherwise the decode kernel (wfd_attn_decode)
                  with one (row base, key count) entry per query row
  attn_cutoff_multi  the decode kernel with key count = qpos + 1
  attn_varlen     the decode kernel over the packed K / V (token-major), its
                  row tables expanded from cu_q / cu_k on the device
                  (wfd_attn_varlen_rows), so nothing is read back to the host
  attn_varlen_q1_padded  attn_varlen with one query row per segment (the
                  reference pads each to two causal rows to steer FA2's tile
                  choice; the decode kernel has no such template switch, and
                  the kept row's result is the same full-segment attention)
  compute_qkv     the fused Wqkv projection (wfd_linear) and RoPE
                  (wfd_qkv_rope_append into a scratch buffer)

A query row with no keys (bottom-right causal with k_len < q_len) gets a
zero row, the flash-attention convention the reference's default backend
follows. Inputs are caller-owned; outputs are allocated by torch's caching
allocator (as in the reference). Errors raise WfdError (bad shapes, dtypes
other than float32 / bfloat16, head sizes other than 64 / 128).
"""
from __future__ import annotations

import math

import torch

from . import _lib, ops

_BACKEND = "hip"
# The reference's fused-kernel backends: a caller that selects either keeps
# running on this library's kernels.
_FUSED_ALIASES = ("torch", "fa4")


def set_backend(name: str) -> None:
    """'hip' (this library; the default). The reference's fused backends
    'torch' and 'fa4' name the same fast path and select it too. Its 'sdpa'
    backend (slow explicit-mask twins kept for parity tests) has no place in
    the product: parity references live in the test oracle."""
    global _BACKEND
    if name == "hip" or name in _FUSED_ALIASES:
        _BACKEND = "hip"
        return
    if name == "sdpa":
        raise ValueError("the 'sdpa' twins are test references, not a product backend (see oracle.kernels)")
    raise ValueError(f"unknown attention backend {name!r}")


def backend() -> str:
    return _BACKEND


_TABLES: dict[tuple, tuple[torch.Tensor, ...]] = {}


def _cached(key, build):
    t = _TABLES.get(key)
    if t is None:
        if len(_TABLES) > 256:
            _TABLES.clear()
        t = _TABLES[key] = build()
    return t


def _scale(Dh: int) -> float:
    return 1.0 / math.sqrt(Dh)


def _dense_rows(B: int, Tq: int, Tk: int, causal: bool, device) -> tuple[torch.Tensor, torch.Tensor]:
    def build():
        b = torch.arange(B, dtype=torch.int64).repeat_interleave(Tq)
        j = torch.arange(Tq, dtype=torch.int64).repeat(B)
        kv = (Tk - Tq + j + 1).clamp(min=0) if causal else torch.full_like(j, Tk)
        return (b * Tk).to(device), kv.to(torch.int32).to(device)

    return _cached(("dense", B, Tq, Tk, causal, str(device)), build)


def _prefill_segments(B: int, Tq: int, Tk: int, device):
    def build():
        rb = torch.arange(B, dtype=torch.int64) * Tk
        qs = (torch.arange(B + 1, dtype=torch.int32) * Tq)
        p0 = torch.full((B,), Tk - Tq, dtype=torch.int32)
        return rb.to(device), qs.to(device), p0.to(device)

    return _cached(("prefill", B, Tq, Tk, str(device)), build)


def attn_dense(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, *, causal: bool) -> torch.Tensor:
    """q (B, Tq, H, Dh), k / v (B, Tk, Hkv, Dh) -> (B, Tq, H, Dh). causal is
    bottom-right aligned (query i attends keys <= i + Tk - Tq); a lone query
    (Tq = 1) attends the whole prefix either way."""
    B, Tq, H, Dh = q.shape
    Bk, Tk, Hkv, Dk = k.shape
    if (Bk, Dk) != (B, Dh) or v.shape != k.shape:
        raise _lib.WfdError(f"attn_dense: q {tuple(q.shape)} / k {tuple(k.shape)} / v {tuple(v.shape)} do not match")
    qf = q.contiguous().view(B * Tq, H, Dh)
    kf = k.contiguous().view(B * Tk, Hkv, Dh)
    vf = v.contiguous().view(B * Tk, Hkv, Dh)
    if causal and Tq > 1 and Tq <= Tk and q.dtype == torch.bfloat16 and Dh in (64, 128):
        rb, qs, p0 = _prefill_segments(B, Tq, Tk, q.device)
        out = ops.attn_prefill(qf, kf, vf, rb, qs, p0, max_seg_len=Tq, scale=_scale(Dh))
    else:
        rb, kl = _dense_rows(B, Tq, Tk, causal and Tq > 1, q.device)
        out = ops.attn_decode(qf, kf, vf, rb, kl, kv_len_max=max(Tk, 1), scale=_scale(Dh))
    return out.view(B, Tq, H, Dh)


def attn_cutoff_multi(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, qpos) -> torch.Tensor:
    """Disjoint multi-query cutoff: q (1, nq, H, Dh), k / v (1, Tk, Hkv, Dh),
    qpos the queries' absolute positions (list or 1-D tensor); query j
    attends keys [0, qpos[j]]. Contract (as in the reference): Tk == max(qpos) + 1."""
    B, nq, H, Dh = q.shape
    Tk, Hkv = k.shape[1], k.shape[2]
    if B != 1 or k.shape[0] != 1 or v.shape != k.shape or k.shape[3] != Dh:
        raise _lib.WfdError("attn_cutoff_multi: q (1, nq, H, Dh), k / v (1, Tk, Hkv, Dh)")
    if isinstance(qpos, (list, tuple)):
        if Tk != max(qpos) + 1:
            raise AssertionError("attn_cutoff_multi expects K sliced to max(qpos)+1")
        kl = torch.tensor([p + 1 for p in qpos], dtype=torch.int32).to(q.device)
    else:
        kl = torch.as_tensor(qpos).to(device=q.device, dtype=torch.int32) + 1
    rb = torch.zeros(nq, dtype=torch.int64, device=q.device)
    out = ops.attn_decode(q.contiguous().view(nq, H, Dh), k.contiguous().view(Tk, Hkv, Dh),
                          v.contiguous().view(Tk, Hkv, Dh), rb, kl, kv_len_max=max(Tk, 1), scale=_scale(Dh))
    return out.view(1, nq, H, Dh)


def attn_varlen(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, cu_q: torch.Tensor, cu_k: torch.Tensor,
                max_q: int, max_k: int, causal: bool = False) -> torch.Tensor:
    """Packed varlen attention: q (total_q, H, Dh), k / v (total_k, Hkv, Dh),
    cu_q / cu_k int32 (n + 1,) segment offsets -> (total_q, H, Dh).
    causal=False: every row of a segment attends the whole segment;
    causal=True: bottom-right causal per segment -- row r of a
    (q_len, k_len) segment attends keys <= k_len - q_len + r."""
    total_q, H, Dh = q.shape
    if k.dim() != 3 or v.shape != k.shape or k.shape[2] != Dh:
        raise _lib.WfdError("attn_varlen: q (total_q, H, Dh), k / v (total_k, Hkv, Dh)")
    cq = cu_q.to(device=q.device, dtype=torch.int32).contiguous()
    ck = cu_k.to(device=q.device, dtype=torch.int32).contiguous()
    rb, kl = ops.attn_varlen_rows(cq, ck, total_q, causal=causal)
    return ops.attn_decode(q.contiguous(), k.contiguous(), v.contiguous(), rb, kl, kv_len_max=max(int(max_k), 1),
                           scale=_scale(Dh))


def attn_varlen_q1_padded(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, cu_k: torch.Tensor,
                          max_k: int) -> torch.Tensor:
    """n single-query segments: q (n, H, Dh), row i attends the whole segment
    [cu_k[i], cu_k[i+1]) -- the result of the reference's padded form."""
    n = q.shape[0]
    cu_q = _cached(("q1", n, str(q.device)), lambda: (torch.arange(n + 1, dtype=torch.int32).to(q.device),))[0]
    return attn_varlen(q, k, v, cu_q, cu_k, 1, max_k, causal=False)


def compute_qkv(attn, x: torch.Tensor, freqs, ve=None, config=None):
    """x (B, T, C) -> q (B, T, H, Dh), k / v (B, T, Hkv, Dh): the fused Wqkv
    projection then RoPE on q and k (interleaved pairs). `attn` carries
    Wqkv (a PackedWeight or an (N, C) weight), n_head, n_kv_head (or
    n_kv_heads) and head_dim; `freqs` is (cos, sin, positions): float32
    (S, Dh/2) tables and the T positions (int32 tensor, or a start position).
    The parcae-only extras (value embeddings, clipping, qk bias, qk norm) are
    absent from this model family: asking for one raises."""
    if ve is not None or (config is not None and any(getattr(config, f, None) for f in
                                                     ("clip_qkv", "qk_bias", "qk_norm"))):
        raise _lib.WfdError("compute_qkv: value embeddings / clip_qkv / qk_bias / qk_norm are not supported")
    B, T, C = x.shape
    H = attn.n_head
    Hkv = getattr(attn, "n_kv_head", None) or attn.n_kv_heads
    Dh = attn.head_dim
    cos, sin, positions = freqs
    if isinstance(positions, int):
        positions = torch.arange(positions, positions + T, dtype=torch.int32, device=x.device)
    pos = positions.to(device=x.device, dtype=torch.int32).reshape(-1)
    if pos.numel() != T:
        raise _lib.WfdError(f"compute_qkv: {pos.numel()} positions for T={T}")
    n = B * T
    qkv = ops.linear(x.contiguous().view(n, C), attn.Wqkv)
    kbuf = torch.empty(n, Hkv, Dh, dtype=x.dtype, device=x.device)
    vbuf = torch.empty_like(kbuf)
    rows = torch.arange(n, dtype=torch.int64, device=x.device)
    q = ops.qkv_rope_append(qkv, pos.repeat(B), cos, sin, rows, kbuf, vbuf, H, Hkv, Dh)
    return q.view(B, T, H, Dh), kbuf.view(B, T, Hkv, Dh), vbuf.view(B, T, Hkv, Dh)
