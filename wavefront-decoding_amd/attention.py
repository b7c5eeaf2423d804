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
  compute_qkv     the reference's c_q / c_k / c_v (packed together once) or
                  a fused Wqkv, with RoPE from its complex freqs_cis, in one
                  launch (wfd_linear_qkv_rope_append into fresh buffers)

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
        raise ValueError("set_backend('sdpa'): the reference's slow explicit-mask twins are a parity reference, "
                         "not a product backend, and this library runs only its HIP kernels; the explicit-mask "
                         "reference for parity checks is the test oracle (oracle.kernels.attention)")
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


def _fused_qkv_weight(attn):
    """The projection weight of `attn`: its fused Wqkv, or c_q / c_k / c_v
    (the reference's separate bias-free nn.Linear modules) concatenated and
    packed once; the packed copy is kept on the module and rebuilt when any
    of the three weights is replaced or changed in place."""
    W = getattr(attn, "Wqkv", None)
    if W is not None:
        return W
    if not all(hasattr(attn, m) for m in ("c_q", "c_k", "c_v")):
        raise _lib.WfdError("compute_qkv: attn needs c_q / c_k / c_v projections or a fused Wqkv weight")
    mods = (attn.c_q, attn.c_k, attn.c_v)
    if any(getattr(m, "bias", None) is not None for m in mods):
        raise _lib.WfdError("compute_qkv: projections with a bias are not supported (the reference's are bias-free)")
    key = tuple((m.weight.data_ptr(), m.weight._version) for m in mods)
    cached = attn.__dict__.get("_wfd_packed_qkv")
    if cached is None or cached[0] != key:
        fused = torch.cat([m.weight.detach() for m in mods]).contiguous()
        cached = (key, ops.pack_linear(fused))
        attn.__dict__["_wfd_packed_qkv"] = cached
    return cached[1]


def _rope_tables(freqs, B: int, T: int, Dh: int, device):
    """(cos, sin, per-row positions) for the QKV epilogue from the
    reference's complex freqs_cis (row t = position t's rotation, the same
    for every batch row) or from a (cos, sin, positions) tuple."""
    if torch.is_tensor(freqs) and freqs.is_complex():
        f = freqs.reshape(-1, Dh // 2)
        if f.shape[0] != T:
            raise _lib.WfdError(f"compute_qkv: freqs_cis holds {f.shape[0]} positions for T={T}")
        f = f.to(device)
        cos = f.real.to(torch.float32).contiguous()
        sin = f.imag.to(torch.float32).contiguous()
        pos = torch.arange(T, dtype=torch.int32, device=device)
    else:
        cos, sin, positions = freqs
        if isinstance(positions, int):
            positions = torch.arange(positions, positions + T, dtype=torch.int32, device=device)
        pos = positions.to(device=device, dtype=torch.int32).reshape(-1)
        if pos.numel() != T:
            raise _lib.WfdError(f"compute_qkv: {pos.numel()} positions for T={T}")
    return cos, sin, pos.repeat(B).contiguous()


def compute_qkv(attn, x: torch.Tensor, freqs, ve=None, config=None):
    """x (B, T, C) -> q (B, T, H, Dh), k / v (B, T, Hkv, Dh): the Q/K/V
    projections, then RoPE on q and k (src/decoding/fa4_attention.py:128-152),
    as one launch -- the fused projection with RoPE in its epilogue
    (wfd_linear_qkv_rope_append) -- or the projection alone when
    config.rope_settings.use_rope is False.

    attn: the reference's attention module (separate bias-free c_q / c_k /
    c_v projections, packed together once and kept on the module) or any
    object with a fused `Wqkv` ((H + 2 Hkv) Dh, C) weight or PackedWeight;
    plus n_head, n_kv_head (or n_kv_heads) and head_dim.
    freqs: the reference's freqs_cis -- complex, T x Dh/2 values (e.g. shaped
    (T, Dh/2) or (1, T, 1, Dh/2)), row t rotating position t of every batch
    row -- or (cos, sin, positions): float32 (S, Dh/2) tables and the T
    positions (int32 tensor, or a start position).
    RoPE rotates interleaved pairs: (x[2j], x[2j+1]) as the complex number
    x[2j] + i x[2j+1] times the rotation of pair j.
    The parcae-only extras the reference also handles (value embeddings,
    clip_qkv, qk_bias, qk_norm) are absent from this model family: asking
    for one raises."""
    if ve is not None or (config is not None and any(getattr(config, f, None) for f in
                                                     ("clip_qkv", "qk_bias", "qk_norm"))):
        raise _lib.WfdError("compute_qkv: value embeddings / clip_qkv / qk_bias / qk_norm are not supported")
    B, T, C = x.shape
    H = attn.n_head
    Hkv = getattr(attn, "n_kv_head", None) or attn.n_kv_heads
    Dh = attn.head_dim
    W = _fused_qkv_weight(attn)
    n = B * T
    xf = x.contiguous().view(n, C)
    rope = getattr(getattr(config, "rope_settings", None), "use_rope", True)
    if not rope:
        qkv = ops.linear(xf, W)
        q = qkv[:, : H * Dh].view(B, T, H, Dh)
        k = qkv[:, H * Dh: (H + Hkv) * Dh].view(B, T, Hkv, Dh)
        v = qkv[:, (H + Hkv) * Dh:].view(B, T, Hkv, Dh)
        return q, k, v
    cos, sin, pos = _rope_tables(freqs, B, T, Dh, x.device)
    kbuf = torch.empty(n, Hkv, Dh, dtype=x.dtype, device=x.device)
    vbuf = torch.empty_like(kbuf)
    rows = torch.arange(n, dtype=torch.int64, device=x.device)
    q = ops.linear_qkv_rope_append(xf, W, pos, cos, sin, rows, kbuf, vbuf, H, Hkv, Dh)
    return q.view(B, T, H, Dh), kbuf.view(B, T, Hkv, Dh), vbuf.view(B, T, Hkv, Dh)
