"""Torch-tensor front end of the C ABI (include/wfd.h).

Every function validates shapes/dtypes/devices on the host, then launches the
HIP kernel on torch's current stream through libwfd.so. Nothing here computes
on the host and nothing falls back to torch math: a missing library raises.
Outputs may be passed in (`out=`) so a caller can keep every buffer at a fixed
address for hipGraph capture; otherwise they are allocated with torch.

What the host checks: dtypes, devices, widths, contiguity, and that every
buffer addressed by plain row number (no row table) holds at least the rows
the launch touches. Row tables (x_rows, a_rows, out_rows, src_rows, ...) are
device data and are trusted, as the C ABI states: their entries are not read
back, so the caller guarantees they index inside the buffers passed.
"""
from __future__ import annotations

import ctypes
import math

import torch

from . import _lib

_DT = {torch.float32: _lib.F32, torch.bfloat16: _lib.BF16}


def _dt(t: torch.Tensor) -> int:
    try:
        return _DT[t.dtype]
    except KeyError:
        raise _lib.WfdError(f"unsupported dtype {t.dtype} (float32 / bfloat16)") from None


def _p(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()


def _stream() -> int:
    return torch.cuda.current_stream().cuda_stream


def _need_cuda(*ts: torch.Tensor | None) -> None:
    for t in ts:
        if t is not None and not t.is_cuda:
            raise _lib.WfdError("wfd ops need GPU tensors (no host fallback)")


def _need(cond: bool, msg: str) -> None:
    if not cond:
        raise _lib.WfdError(msg)


def _rows(t: torch.Tensor | None, n: int, name: str) -> None:
    if t is not None:
        _need(t.dtype == torch.int32 and t.is_contiguous() and t.numel() >= n, f"{name}: int32 contiguous (>= {n})")


# group-sum pairs per row of a few-row producer (wfd_prep_t.part)
FOLD_SLOTS = 256


class RowScale:
    """Where a linear finds its rows' folded-norm scales (wfd_rowscale_t):
    `scale` (n,) float32 precomputed by norm_prep, or `part` -- the group sums
    linear_prep left, FOLD_SLOTS float pairs per row, few-row launches only --
    with the pair's form (`two`: norm a present) and eps; with `part`,
    `s_out` (n,) float32 receives s_a."""

    __slots__ = ("scale", "part", "D", "two", "eps", "s_out")

    def __init__(self, *, D: int, eps: float, two: bool, scale: torch.Tensor | None = None,
                 part: torch.Tensor | None = None, s_out: torch.Tensor | None = None):
        _need((scale is None) != (part is None), "RowScale: exactly one of scale / part")
        self.scale, self.part, self.D, self.two, self.eps, self.s_out = scale, part, D, two, eps, s_out

    def check(self, n: int) -> None:
        _need_cuda(self.scale, self.part, self.s_out)
        for name, t, size in (("scale", self.scale, n), ("part", self.part, n * FOLD_SLOTS * 2),
                              ("s_out", self.s_out, n)):
            if t is not None:
                _need(t.dtype == torch.float32 and t.is_contiguous() and t.numel() >= size,
                      f"RowScale.{name}: float32 contiguous (>= {size})")

    def args(self, n: int) -> _lib.RowScaleArgs:
        self.check(n)
        return _lib.RowScaleArgs(_p(self.scale), _p(self.part), self.D, int(bool(self.two)), float(self.eps),
                                 _p(self.s_out))


def _rs_ptr(rowscale: RowScale | None, n: int):
    """(struct kept alive, its address or None) for a C call."""
    if rowscale is None:
        return None, None
    st = rowscale.args(n)
    return st, ctypes.addressof(st)


def _prep_args(n: int, D: int, dtype, *, r_in=None, s_in=None, w_in=None, r_out=None, a_out=None, wa=None,
               wb=None, part=None) -> _lib.PrepArgs:
    """wfd_prep_t from torch tensors (rows (n, D) with a row pitch; weights (D,))."""
    _need_cuda(r_in, s_in, w_in, r_out, a_out, wa, wb, part)
    for name, t in (("r_in", r_in), ("r_out", r_out), ("a_out", a_out)):
        if t is not None:
            _need(t.dim() == 2 and t.stride(1) == 1 and t.shape[0] >= n and t.shape[1] >= D and t.dtype == dtype,
                  f"{name}: ({n}+, {D}+) rows of {dtype}")
    for name, t in (("w_in", w_in), ("wa", wa), ("wb", wb)):
        if t is not None:
            _need(t.is_contiguous() and t.numel() >= D and t.dtype == dtype, f"{name}: ({D},) {dtype}")
    if s_in is not None:
        _need(s_in.dtype == torch.float32 and s_in.is_contiguous() and s_in.numel() >= n, "s_in: float32 (n,)")
    if part is not None:
        _need(part.dtype == torch.float32 and part.is_contiguous() and part.numel() >= n * FOLD_SLOTS * 2,
              f"part: float32 (n, {FOLD_SLOTS}, 2)")
    ld = lambda t: t.stride(0) if t is not None else 0  # noqa: E731
    return _lib.PrepArgs(_p(r_in), ld(r_in), _p(s_in), _p(w_in), _p(r_out), ld(r_out), _p(a_out), ld(a_out), _p(wa),
                         _p(wb), _p(part))


# ---------------------------------------------------------------------------
# attention
# ---------------------------------------------------------------------------
_WS: dict[int, torch.Tensor] = {}


def attn_workspace_bytes(n: int, H: int, Dh: int, kv_len_max: int) -> int:
    return int(_lib.load().wfd_attn_workspace_bytes(n, H, Dh, kv_len_max))


def attn_workspace(n: int, H: int, Dh: int, kv_len_max: int, device) -> torch.Tensor:
    """A reusable uint8 workspace large enough for this launch shape."""
    need = attn_workspace_bytes(n, H, Dh, kv_len_max)
    dev = torch.device(device)
    key = dev.index if dev.index is not None else torch.cuda.current_device()
    ws = _WS.get(key)
    if ws is None or ws.numel() < need:
        ws = torch.zeros(max(need, 1 << 20), dtype=torch.uint8, device=dev)
        _WS[key] = ws
    return ws


def kv_layout(k_cache: torch.Tensor, v_cache: torch.Tensor) -> tuple[int, int, int]:
    """(Hkv, Dh, block_rows) of a pair of KV caches, read from their shape:
    3-D (rows, Hkv, Dh) is token-major (block_rows 1); 4-D
    (blocks, Hkv, block_rows, Dh) is head-major blocks, cache row r of kv head
    h at [r // block_rows, h, r % block_rows]."""
    _need(k_cache.shape == v_cache.shape and k_cache.dtype == v_cache.dtype, "k/v caches differ in shape or dtype")
    _need(k_cache.is_contiguous() and v_cache.is_contiguous(), "caches must be contiguous")
    if k_cache.dim() == 3:
        return k_cache.shape[1], k_cache.shape[2], 1
    _need(k_cache.dim() == 4, "a KV cache is (rows, Hkv, Dh) or (blocks, Hkv, block_rows, Dh)")
    return k_cache.shape[1], k_cache.shape[3], k_cache.shape[2]


def attn_group_max_rows(H: int, Hkv: int) -> int:
    """Most query rows one attention group may hold for this head shape."""
    return int(_lib.load().wfd_attn_group_max_rows(H, Hkv))


def attn_decode(q: torch.Tensor, k_cache: torch.Tensor, v_cache: torch.Tensor, kv_row_base: torch.Tensor,
                kv_len: torch.Tensor, *, kv_len_max: int, scale: float | None = None,
                out: torch.Tensor | None = None, workspace: torch.Tensor | None = None,
                group_first: torch.Tensor | None = None) -> torch.Tensor:
    """Wavefront decode attention: q (n, H, Dh) over slot rows of the KV
    caches (layout: kv_layout); query i reads cache rows
    kv_row_base[i] + [0, kv_len[i]). `group_first` (int32, n + 1) groups rows
    that share a slot so the prefix is read once per group (same bits)."""
    _need_cuda(q, k_cache, v_cache, kv_row_base, kv_len, group_first)
    _need(q.dim() == 3 and q.is_contiguous(), "q must be contiguous (n, H, Dh)")
    n, H, Dh = q.shape
    Hkv, cDh, br = kv_layout(k_cache, v_cache)
    _need(cDh == Dh and k_cache.dtype == q.dtype, "q/k/v dtype or head_dim mismatch")
    _need(br == 1 or kv_len_max <= br, f"kv_len_max {kv_len_max} exceeds the cache block ({br} rows)")
    _need(kv_row_base.dtype == torch.int64 and kv_row_base.numel() >= n and kv_row_base.is_contiguous(),
          "kv_row_base: int64 (n,)")
    _need(kv_len.dtype == torch.int32 and kv_len.numel() >= n and kv_len.is_contiguous(), "kv_len: int32 (n,)")
    _need(kv_len_max >= 1, "kv_len_max must be >= 1")
    _need(group_first is None or (group_first.dtype == torch.int32 and group_first.is_contiguous()
                                  and group_first.numel() >= n + 1), "group_first: int32 (n + 1,)")
    if out is None:
        out = torch.empty_like(q)
    _need(out.shape == q.shape and out.dtype == q.dtype and out.is_contiguous(), "bad out")
    if workspace is None:
        workspace = attn_workspace(n, H, Dh, kv_len_max, q.device)
    sc = 1.0 / math.sqrt(Dh) if scale is None else float(scale)
    rc = _lib.load().wfd_attn_decode(
        q.data_ptr(), k_cache.data_ptr(), v_cache.data_ptr(), br, kv_row_base.data_ptr(), kv_len.data_ptr(),
        _p(group_first), out.data_ptr(), n, H, Hkv, Dh, _dt(q), sc, int(kv_len_max), workspace.data_ptr(),
        workspace.numel() * workspace.element_size(), _stream())
    _lib.check(rc, "wfd_attn_decode")
    return out


def attn_varlen_rows(cu_q: torch.Tensor, cu_k: torch.Tensor, total_q: int, *, causal: bool,
                     kv_row_base: torch.Tensor | None = None, kv_len: torch.Tensor | None = None):
    """Per-row (kv_row_base int64, kv_len int32) tables of a packed varlen call,
    built on the device from cu_q / cu_k (int32, nseg + 1): row r of segment s
    reads keys from row cu_k[s] of a token-major K / V; all of the segment, or
    (causal) keys [0, k_len - q_len + r - cu_q[s]]."""
    _need_cuda(cu_q, cu_k, kv_row_base, kv_len)
    _need(cu_q.dtype == torch.int32 and cu_k.dtype == torch.int32 and cu_q.is_contiguous() and cu_k.is_contiguous()
          and cu_q.numel() == cu_k.numel() and cu_q.numel() >= 1, "cu_q / cu_k: int32 (nseg + 1,)")
    if kv_row_base is None:
        kv_row_base = torch.empty(total_q, dtype=torch.int64, device=cu_q.device)
    if kv_len is None:
        kv_len = torch.empty(total_q, dtype=torch.int32, device=cu_q.device)
    _need(kv_row_base.dtype == torch.int64 and kv_row_base.is_contiguous() and kv_row_base.numel() >= total_q,
          "kv_row_base: int64 (>= total_q,)")
    _need(kv_len.dtype == torch.int32 and kv_len.is_contiguous() and kv_len.numel() >= total_q,
          "kv_len: int32 (>= total_q,)")
    rc = _lib.load().wfd_attn_varlen_rows(cu_q.data_ptr(), cu_k.data_ptr(), cu_q.numel() - 1, int(total_q),
                                          1 if causal else 0, kv_row_base.data_ptr(), kv_len.data_ptr(), _stream())
    _lib.check(rc, "wfd_attn_varlen_rows")
    return kv_row_base, kv_len


def attn_prefill(q: torch.Tensor, k_cache: torch.Tensor, v_cache: torch.Tensor, seg_row_base: torch.Tensor,
                 seg_q_start: torch.Tensor, seg_pos0: torch.Tensor, *, max_seg_len: int, scale: float | None = None,
                 out: torch.Tensor | None = None) -> torch.Tensor:
    """Causal prefill attention (bf16, MFMA): segment s = q rows
    [seg_q_start[s], seg_q_start[s+1]) at positions seg_pos0[s] + 0, 1, ... of
    the slot at cache row seg_row_base[s]; each row attends keys [0, position]."""
    _need_cuda(q, k_cache, v_cache, seg_row_base, seg_q_start, seg_pos0)
    _need(q.dim() == 3 and q.is_contiguous(), "q must be contiguous (n, H, Dh)")
    n, H, Dh = q.shape
    Hkv, cDh, br = kv_layout(k_cache, v_cache)
    _need(cDh == Dh and k_cache.dtype == q.dtype, "q/k/v dtype or head_dim mismatch")
    nseg = seg_row_base.numel()
    _need(seg_row_base.dtype == torch.int64 and seg_row_base.is_contiguous(), "seg_row_base: int64 (nseg,)")
    _need(seg_q_start.dtype == torch.int32 and seg_q_start.is_contiguous() and seg_q_start.numel() == nseg + 1,
          "seg_q_start: int32 (nseg + 1,)")
    _need(seg_pos0.dtype == torch.int32 and seg_pos0.is_contiguous() and seg_pos0.numel() == nseg,
          "seg_pos0: int32 (nseg,)")
    if out is None:
        out = torch.empty_like(q)
    _need(out.shape == q.shape and out.dtype == q.dtype and out.is_contiguous(), "bad out")
    sc = 1.0 / math.sqrt(Dh) if scale is None else float(scale)
    rc = _lib.load().wfd_attn_prefill(q.data_ptr(), k_cache.data_ptr(), v_cache.data_ptr(), br,
                                      seg_row_base.data_ptr(), seg_q_start.data_ptr(), seg_pos0.data_ptr(),
                                      out.data_ptr(), nseg, int(max_seg_len), H, Hkv, Dh, _dt(q), sc, _stream())
    _lib.check(rc, "wfd_attn_prefill")
    return out


# ---------------------------------------------------------------------------
# slot-cache append
# ---------------------------------------------------------------------------
def kv_append(k: torch.Tensor, v: torch.Tensor, k_cache: torch.Tensor, v_cache: torch.Tensor,
              flat_row: torch.Tensor) -> None:
    """Cache row flat_row[i] of k_cache / v_cache = k[i] / v[i] (each (Hkv, Dh))."""
    _need_cuda(k, v, k_cache, v_cache, flat_row)
    n = k.shape[0]
    Hkv, Dh, br = kv_layout(k_cache, v_cache)
    _need(k.is_contiguous() and v.is_contiguous() and k.shape == v.shape and k[0].numel() == Hkv * Dh,
          "k/v rows must match cache rows")
    _need(k.dtype == v.dtype == k_cache.dtype, "dtype mismatch")
    _need(flat_row.dtype == torch.int64 and flat_row.numel() >= n and flat_row.is_contiguous(), "flat_row: int64")
    rc = _lib.load().wfd_kv_append(k.data_ptr(), v.data_ptr(), k_cache.data_ptr(), v_cache.data_ptr(), br,
                                   flat_row.data_ptr(), n, Hkv, Dh, _dt(k), _stream())
    _lib.check(rc, "wfd_kv_append")


def swiglu(gu: torch.Tensor, *, n: int | None = None, out: torch.Tensor | None = None) -> torch.Tensor:
    """silu(gate) * up of rows gu = [gate (F) | up (F)] (wfd_swiglu): the
    linear layer's SwiGLU epilogue for a gate|up product computed elsewhere."""
    _need_cuda(gu)
    _need(gu.dim() == 2 and gu.stride(1) == 1 and gu.shape[1] % 2 == 0, "gu: (n, 2F) with unit column stride")
    n = gu.shape[0] if n is None else n
    F = gu.shape[1] // 2
    if out is None:
        out = torch.empty(n, F, dtype=gu.dtype, device=gu.device)
    _need_cuda(out)
    _need(out.dtype == gu.dtype and out.dim() == 2 and out.stride(1) == 1 and out.shape[1] == F, "out: (n, F)")
    _need(0 <= n <= min(gu.shape[0], out.shape[0]), "n: within the rows of gu and out")
    rc = _lib.load().wfd_swiglu(gu.data_ptr(), gu.stride(0), out.data_ptr(), out.stride(0), n, F, _dt(gu), _stream())
    _lib.check(rc, "wfd_swiglu")
    return out


def qkv_rope_append(qkv: torch.Tensor, pos: torch.Tensor, rope_cos: torch.Tensor, rope_sin: torch.Tensor,
                    flat_row: torch.Tensor, k_cache: torch.Tensor, v_cache: torch.Tensor, H: int, Hkv: int, Dh: int,
                    q_out: torch.Tensor | None = None) -> torch.Tensor:
    _need_cuda(qkv, pos, rope_cos, rope_sin, flat_row, k_cache, v_cache)
    n = qkv.shape[0]
    _need(qkv.dim() == 2 and qkv.stride(1) == 1 and qkv.shape[1] >= (H + 2 * Hkv) * Dh, "qkv (n, (H+2Hkv)Dh)")
    _need(pos.dtype == torch.int32 and pos.numel() >= n and pos.is_contiguous(), "pos: int32")
    _need(flat_row.dtype == torch.int64 and flat_row.numel() >= n and flat_row.is_contiguous(), "flat_row: int64")
    _need(rope_cos.dtype == torch.float32 and rope_cos.shape == rope_sin.shape and rope_cos.shape[1] == Dh // 2,
          "rope tables: float32 (S, Dh/2)")
    cHkv, cDh, br = kv_layout(k_cache, v_cache)
    _need((cHkv, cDh) == (Hkv, Dh) and k_cache.dtype == qkv.dtype, "cache shape/dtype mismatch")
    if q_out is None:
        q_out = torch.empty(n, H, Dh, dtype=qkv.dtype, device=qkv.device)
    _need_cuda(q_out)
    _need(q_out.is_contiguous() and q_out.numel() >= n * H * Dh and q_out.dtype == qkv.dtype, "q_out (n, H, Dh)")
    rc = _lib.load().wfd_qkv_rope_append(qkv.data_ptr(), qkv.stride(0), pos.data_ptr(), rope_cos.data_ptr(),
                                         rope_sin.data_ptr(), rope_cos.shape[0], flat_row.data_ptr(),
                                         q_out.data_ptr(), k_cache.data_ptr(), v_cache.data_ptr(), br, n, H, Hkv,
                                         Dh, _dt(qkv), _stream())
    _lib.check(rc, "wfd_qkv_rope_append")
    return q_out


def linear_qkv_rope_append(x: torch.Tensor, Wqkv: torch.Tensor, pos: torch.Tensor, rope_cos: torch.Tensor,
                           rope_sin: torch.Tensor, flat_row: torch.Tensor, k_cache: torch.Tensor,
                           v_cache: torch.Tensor, H: int, Hkv: int, Dh: int, *, n: int | None = None,
                           x_rows: torch.Tensor | None = None, q_out: torch.Tensor | None = None,
                           rowscale: RowScale | None = None) -> torch.Tensor:
    """q_out, plus k/v appended at flat_row: the Wqkv projection with RoPE and
    the cache append as its epilogue (== linear() then qkv_rope_append()).
    rowscale: x holds a folded norm pair's operand rows, scaled per row."""
    _need_cuda(x, pos, rope_cos, rope_sin, flat_row, k_cache, v_cache, x_rows, q_out)
    Wp = _packed(Wqkv, False)
    n = (x.shape[0] if x_rows is None else x_rows.numel()) if n is None else n
    _rows(x_rows, n, "x_rows")
    K = Wp.K
    _need(x.dim() == 2 and x.stride(1) == 1 and x.shape[1] >= K and x.dtype == Wp.dtype, "x (rows, K+)")
    _need(n >= 0 and (x_rows is not None or x.shape[0] >= n), f"x holds {x.shape[0]} rows < n={n}")
    _need(Wp.N == (H + 2 * Hkv) * Dh, "Wqkv ((H+2Hkv)Dh, K)")
    _need(pos.dtype == torch.int32 and pos.numel() >= n and pos.is_contiguous(), "pos: int32")
    _need(flat_row.dtype == torch.int64 and flat_row.numel() >= n and flat_row.is_contiguous(), "flat_row: int64")
    _need(rope_cos.dtype == torch.float32 and rope_cos.shape == rope_sin.shape and rope_cos.shape[1] == Dh // 2
          and rope_cos.is_contiguous() and rope_sin.is_contiguous(), "rope tables: float32 (S, Dh/2)")
    cHkv, cDh, br = kv_layout(k_cache, v_cache)
    _need((cHkv, cDh) == (Hkv, Dh) and k_cache.dtype == x.dtype, "cache shape/dtype mismatch")
    if q_out is None:
        q_out = torch.empty(n, H, Dh, dtype=x.dtype, device=x.device)
    _need(q_out.is_contiguous() and q_out.numel() >= n * H * Dh and q_out.dtype == x.dtype, "q_out (n, H, Dh)")
    keep, rsp = _rs_ptr(rowscale, n)
    rc = _lib.load().wfd_linear_qkv_rope_append(x.data_ptr(), _p(x_rows), x.stride(0), Wp.data.data_ptr(), n, K,
                                                pos.data_ptr(), rope_cos.data_ptr(), rope_sin.data_ptr(),
                                                rope_cos.shape[0], flat_row.data_ptr(), q_out.data_ptr(),
                                                k_cache.data_ptr(), v_cache.data_ptr(), br, H, Hkv, Dh, _dt(x), rsp,
                                                _stream())
    _lib.check(rc, "wfd_linear_qkv_rope_append")
    return q_out


# ---------------------------------------------------------------------------
# linear / norms / small gathers
# ---------------------------------------------------------------------------
def linear_k_multiple(dtype: torch.dtype) -> int:
    return int(_lib.load().wfd_linear_k_multiple(_DT[dtype]))


def fold_max_d(dtype: torch.dtype) -> int:
    """Widest row (d_model) a folded norm pair takes: one wave holds a whole
    row as 16 chunks of the linears' K granularity (wfd_linear_prep,
    wfd_norm_prep): 2048 bf16, 1024 fp32."""
    return 16 * linear_k_multiple(dtype)


class PackedWeight:
    """A linear weight in the kernels' packed layout (wfd_linear_pack): same
    bytes as the (N, K) nn.Linear weight, in MFMA fragment order. `swiglu`
    records the gate|up pairing the packing baked in."""

    __slots__ = ("data", "N", "K", "swiglu")

    def __init__(self, data: torch.Tensor, N: int, K: int, swiglu: bool):
        self.data, self.N, self.K, self.swiglu = data, N, K, swiglu

    @property
    def dtype(self) -> torch.dtype:
        return self.data.dtype

    @property
    def device(self) -> torch.device:
        return self.data.device

    @property
    def shape(self) -> tuple[int, int]:
        return (self.N, self.K)


def pack_linear(W: torch.Tensor, *, swiglu: bool = False) -> PackedWeight:
    """Pack a (N, K) weight (for swiglu: gate rows then up rows) once."""
    _need_cuda(W)
    _need(W.dim() == 2 and W.is_contiguous(), "W: contiguous (N, K)")
    N, K = W.shape
    out = torch.empty_like(W)
    epi = _lib.EPI_SWIGLU if swiglu else _lib.EPI_PLAIN
    rc = _lib.load().wfd_linear_pack(W.data_ptr(), out.data_ptr(), N, K, _dt(W), epi, N // 2 if swiglu else 0,
                                     _stream())
    _lib.check(rc, "wfd_linear_pack")
    return PackedWeight(out, N, K, swiglu)


def _packed(W, swiglu: bool) -> PackedWeight:
    if isinstance(W, PackedWeight):
        _need(W.swiglu == swiglu, "weight packed for a different epilogue")
        return W
    return pack_linear(W, swiglu=swiglu)  # a plain (N, K) tensor: pack a copy for this call


def linear(x: torch.Tensor, W, *, n: int | None = None, x_rows: torch.Tensor | None = None,
           out: torch.Tensor | None = None, swiglu: bool = False, out_dtype: torch.dtype | None = None,
           k: int | None = None, rowscale: RowScale | None = None) -> torch.Tensor:
    """y = x[rows, :K] @ W^T (W: PackedWeight or plain (N, K)); swiglu: N = 2F,
    y (n, F) = silu(g) * u. rowscale: x holds a folded norm pair's operand
    rows, and each output row is scaled (before the SwiGLU)."""
    _need_cuda(x, x_rows, out)
    Wp = _packed(W, swiglu)
    _need_cuda(Wp.data)
    _need(x.dim() == 2 and x.stride(1) == 1, "x (rows, K+)")
    N, K = Wp.N, Wp.K
    if k is not None:
        _need(k == K, "K mismatch")
    n = x.shape[0] if (n is None and x_rows is None) else (n if n is not None else x_rows.numel())
    _rows(x_rows, n, "x_rows")
    _need(x.shape[1] >= K and x.dtype == Wp.dtype, f"x width {x.shape[1]} < K={K} or dtype mismatch")
    _need(n >= 0 and (x_rows is not None or x.shape[0] >= n), f"x holds {x.shape[0]} rows < n={n}")
    od = out_dtype or x.dtype
    width = N // 2 if swiglu else N
    if out is None:
        out = torch.empty(n, width, dtype=od, device=x.device)
    _need(out.dim() == 2 and out.stride(1) == 1 and out.shape[0] >= n and out.shape[1] >= width and out.dtype == od,
          "bad out")
    epi = _lib.EPI_SWIGLU if swiglu else _lib.EPI_PLAIN
    keep, rsp = _rs_ptr(rowscale, n)
    rc = _lib.load().wfd_linear(x.data_ptr(), _p(x_rows), x.stride(0), Wp.data.data_ptr(), out.data_ptr(),
                                out.stride(0), n, N, K, _dt(x), _DT[od], epi, N // 2 if swiglu else 0, rsp, _stream())
    _lib.check(rc, "wfd_linear")
    return out


def linear_prep(x: torch.Tensor, W, *, n: int, a_out: torch.Tensor, wb: torch.Tensor, part: torch.Tensor,
                x_rows: torch.Tensor | None = None, r_in: torch.Tensor | None = None,
                s_in: torch.Tensor | None = None, w_in: torch.Tensor | None = None,
                r_out: torch.Tensor | None = None, wa: torch.Tensor | None = None) -> None:
    """A d_model-output linear (n <= 16) whose epilogue prepares a folded norm
    pair (wfd_linear_prep): r = round(y + x_in) into r_out (x_in from r_in /
    s_in / w_in, or none), A = round((r * wa) * wb) into a_out, and the
    group sums into part."""
    _need_cuda(x, x_rows)
    Wp = _packed(W, False)
    _need_cuda(Wp.data)
    _need(x.dim() == 2 and x.stride(1) == 1 and x.dtype == Wp.dtype and x.shape[1] >= Wp.K, "x (rows, K+)")
    _rows(x_rows, n, "x_rows")
    _need(n >= 0 and (x_rows is not None or x.shape[0] >= n), f"x holds {x.shape[0]} rows < n={n}")
    pp = _prep_args(n, Wp.N, x.dtype, r_in=r_in, s_in=s_in, w_in=w_in, r_out=r_out, a_out=a_out, wa=wa, wb=wb,
                    part=part)
    rc = _lib.load().wfd_linear_prep(x.data_ptr(), _p(x_rows), x.stride(0), Wp.data.data_ptr(), n, Wp.N, Wp.K,
                                     _dt(x), ctypes.addressof(pp), _stream())
    _lib.check(rc, "wfd_linear_prep")


def norm_prep(*, n: int, D: int, dtype: torch.dtype, eps: float, a: torch.Tensor | None = None,
              part: torch.Tensor | None = None, nslices: int = 0, r_in: torch.Tensor | None = None,
              s_in: torch.Tensor | None = None, w_in: torch.Tensor | None = None,
              r_out: torch.Tensor | None = None, a_out: torch.Tensor | None = None, wa: torch.Tensor | None = None,
              wb: torch.Tensor | None = None, two: bool = True, scale_out: torch.Tensor | None = None,
              s_out: torch.Tensor | None = None, h_out: torch.Tensor | None = None,
              h_rows: torch.Tensor | None = None) -> None:
    """The row form of a folded norm pair (wfd_norm_prep): y = a rows, or the
    in-order slice sums of linear_partials (part, nslices); with a_out: A,
    scale_out (s_a * s_b), s_out (s_a) and r into r_out if given; with
    h_out: norm a's output round((r * s_a) * wa) into rows h_rows (without
    a_out: the block's last norm)."""
    _need_cuda(a, part, scale_out, s_out, h_out, h_rows)
    _need((a is None) != (part is None), "norm_prep: exactly one of a / part")
    if a is not None:
        _need(a.dim() == 2 and a.stride(1) == 1 and a.dtype == dtype and a.shape[1] >= D
              and a.shape[0] >= n, "a: (n, D) rows")
    if part is not None:
        _need(part.dtype == torch.float32 and part.is_contiguous() and part.numel() >= nslices * n * D,
              "part: the slice sums of linear_partials")
    for name, t in (("scale_out", scale_out), ("s_out", s_out)):
        if t is not None:
            _need(t.dtype == torch.float32 and t.is_contiguous() and t.numel() >= n, f"{name}: float32 (n,)")
    if h_out is not None:
        _need(h_out.dim() == 2 and h_out.stride(1) == 1 and h_out.dtype == dtype and h_out.shape[1] >= D, "h_out")
        _rows(h_rows, n, "h_rows")
        if h_rows is None:
            _need(h_out.shape[0] >= n, "h_out rows < n")
    pp = _prep_args(n, D, dtype, r_in=r_in, s_in=s_in, w_in=w_in, r_out=r_out, a_out=a_out, wa=wa, wb=wb)
    rc = _lib.load().wfd_norm_prep(_p(a), a.stride(0) if a is not None else 0, _p(part), n * D, nslices,
                                   ctypes.addressof(pp), int(bool(two)), float(eps), _p(scale_out), _p(s_out),
                                   _p(h_out), _p(h_rows), h_out.stride(0) if h_out is not None else 0, n, D,
                                   _DT[dtype], _stream())
    _lib.check(rc, "wfd_norm_prep")


def add_rmsnorm(a: torch.Tensor, w1: torch.Tensor, eps: float, *, res: torch.Tensor | None = None,
                w2: torch.Tensor | None = None, n: int | None = None, a_rows: torch.Tensor | None = None,
                x_out: torch.Tensor | None = None, out_rows: torch.Tensor | None = None,
                h_out: torch.Tensor | None = None):
    """x_out = rmsnorm(a + res) * w1; if w2: also h_out = rmsnorm(x_out) * w2.
    Returns x_out, or (x_out, h_out) when w2 is given."""
    _need_cuda(a, w1, res, w2, a_rows, x_out, out_rows, h_out)
    D = w1.numel()
    n = (a.shape[0] if a_rows is None else a_rows.numel()) if n is None else n
    _rows(a_rows, n, "a_rows")
    _rows(out_rows, n, "out_rows")
    _need(a.dim() == 2 and a.stride(1) == 1 and a.shape[1] >= D, "a (rows, D+)")
    _need(n >= 0 and (a_rows is not None or a.shape[0] >= n), f"a holds {a.shape[0]} rows < n={n}")
    if res is not None:
        _need(res.dim() == 2 and res.stride(1) == 1 and res.shape[0] >= n and res.shape[1] >= D
              and res.dtype == a.dtype, "bad res")
    if x_out is None:
        x_out = torch.empty(n, D, dtype=a.dtype, device=a.device)
    if w2 is not None and h_out is None:
        h_out = torch.empty(n, D, dtype=a.dtype, device=a.device)
    if x_out is not None:
        _need(x_out.dim() == 2 and x_out.stride(1) == 1 and x_out.shape[1] >= D and x_out.dtype == a.dtype
              and (out_rows is not None or x_out.shape[0] >= n), "x_out: (>= n rows, D+) of a's dtype")
    if h_out is not None:
        _need(h_out.dim() == 2 and h_out.stride(1) == 1 and h_out.shape[1] >= D and h_out.shape[0] >= n
              and h_out.dtype == a.dtype, "h_out: (>= n rows, D+) of a's dtype")
    rc = _lib.load().wfd_add_rmsnorm(a.data_ptr(), _p(a_rows), a.stride(0), _p(res),
                                     res.stride(0) if res is not None else 0, w1.data_ptr(), _p(w2),
                                     x_out.data_ptr(), _p(out_rows), x_out.stride(0), _p(h_out),
                                     h_out.stride(0) if h_out is not None else 0, n, D, float(eps), _dt(a), _stream())
    _lib.check(rc, "wfd_add_rmsnorm")
    return (x_out, h_out) if w2 is not None else x_out


def rmsnorm(x: torch.Tensor, w: torch.Tensor, eps: float, **kw) -> torch.Tensor:
    return add_rmsnorm(x, w, eps, **kw)


def linear_slices(K: int, dtype: torch.dtype) -> int:
    """K slices of the linear's arithmetic contract for this K (1..4)."""
    s = _lib.load().wfd_linear_slices(K, _DT[dtype])
    _need(s > 0, f"K={K} is not a multiple of the linear's chunk")
    return s


def linear_partials(x: torch.Tensor, W, part: torch.Tensor, *, n: int | None = None,
                    x_rows: torch.Tensor | None = None) -> int:
    """Split-K linear: part (flat fp32, >= slices * n * N) receives the slice
    sums, slice q of row m at part[(q * n + m) * N:]. Returns the number of
    slices; add_rmsnorm_split turns them into the linear's output rows."""
    _need_cuda(x, x_rows, part)
    Wp = _packed(W, False)
    _need_cuda(Wp.data)
    _need(x.dim() == 2 and x.stride(1) == 1, "x (rows, K+)")
    N, K = Wp.N, Wp.K
    n = x.shape[0] if (n is None and x_rows is None) else (n if n is not None else x_rows.numel())
    _rows(x_rows, n, "x_rows")
    _need(x.shape[1] >= K and x.dtype == Wp.dtype, f"x width {x.shape[1]} < K={K} or dtype mismatch")
    _need(n >= 0 and (x_rows is not None or x.shape[0] >= n), f"x holds {x.shape[0]} rows < n={n}")
    S = linear_slices(K, x.dtype)
    _need(part.dtype == torch.float32 and part.is_contiguous() and part.numel() >= S * n * N,
          f"part: contiguous fp32 of >= {S}*{n}*{N} elements")
    rc = _lib.load().wfd_linear_partials(x.data_ptr(), _p(x_rows), x.stride(0), Wp.data.data_ptr(),
                                         part.data_ptr(), n, N, K, _dt(x), _stream())
    _lib.check(rc, "wfd_linear_partials")
    return S


def add_rmsnorm_split(part: torch.Tensor, nslices: int, n: int, w1: torch.Tensor, eps: float, *,
                      dtype: torch.dtype, res: torch.Tensor | None = None, w2: torch.Tensor | None = None,
                      a_out: torch.Tensor | None = None, x_out: torch.Tensor | None = None,
                      out_rows: torch.Tensor | None = None, h_out: torch.Tensor | None = None):
    """add_rmsnorm whose `a` rows are the slice sums linear_partials left in
    `part` (n rows, D = w1.numel() columns), added in slice order and rounded
    to `dtype`; a_out, if given, keeps those rows. Returns like add_rmsnorm."""
    _need_cuda(part, w1, res, w2, a_out, x_out, out_rows, h_out)
    D = w1.numel()
    _rows(out_rows, n, "out_rows")
    _need(n >= 0 and 1 <= nslices <= 4, f"n={n} nslices={nslices}")
    _need(part.dtype == torch.float32 and part.is_contiguous() and part.numel() >= nslices * n * D,
          f"part: contiguous fp32 of >= {nslices}*{n}*{D} elements")
    for name, t in (("res", res), ("a_out", a_out)):
        if t is not None:
            _need(t.dim() == 2 and t.stride(1) == 1 and t.shape[0] >= n and t.shape[1] >= D and t.dtype == dtype,
                  f"bad {name}")
    if x_out is None:
        x_out = torch.empty(n, D, dtype=dtype, device=part.device)
    if w2 is not None and h_out is None:
        h_out = torch.empty(n, D, dtype=dtype, device=part.device)
    _need(x_out.dim() == 2 and x_out.stride(1) == 1 and x_out.shape[1] >= D and x_out.dtype == dtype
          and (out_rows is not None or x_out.shape[0] >= n), "x_out: (>= n rows, D+)")
    if h_out is not None:
        _need(h_out.dim() == 2 and h_out.stride(1) == 1 and h_out.shape[1] >= D and h_out.shape[0] >= n
              and h_out.dtype == dtype, "h_out: (>= n rows, D+)")
    rc = _lib.load().wfd_add_rmsnorm_split(
        part.data_ptr(), n * D, nslices, _p(a_out), a_out.stride(0) if a_out is not None else 0, _p(res),
        res.stride(0) if res is not None else 0, w1.data_ptr(), _p(w2), x_out.data_ptr(), _p(out_rows),
        x_out.stride(0), _p(h_out), h_out.stride(0) if h_out is not None else 0, n, D, float(eps), _DT[dtype],
        _stream())
    _lib.check(rc, "wfd_add_rmsnorm_split")
    return (x_out, h_out) if w2 is not None else x_out


def embed(ids: torch.Tensor, table: torch.Tensor, scale: float = 1.0, *, out: torch.Tensor | None = None,
          ring: torch.Tensor | None = None):
    """out[i] = table[id_i] * scale; with `ring`, a negative ids[i] = -(slot + 1)
    takes its id from ring[slot] on the device."""
    _need_cuda(ids, table, out, ring)
    _need(ids.dtype == torch.int64 and ids.is_contiguous(), "ids: int64")
    if ring is not None:
        _need(ring.dtype == torch.int64 and ring.is_contiguous(), "ring: int64 contiguous")
    n = ids.numel()
    Vocab, D = table.shape
    _need(table.dim() == 2 and table.is_contiguous(), "table: contiguous (vocab, D)")
    if out is None:
        out = torch.empty(n, D, dtype=table.dtype, device=table.device)
    _need(out.dim() == 2 and out.stride(1) == 1 and out.shape[0] >= n and out.shape[1] >= D
          and out.dtype == table.dtype, "out: (>= n rows, D+) of the table's dtype")
    rc = _lib.load().wfd_embed(ids.data_ptr(), _p(ring), ring.numel() if ring is not None else 0, table.data_ptr(),
                               float(scale), out.data_ptr(), out.stride(0), n, Vocab, D, _dt(table), _stream())
    _lib.check(rc, "wfd_embed")
    return out


def embed_rmsnorm(ids: torch.Tensor, table: torch.Tensor, scale: float, w1: torch.Tensor, eps: float, *,
                  h_out: torch.Tensor, x_out: torch.Tensor | None = None, ring: torch.Tensor | None = None,
                  n: int | None = None, copy: tuple | None = None) -> None:
    """One launch for embed(ids) -> x_out (optional) and rmsnorm(x) * w1 ->
    h_out, the bits of embed + rmsnorm; `copy` = (src, src_rows, dst,
    dst_rows, width) adds copy_rows(src, dst, ...) for the same n rows."""
    _need_cuda(ids, table, w1, h_out, x_out, ring)
    _need(ids.dtype == torch.int64 and ids.is_contiguous(), "ids: int64")
    if ring is not None:
        _need(ring.dtype == torch.int64 and ring.is_contiguous(), "ring: int64 contiguous")
    n = ids.numel() if n is None else n
    _need(0 <= n <= ids.numel(), f"ids hold {ids.numel()} < n={n}")
    Vocab, D = table.shape
    _need(table.dim() == 2 and table.is_contiguous() and w1.numel() == D, "table: contiguous (vocab, D); w1: (D,)")
    for name, t in (("h_out", h_out), ("x_out", x_out)):
        if t is not None:
            _need(t.dim() == 2 and t.stride(1) == 1 and t.shape[0] >= n and t.shape[1] >= D and t.dtype == table.dtype,
                  f"{name}: (>= n rows, D+) of the table's dtype")
    cp = (None, None, 0, None, None, 0, 0)
    if copy is not None:
        src, src_rows, dst, dst_rows, width = copy
        _need_cuda(src, src_rows, dst, dst_rows)
        _rows(src_rows, n, "src_rows")
        _rows(dst_rows, n, "dst_rows")
        _need(src.dtype == dst.dtype == table.dtype and src.dim() == 2 and dst.dim() == 2 and src.stride(1) == 1
              and dst.stride(1) == 1 and 0 < width <= min(src.shape[1], dst.shape[1]), "copy: 2-D src/dst, width")
        _need(src_rows is not None or src.shape[0] >= n, f"src holds {src.shape[0]} rows < n={n}")
        _need(dst_rows is not None or dst.shape[0] >= n, f"dst holds {dst.shape[0]} rows < n={n}")
        cp = (src.data_ptr(), _p(src_rows), src.stride(0), dst.data_ptr(), _p(dst_rows), dst.stride(0), width)
    rc = _lib.load().wfd_embed_rmsnorm(
        ids.data_ptr(), _p(ring), ring.numel() if ring is not None else 0, table.data_ptr(), float(scale), Vocab,
        w1.data_ptr(), _p(x_out), x_out.stride(0) if x_out is not None else 0, h_out.data_ptr(), h_out.stride(0),
        *cp, n, D, float(eps), _dt(table), _stream())
    _lib.check(rc, "wfd_embed_rmsnorm")


def copy_rows(src: torch.Tensor, dst: torch.Tensor, *, n: int, width: int, src_rows: torch.Tensor | None = None,
              dst_rows: torch.Tensor | None = None) -> None:
    _need_cuda(src, dst, src_rows, dst_rows)
    _need(src.dtype == dst.dtype and src.stride(-1) == 1 and dst.stride(-1) == 1, "copy_rows dtype/layout")
    _rows(src_rows, n, "src_rows")
    _rows(dst_rows, n, "dst_rows")
    _need(src.dim() == 2 and dst.dim() == 2 and 0 <= width <= min(src.shape[1], dst.shape[1]) and n >= 0,
          "copy_rows: 2-D src/dst at least `width` wide")
    _need(src_rows is not None or src.shape[0] >= n, f"src holds {src.shape[0]} rows < n={n}")
    _need(dst_rows is not None or dst.shape[0] >= n, f"dst holds {dst.shape[0]} rows < n={n}")
    rc = _lib.load().wfd_copy_rows(src.data_ptr(), _p(src_rows), src.stride(0), dst.data_ptr(), _p(dst_rows),
                                   dst.stride(0), n, width, _dt(src), _stream())
    _lib.check(rc, "wfd_copy_rows")


def argmax(logits: torch.Tensor, *, n: int | None = None, out: torch.Tensor | None = None,
           ring: torch.Tensor | None = None, ring_rows: torch.Tensor | None = None,
           expect: torch.Tensor | None = None, accept: torch.Tensor | None = None,
           accept_mapped: tuple[int, int] | None = None) -> torch.Tensor:
    """out[i] = argmax logits[i] (first index on ties); with `ring`, also
    ring[ring_rows[i]] = out[i]; with `expect` (int64: a plain id, a ring
    handle, or anything below -len(ring) for no comparison) also
    accept[i] = int32(out[i] == expected token). The flags go to `accept` (a
    device tensor) or to `accept_mapped` = (device address, capacity in
    flags) of mapped pinned host memory, which the host polls without a copy."""
    _need_cuda(logits, out, ring, ring_rows, expect, accept)
    _need(logits.dtype == torch.float32 and logits.dim() == 2 and logits.stride(1) == 1, "logits: float32 (n, V)")
    n = logits.shape[0] if n is None else n
    _need(0 <= n <= logits.shape[0], f"n={n} outside the {logits.shape[0]} logits rows")
    out, acc = _argmax_outputs(n, logits.device, out, ring, ring_rows, expect, accept, accept_mapped)
    rc = _lib.load().wfd_argmax(logits.data_ptr(), logits.stride(0), out.data_ptr(), _p(ring), _p(ring_rows),
                                ring.numel() if ring is not None else 0, _p(expect), acc, n, logits.shape[1],
                                _stream())
    _lib.check(rc, "wfd_argmax")
    return out


def _argmax_outputs(n, device, out, ring, ring_rows, expect, accept, accept_mapped):
    """Checks argmax's ring / expect / accept operands; returns (out, accept address)."""
    if ring is not None:
        _need(ring.dtype == torch.int64 and ring.is_contiguous(), "ring: int64 contiguous")
        _rows(ring_rows, n, "ring_rows")
        _need(ring_rows is not None, "ring needs ring_rows")
    if out is None:
        out = torch.empty(n, dtype=torch.int64, device=device)
    _need(out.dtype == torch.int64 and out.is_contiguous() and out.numel() >= n, "out: int64 (>= n,)")
    _need(accept is None or accept_mapped is None, "accept or accept_mapped, not both")
    _need((expect is None) == (accept is None and accept_mapped is None), "expect and accept go together")
    if expect is not None:
        _need(expect.dtype == torch.int64 and expect.is_contiguous() and expect.numel() >= n, "expect: int64 (>= n,)")
        if accept is not None:
            _need(accept.dtype == torch.int32 and accept.is_contiguous() and accept.numel() >= n,
                  "accept: int32 (>= n,)")
        else:
            _need(accept_mapped[0] != 0 and accept_mapped[0] % 4 == 0 and accept_mapped[1] >= n,
                  "accept_mapped: (aligned device address, capacity >= n)")
    acc = _p(accept) if accept is not None else (accept_mapped[0] if accept_mapped is not None else None)
    return out, acc


def linear_argmax_groups(n: int, W) -> int:
    """Column groups per row that linear_argmax leaves for n rows of the
    packed plain weight W (0 where the few-row kernel would not run)."""
    Wp = _packed(W, False)
    return int(_lib.load().wfd_linear_argmax_groups(n, Wp.N, Wp.K, _DT[Wp.dtype]))


def linear_argmax(x: torch.Tensor, W, *, n: int | None = None, x_rows: torch.Tensor | None = None,
                  out: torch.Tensor | None = None, part_val: torch.Tensor | None = None,
                  part_idx: torch.Tensor | None = None, rowscale: RowScale | None = None):
    """linear(x, W, out_dtype=float32) for bf16 x / W -- the same kernel, so
    the same bits -- that also leaves, per row and column group (G =
    linear_argmax_groups(n, W)), the first largest logit and its column in
    part_val / part_idx (m * G + s). Returns (out, part_val, part_idx)."""
    _need_cuda(x, x_rows, out, part_val, part_idx)
    Wp = _packed(W, False)
    _need_cuda(Wp.data)
    _need(x.dim() == 2 and x.stride(1) == 1 and x.dtype == torch.bfloat16 and Wp.dtype == torch.bfloat16,
          "x (rows, K+) and W bf16")
    N, K = Wp.N, Wp.K
    n = x.shape[0] if (n is None and x_rows is None) else (n if n is not None else x_rows.numel())
    _rows(x_rows, n, "x_rows")
    _need(x.shape[1] >= K, f"x width {x.shape[1]} < K={K}")
    _need(n >= 1 and (x_rows is not None or x.shape[0] >= n), f"x holds {x.shape[0]} rows < n={n}")
    G = linear_argmax_groups(n, Wp)
    _need(G > 0, f"n={n} N={N} K={K}: not a few-row launch (no column groups)")
    if out is None:
        out = torch.empty(n, N, dtype=torch.float32, device=x.device)
    _need(out.dim() == 2 and out.stride(1) == 1 and out.shape[0] >= n and out.shape[1] >= N
          and out.dtype == torch.float32, "out: float32 (>= n, >= N)")
    if part_val is None:
        part_val = torch.empty(n * G, dtype=torch.float32, device=x.device)
    if part_idx is None:
        part_idx = torch.empty(n * G, dtype=torch.int32, device=x.device)
    _need(part_val.dtype == torch.float32 and part_val.is_contiguous() and part_val.numel() >= n * G,
          f"part_val: float32 (>= {n * G},)")
    _need(part_idx.dtype == torch.int32 and part_idx.is_contiguous() and part_idx.numel() >= n * G,
          f"part_idx: int32 (>= {n * G},)")
    keep, rsp = _rs_ptr(rowscale, n)
    rc = _lib.load().wfd_linear_argmax(x.data_ptr(), _p(x_rows), x.stride(0), Wp.data.data_ptr(), out.data_ptr(),
                                       out.stride(0), n, N, K, _dt(x), part_val.data_ptr(), part_idx.data_ptr(), rsp,
                                       _stream())
    _lib.check(rc, "wfd_linear_argmax")
    return out, part_val, part_idx


def argmax_groups(part_val: torch.Tensor, part_idx: torch.Tensor, groups: int, *, n: int,
                  out: torch.Tensor | None = None, ring: torch.Tensor | None = None,
                  ring_rows: torch.Tensor | None = None, expect: torch.Tensor | None = None,
                  accept: torch.Tensor | None = None, accept_mapped: tuple[int, int] | None = None) -> torch.Tensor:
    """argmax from the column-group bests linear_argmax left (`groups` per
    row): the same ids, ring and accept flags as argmax over the logits."""
    _need_cuda(part_val, part_idx, out, ring, ring_rows, expect, accept)
    _need(n >= 0 and groups >= 1, f"n={n} groups={groups}")
    _need(part_val.dtype == torch.float32 and part_val.is_contiguous() and part_val.numel() >= n * groups
          and part_idx.dtype == torch.int32 and part_idx.is_contiguous() and part_idx.numel() >= n * groups,
          f"part_val float32 / part_idx int32 (>= {n * groups},)")
    out, acc = _argmax_outputs(n, part_val.device, out, ring, ring_rows, expect, accept, accept_mapped)
    rc = _lib.load().wfd_argmax_groups(part_val.data_ptr(), part_idx.data_ptr(), groups, out.data_ptr(), _p(ring),
                                       _p(ring_rows), ring.numel() if ring is not None else 0, _p(expect), acc, n,
                                       _stream())
    _lib.check(rc, "wfd_argmax_groups")
    return out
