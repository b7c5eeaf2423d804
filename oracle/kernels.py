"""Oracle kernels: brute-force numpy restatements of the per-op math.

Each function computes in the floating type of its inputs (float32 for the
model-level oracle, float64 when a test wants a tighter reference) and is
written for clarity, one query / row at a time where that makes the
semantics plain.
"""
from __future__ import annotations

import numpy as np


def attention(q: np.ndarray, K: np.ndarray, V: np.ndarray, kv_len: int, scale: float | None = None) -> np.ndarray:
    """One query over a slot prefix: softmax(q . K[:kv_len]^T * scale) @ V[:kv_len].

    q: (H, Dh); K, V: (S, Hkv, Dh) with key position == row (the slot-cache
    invariant, src/decoding/kv_cache.py:8-22); head h reads kv head h // (H / Hkv).
    Follows the reference's explicit-mask twins: a query attends exactly the
    keys at positions <= its own (src/decoding/fa4_attention.py:218-232 for the
    bottom-right dense case, :281-291 for the per-query cutoff, :369-381 for
    the per-segment varlen loop).
    """
    H, Dh = q.shape
    Hkv = K.shape[1]
    G = H // Hkv
    sc = 1.0 / np.sqrt(Dh) if scale is None else scale
    out = np.zeros((H, Dh), dtype=q.dtype)
    if kv_len <= 0:
        return out
    for h in range(H):
        g = h // G
        s = (K[:kv_len, g, :] @ q[h]) * q.dtype.type(sc)
        s = s - s.max()
        p = np.exp(s)
        p = p / p.sum()
        out[h] = p @ V[:kv_len, g, :]
    return out


def attention_rows(q: np.ndarray, Kflat: np.ndarray, Vflat: np.ndarray, row_base, kv_len, scale=None) -> np.ndarray:
    """Batched form over a flat (rows, Hkv, Dh) cache: query i reads rows
    row_base[i] + [0, kv_len[i]) (flat row = (slot*B + b)*S + pos,
    src/decoding/batch_kv_cache.py:64-65)."""
    out = np.zeros_like(q)
    for i in range(q.shape[0]):
        rb, n = int(row_base[i]), int(kv_len[i])
        out[i] = attention(q[i], Kflat[rb: rb + max(n, 0)], Vflat[rb: rb + max(n, 0)], n, scale)
    return out


def rmsnorm(x: np.ndarray, w: np.ndarray, eps: float) -> np.ndarray:
    """y = x / sqrt(mean(x^2) + eps) * w over the last axis."""
    ms = np.mean(x * x, axis=-1, keepdims=True)
    return (x / np.sqrt(ms + x.dtype.type(eps))) * w


def rope_tables(max_pos: int, head_dim: int, base: float = 10000.0) -> tuple[np.ndarray, np.ndarray]:
    """cos/sin tables (max_pos, head_dim/2) of angle pos * base^(-2j/head_dim),
    evaluated in float64 and rounded to float32."""
    j = np.arange(head_dim // 2, dtype=np.float64)
    theta = base ** (-2.0 * j / head_dim)
    ang = np.arange(max_pos, dtype=np.float64)[:, None] * theta[None, :]
    return np.cos(ang).astype(np.float32), np.sin(ang).astype(np.float32)


def rope(x: np.ndarray, pos: int, cos: np.ndarray, sin: np.ndarray) -> np.ndarray:
    """Rotate interleaved pairs (x[2j], x[2j+1]) of every head by angle
    pos*theta_j: the complex-like RoPE of Huginn/parcae
    (apply_rotary_emb_complex_like, used at src/decoding/huginn_blocks.py:86).
    x: (heads, Dh)."""
    c = cos[pos].astype(x.dtype)
    s = sin[pos].astype(x.dtype)
    x0 = x[..., 0::2]
    x1 = x[..., 1::2]
    y = np.empty_like(x)
    y[..., 0::2] = x0 * c - x1 * s
    y[..., 1::2] = x0 * s + x1 * c
    return y


def silu(x: np.ndarray) -> np.ndarray:
    return x / (x.dtype.type(1.0) + np.exp(-x))


def swiglu(gate: np.ndarray, up: np.ndarray) -> np.ndarray:
    return silu(gate) * up


def linear_row(x: np.ndarray, W: np.ndarray) -> np.ndarray:
    """One row through a (N, K) weight: W @ x. Rows are computed one at a time
    so the oracle is itself batch-invariant (the same call shape for every row,
    whatever the tick width) -- the concern probed by
    experiments/exp2_spec_bench/check_tokenwise.py:21-71."""
    return W @ x


def linear(x: np.ndarray, W: np.ndarray) -> np.ndarray:
    return np.stack([linear_row(x[i], W) for i in range(x.shape[0])]) if x.shape[0] else np.zeros(
        (0, W.shape[0]), dtype=x.dtype)
