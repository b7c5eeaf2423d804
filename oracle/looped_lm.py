"""Oracle looped LM: numpy float32, one token at a time.

Restates the Huginn-style P / R / C block forwards the reference decodes with
(src/decoding/huginn_blocks.py:93-103 SandwichBlock, :179-191 P, :197-255 R,
:261-292 C; batch twins src/decoding/huginn_blocks_batch.py:209-346) over a
per-depth slot cache with position == buffer index
(src/decoding/kv_cache.py:8-22, batch_kv_cache.py:37-73). Every op runs on a
single token row, so a token's numbers never depend on what else is in
flight -- the oracle is batch-invariant by construction.

The block structure (sandwich norms, concat adapter, interleaved-pair RoPE,
SwiGLU) follows the reference's own block code (huginn_blocks.py:93-103,216,
261-292); the Huginn module internals it calls live in absent external model
code. The per-op pieces are pinned in tests/test_oracle_kernels.py, and the
composition here in tests/test_oracle_composition.py (closed forms, the
adapter's halves, and a dense causal torch formulation over whole prompts).

`OracleBatchBlocks` exposes the union API that oracle/scheduler.py drives.
"""
from __future__ import annotations

import numpy as np

from . import kernels as K


class OracleLM:
    def __init__(self, cfg, weights: dict[str, np.ndarray], max_seq_len: int, batch: int = 1,
                 s0_tokens=None, s0_prefill=None):
        """cfg: any object with the LoopedLMConfig fields; weights: float32
        arrays keyed like model.param_specs; s0_tokens(p) -> (D,) and
        s0_prefill(L) -> (L, D) give the initial loop state."""
        self.c = cfg
        self.w = {k: np.asarray(v, dtype=np.float32) for k, v in weights.items()}
        self.S = max_seq_len
        self.B = batch
        self.cos, self.sin = K.rope_tables(max_seq_len, cfg.head_dim, cfg.rope_base)
        n_slots = cfg.n_prelude + cfg.T_total * cfg.n_core + cfg.n_coda
        shape = (n_slots, batch, max_seq_len, cfg.n_kv_heads, cfg.head_dim)
        self.Kc = np.zeros(shape, dtype=np.float32)
        self.Vc = np.zeros(shape, dtype=np.float32)
        self.s0_tokens = s0_tokens
        self.s0_prefill = s0_prefill
        self.coda_base = cfg.n_prelude + cfg.T_total * cfg.n_core

    # slot ids: src/decoding/kv_cache.py:12-15
    def slot_core(self, step: int, layer: int) -> int:
        return self.c.n_prelude + step * self.c.n_core + layer

    def block(self, prefix: str, x: np.ndarray, slot: int, b: int, pos: int) -> np.ndarray:
        c, w = self.c, self.w
        H, Hkv, Dh = c.n_heads, c.n_kv_heads, c.head_dim
        h = K.rmsnorm(x, w[prefix + "norm_1"], c.norm_eps)
        qkv = K.linear_row(h, w[prefix + "Wqkv"])
        q = qkv[: H * Dh].reshape(H, Dh)
        k = qkv[H * Dh: (H + Hkv) * Dh].reshape(Hkv, Dh)
        v = qkv[(H + Hkv) * Dh:].reshape(Hkv, Dh)
        q = K.rope(q, pos, self.cos, self.sin)
        k = K.rope(k, pos, self.cos, self.sin)
        self.Kc[slot, b, pos] = k                          # append at position == buffer row
        self.Vc[slot, b, pos] = v
        o = K.attention(q, self.Kc[slot, b], self.Vc[slot, b], pos + 1)   # keys at positions <= pos
        a = K.linear_row(o.reshape(-1), w[prefix + "proj"])
        x = K.rmsnorm(a + x, w[prefix + "norm_2"], c.norm_eps)
        gu = K.linear_row(K.rmsnorm(x, w[prefix + "norm_3"], c.norm_eps), w[prefix + "fc"])
        m = K.linear_row(K.swiglu(gu[: c.ffn], gu[c.ffn:]), w[prefix + "mlp_proj"])
        return K.rmsnorm(m + x, w[prefix + "norm_4"], c.norm_eps)

    def prelude(self, b: int, pos: int, tok: int) -> np.ndarray:
        x = self.w["wte"][tok] * np.float32(self.c.emb_scale)
        for i in range(self.c.n_prelude):
            x = self.block(f"prelude.{i}.", x, i, b, pos)
        return x                                           # static state e

    def core(self, b: int, pos: int, step: int, s: np.ndarray, e: np.ndarray) -> np.ndarray:
        x = K.linear_row(np.concatenate([s, e]), self.w["adapter"])   # adapter(cat[s, e])
        for l in range(self.c.n_core):
            x = self.block(f"core.{l}.", x, self.slot_core(step, l), b, pos)
        return x

    def coda(self, b: int, pos: int, s: np.ndarray) -> np.ndarray:
        x = K.rmsnorm(s, self.w["ln_f"], self.c.norm_eps)
        for i in range(self.c.n_coda):
            x = self.block(f"coda.{i}.", x, self.coda_base + i, b, pos)
        x = K.rmsnorm(x, self.w["ln_f"], self.c.norm_eps)
        return K.linear_row(x, self.w["lm_head"])           # logits (V,)

    def prefill(self, b: int, ids) -> np.ndarray:
        """Prompt positions one by one through the full depth; equal to a dense
        causal prefill because each position only reads earlier positions of
        the same slot. Returns the last position's logits."""
        ids = list(ids)
        s0 = self.s0_prefill(len(ids))
        logits = None
        for p, tok in enumerate(ids):
            e = self.prelude(b, p, tok)
            s = np.asarray(s0[p], dtype=np.float32)
            for r in range(self.c.T_total):
                s = self.core(b, p, r, s, e)
            logits = self.coda(b, p, s)
        return logits


class OracleBatchBlocks:
    """Union API over OracleLM (each union is a loop of single-row calls)."""

    class _Cache:
        def __init__(self):
            self.drops = []
            self.seqlen = [[0]]

        nbytes = 0

        def drop_positions_at_and_after(self, b, position):
            self.drops.append((b, position))

    def __init__(self, lm: OracleLM):
        self.lm = lm
        self.T_total = lm.c.T_total
        self.last_logits = None

    def prefill(self, prompts):
        rows = [list(np.asarray(p).reshape(-1)) for p in prompts]
        self.last_logits = np.stack([self.lm.prefill(b, r) for b, r in enumerate(rows)])
        return self._Cache(), self.last_logits

    def prelude_union(self, seq_ids, toks, cache) -> None:
        for b, t in zip(seq_ids, toks):
            t.static_state = self.lm.prelude(b, t.position, t.token_id)
            t.hidden = np.asarray(self.lm.s0_tokens(t.position), dtype=np.float32)
            t.step = 0

    def advance_union(self, seq_ids, toks, cache) -> None:
        for b, t in zip(seq_ids, toks):
            t.hidden = self.lm.core(b, t.position, t.step, t.hidden, t.static_state)
            t.step += 1

    def coda_logits_union(self, seq_ids, toks, cache) -> list[np.ndarray]:
        return [self.lm.coda(b, t.position, t.hidden) for b, t in zip(seq_ids, toks)]

    def coda_argmax_union(self, seq_ids, toks, cache) -> list[int]:
        return [int(np.argmax(l)) for l in self.coda_logits_union(seq_ids, toks, cache)]
