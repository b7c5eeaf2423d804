"""Device engine: the looped LM's P / R / C passes as fused libwfd launches.

One `LoopedModel` owns the device weights, the RoPE and initial-state (s0)
tables, the wave-state pool and preallocated scratch. A pass runs a *union*
of rows -- any mix of sequences, positions and loop depths -- through:

  prelude_union  wte*emb_scale -> prelude blocks      -> pool[row] = [s0(pos) | e]
  core_union     adapter(pool[row] = [s | e]) -> core blocks (slot by step) -> pool[row][:D]
  coda_union     ln_f(pool[row][:D]) -> coda blocks -> ln_f -> lm_head -> argmax
  prefill_seq    the same blocks over a whole prompt, every slot filled

and every block is: linear(Wqkv) -> qkv_rope_append -> attn_decode ->
linear(proj) -> add_rmsnorm(norm_2, norm_3) -> linear(fc, swiglu) ->
linear(mlp_proj) -> add_rmsnorm(norm_4, next norm_1).

Row tables (positions, slot row bases, append rows, pool rows) are built on
the host per call and uploaded with one copy through a ring of pinned
buffers; the kernels read them as device data. Each row's arithmetic is
independent of the other rows in the union (every kernel is row-invariant),
so a token computed in a wavefront union is bit-identical to the same token
computed alone -- which is what makes wavefront decoding lossless here.

Wave-state pool: row of (seq b, position p) = b*R + p % R with
R = T_total + 2. At most T_total + 1 consecutive positions of one sequence
are in flight (a token enters only after its predecessor has advanced), so
live tokens never share a row, and a re-entered token after a rollback
reuses its position's row.
"""
from __future__ import annotations

import numpy as np
import torch

from . import ops
from .kv_cache import BatchStaticKVCache
from .model import LoopedLMConfig, initial_state_prefill, initial_state_tokens, rope_tables


class _Staging:
    """Ring of pinned host buffers + device buffers for per-call int tables."""

    def __init__(self, device: torch.device, nbytes: int = 1 << 20, depth: int = 4):
        self.device = device
        self.depth = depth
        self.host = [torch.empty(nbytes, dtype=torch.uint8).pin_memory() for _ in range(depth)]
        self.dev = [torch.empty(nbytes, dtype=torch.uint8, device=device) for _ in range(depth)]
        self.events: list[torch.cuda.Event | None] = [None] * depth
        self.i = 0

    def upload(self, arrays: list[np.ndarray]) -> list[torch.Tensor]:
        offs, total = [], 0
        for a in arrays:
            offs.append(total)
            total += (a.nbytes + 255) & ~255
        j = self.i
        self.i = (j + 1) % self.depth
        if self.events[j] is not None:
            self.events[j].synchronize()
        if self.host[j].numel() < total:
            self.host[j] = torch.empty(2 * total, dtype=torch.uint8).pin_memory()
            self.dev[j] = torch.empty(2 * total, dtype=torch.uint8, device=self.device)
        hbuf = self.host[j].numpy()
        for a, o in zip(arrays, offs):
            hbuf[o: o + a.nbytes] = np.ascontiguousarray(a).view(np.uint8).reshape(-1)
        self.dev[j][:total].copy_(self.host[j][:total], non_blocking=True)
        ev = torch.cuda.Event()
        ev.record()
        self.events[j] = ev
        out = []
        for a, o in zip(arrays, offs):
            dt = {np.dtype(np.int32): torch.int32, np.dtype(np.int64): torch.int64}[a.dtype]
            out.append(self.dev[j][o: o + a.nbytes].view(dt).view(a.shape))
        return out


class LoopedModel:
    """Device-resident looped LM running unions of rows through libwfd."""

    def __init__(self, cfg: LoopedLMConfig, weights: dict[str, torch.Tensor], device="cuda", *, max_seq_len: int,
                 max_batch: int = 1, state_init: str = "random", state_seed: int = 0):
        self.cfg = cfg
        self.device = torch.device(device)
        self.dtype = cfg.torch_dtype
        self.max_seq_len = max_seq_len
        self.max_batch = max_batch
        self.state_init = state_init
        self.state_seed = state_seed
        self.W = {k: v.to(device=self.device, dtype=self.dtype).contiguous() for k, v in weights.items()}
        cos, sin = rope_tables(max_seq_len, cfg.head_dim, cfg.rope_base)
        self.rope_cos = cos.to(self.device)
        self.rope_sin = sin.to(self.device)
        self.s0 = initial_state_tokens(cfg, range(max_seq_len), state_seed, state_init).to(
            device=self.device, dtype=self.dtype)
        self.R = cfg.T_total + 2
        D = cfg.d_model
        self.pool = torch.zeros(max_batch * self.R, 2 * D, dtype=self.dtype, device=self.device)
        self._scratch: dict[str, torch.Tensor] = {}
        self._cap = 0
        self._logit_bufs: dict[str, torch.Tensor] = {}
        self._logit_cap = 0
        self.staging = _Staging(self.device)
        self.coda_base = cfg.n_prelude + cfg.T_total * cfg.n_core
        k_mult = ops.linear_k_multiple(self.dtype)
        for K in (D, 2 * D, cfg.n_heads * cfg.head_dim, cfg.ffn):
            if K % k_mult:
                raise ValueError(f"{cfg.name}: K={K} is not a multiple of {k_mult} (linear kernel granularity)")

    # -- slots / rows ----------------------------------------------------------
    def slot_prelude(self, i: int) -> int:
        return i

    def slot_core(self, step: int, layer: int) -> int:
        return self.cfg.n_prelude + step * self.cfg.n_core + layer

    def slot_coda(self, i: int) -> int:
        return self.coda_base + i

    def pool_row(self, b: int, pos: int) -> int:
        return b * self.R + pos % self.R

    def create_cache(self, batch_size: int | None = None) -> BatchStaticKVCache:
        c = self.cfg
        return BatchStaticKVCache(c.n_slots, batch_size or self.max_batch, c.n_kv_heads, c.head_dim,
                                  self.max_seq_len, self.dtype, self.device)

    # -- scratch -----------------------------------------------------------------
    def _ensure(self, n: int) -> dict[str, torch.Tensor]:
        if n <= self._cap:
            return self._scratch
        c = self.cfg
        cap = max(n, 16)
        mk = lambda w, dt=self.dtype: torch.empty(cap, w, dtype=dt, device=self.device)  # noqa: E731
        self._scratch = dict(
            x=mk(c.d_model), h=mk(c.d_model), qkv=mk(c.qkv_dim),
            q=torch.empty(cap, c.n_heads, c.head_dim, dtype=self.dtype, device=self.device),
            o=torch.empty(cap, c.n_heads, c.head_dim, dtype=self.dtype, device=self.device),
            a=mk(c.d_model), u=mk(c.ffn), m=mk(c.d_model),
        )
        self._scratch.update(self._logit_bufs)
        self._cap = cap
        return self._scratch

    def _ensure_logits(self, n: int) -> None:
        """(n, V) float32 logits + (n,) ids, sized separately from the row scratch
        (a prompt prefill needs one logits row, not L)."""
        if n > self._logit_cap:
            cap = max(n, 16)
            self._logit_bufs = dict(
                logits=torch.empty(cap, self.cfg.vocab_size, dtype=torch.float32, device=self.device),
                ids=torch.empty(cap, dtype=torch.int64, device=self.device))
            self._logit_cap = cap
            self._scratch.update(self._logit_bufs)

    # -- one SandwichBlock over n rows --------------------------------------------
    def _block(self, prefix: str, n: int, sc, pos_d, kvlen_d, rb_d, fr_d, kv_len_max: int,
               cache: BatchStaticKVCache, next_norm: torch.Tensor | None, final_out=None, final_rows=None):
        c, W = self.cfg, self.W
        x, h = sc["x"], sc["h"]
        qkv = ops.linear(h, W[prefix + "Wqkv"], n=n, out=sc["qkv"])
        q = ops.qkv_rope_append(qkv[:n], pos_d, self.rope_cos, self.rope_sin, fr_d, cache.flat_k, cache.flat_v,
                                c.n_heads, c.n_kv_heads, c.head_dim, q_out=sc["q"][:n])
        o = ops.attn_decode(q, cache.flat_k, cache.flat_v, rb_d, kvlen_d, kv_len_max=kv_len_max, out=sc["o"][:n],
                            workspace=self._attn_ws(n, kv_len_max))
        a = ops.linear(o.view(n, -1), W[prefix + "proj"], n=n, out=sc["a"])
        ops.add_rmsnorm(a, W[prefix + "norm_2"], c.norm_eps, res=x, w2=W[prefix + "norm_3"], n=n, x_out=x,
                        h_out=h)
        u = ops.linear(h, W[prefix + "fc"], n=n, out=sc["u"], swiglu=True)
        m = ops.linear(u, W[prefix + "mlp_proj"], n=n, out=sc["m"])
        if next_norm is not None:
            ops.add_rmsnorm(m, W[prefix + "norm_4"], c.norm_eps, res=x, w2=next_norm, n=n, x_out=x, h_out=h)
        else:
            ops.add_rmsnorm(m, W[prefix + "norm_4"], c.norm_eps, res=x, n=n, x_out=final_out, out_rows=final_rows)

    def _attn_ws(self, n: int, kv_len_max: int) -> torch.Tensor:
        return ops.attn_workspace(n, self.cfg.n_heads, self.cfg.head_dim, kv_len_max, self.device)

    def _tables(self, cache, seqs: np.ndarray, pos: np.ndarray, slots: np.ndarray):
        """slots: (layers, n) -> row_base, flat_row: (layers, n) int64."""
        rb = (slots * cache.B + seqs[None, :]) * cache.S
        return rb.astype(np.int64), (rb + pos[None, :]).astype(np.int64)

    def _check(self, cache, seqs, pos):
        if len(pos) and (pos.min() < 0 or pos.max() >= cache.S):
            raise IndexError(f"position out of range [0, {cache.S})")
        if len(seqs) and (seqs.min() < 0 or seqs.max() >= cache.B or seqs.max() >= self.max_batch):
            raise IndexError("sequence index out of range")

    # -- P ---------------------------------------------------------------------------
    def prelude_union(self, cache, seqs, positions, token_ids) -> np.ndarray:
        """Embed + prelude blocks for n new tokens; fills pool[row] = [s0(pos) | e].
        Returns the pool rows."""
        c = self.cfg
        seqs = np.asarray(seqs, dtype=np.int64)
        pos = np.asarray(positions, dtype=np.int64)
        n = len(pos)
        if n == 0:
            return np.zeros(0, dtype=np.int64)
        self._check(cache, seqs, pos)
        rows = seqs * self.R + pos % self.R
        slots = np.repeat(np.arange(c.n_prelude, dtype=np.int64)[:, None], n, axis=1)
        rb, fr = self._tables(cache, seqs, pos, slots)
        i32 = np.concatenate([pos, pos + 1, rows]).astype(np.int32)
        i64 = np.concatenate([np.asarray(token_ids, dtype=np.int64), rb.reshape(-1), fr.reshape(-1)])
        t32, t64 = self.staging.upload([i32, i64])
        pos_d, kvlen_d, rows_d = t32[:n], t32[n: 2 * n], t32[2 * n:]
        ids_d = t64[:n]
        sc = self._ensure(n)
        kv_max = int(pos.max()) + 1
        ops.embed(ids_d, self.W["wte"], c.emb_scale, out=sc["x"])
        ops.rmsnorm(sc["x"], self.W["prelude.0.norm_1"], c.norm_eps, n=n, x_out=sc["h"])
        static_half = self.pool[:, c.d_model:]
        for i in range(c.n_prelude):
            last = i == c.n_prelude - 1
            self._block(f"prelude.{i}.", n, sc, pos_d, kvlen_d, t64[n + i * n: n + (i + 1) * n],
                        t64[n + (c.n_prelude + i) * n: n + (c.n_prelude + i + 1) * n], kv_max, cache,
                        None if last else self.W[f"prelude.{i + 1}.norm_1"], final_out=static_half,
                        final_rows=rows_d)
        ops.copy_rows(self.s0, self.pool, n=n, width=c.d_model, src_rows=pos_d, dst_rows=rows_d)
        for b, p in zip(seqs.tolist(), pos.tolist()):
            for i in range(c.n_prelude):
                cache.note_write(self.slot_prelude(i), b, p)
        return rows

    # -- R ---------------------------------------------------------------------------
    def core_union(self, cache, seqs, positions, steps) -> None:
        """One recurrence for n rows at their own depths: pool[row][:D] advances one step."""
        c = self.cfg
        seqs = np.asarray(seqs, dtype=np.int64)
        pos = np.asarray(positions, dtype=np.int64)
        st = np.asarray(steps, dtype=np.int64)
        n = len(pos)
        if n == 0:
            return
        self._check(cache, seqs, pos)
        if st.min() < 0 or st.max() >= c.T_total:
            raise ValueError(f"core step out of range [0, {c.T_total})")
        rows = seqs * self.R + pos % self.R
        slots = c.n_prelude + st[None, :] * c.n_core + np.arange(c.n_core, dtype=np.int64)[:, None]
        rb, fr = self._tables(cache, seqs, pos, slots)
        i32 = np.concatenate([pos, pos + 1, rows]).astype(np.int32)
        i64 = np.concatenate([rb.reshape(-1), fr.reshape(-1)])
        t32, t64 = self.staging.upload([i32, i64])
        pos_d, kvlen_d, rows_d = t32[:n], t32[n: 2 * n], t32[2 * n:]
        sc = self._ensure(n)
        kv_max = int(pos.max()) + 1
        ops.linear(self.pool, self.W["adapter"], n=n, x_rows=rows_d, out=sc["x"])
        ops.rmsnorm(sc["x"], self.W["core.0.norm_1"], c.norm_eps, n=n, x_out=sc["h"])
        L = c.n_core
        for l in range(L):
            last = l == L - 1
            self._block(f"core.{l}.", n, sc, pos_d, kvlen_d, t64[l * n: (l + 1) * n],
                        t64[(L + l) * n: (L + l + 1) * n], kv_max, cache,
                        None if last else self.W[f"core.{l + 1}.norm_1"], final_out=self.pool, final_rows=rows_d)
        for b, p, s in zip(seqs.tolist(), pos.tolist(), st.tolist()):
            for l in range(L):
                cache.note_write(self.slot_core(s, l), b, p)

    # -- C ---------------------------------------------------------------------------
    def coda_union(self, cache, seqs, positions) -> tuple[torch.Tensor, torch.Tensor]:
        """ln_f -> coda blocks -> ln_f -> lm_head for n rows. Returns
        (logits (n, V) float32, argmax ids (n,) int64), both device views."""
        c = self.cfg
        seqs = np.asarray(seqs, dtype=np.int64)
        pos = np.asarray(positions, dtype=np.int64)
        n = len(pos)
        self._check(cache, seqs, pos)
        rows = seqs * self.R + pos % self.R
        slots = self.coda_base + np.repeat(np.arange(c.n_coda, dtype=np.int64)[:, None], n, axis=1)
        rb, fr = self._tables(cache, seqs, pos, slots)
        i32 = np.concatenate([pos, pos + 1, rows]).astype(np.int32)
        i64 = np.concatenate([rb.reshape(-1), fr.reshape(-1)])
        t32, t64 = self.staging.upload([i32, i64])
        pos_d, kvlen_d, rows_d = t32[:n], t32[n: 2 * n], t32[2 * n:]
        self._ensure_logits(n)
        sc = self._ensure(n)
        kv_max = int(pos.max()) + 1
        ops.rmsnorm(self.pool, self.W["ln_f"], c.norm_eps, n=n, a_rows=rows_d, x_out=sc["x"])
        ops.rmsnorm(sc["x"], self.W["coda.0.norm_1"], c.norm_eps, n=n, x_out=sc["h"])
        L = c.n_coda
        for i in range(L):
            nxt = self.W[f"coda.{i + 1}.norm_1"] if i + 1 < L else self.W["ln_f"]
            self._block(f"coda.{i}.", n, sc, pos_d, kvlen_d, t64[i * n: (i + 1) * n],
                        t64[(L + i) * n: (L + i + 1) * n], kv_max, cache, nxt)
        logits = ops.linear(sc["h"], self.W["lm_head"], n=n, out=sc["logits"], out_dtype=torch.float32)
        ids = ops.argmax(logits, n=n, out=sc["ids"])
        for b, p in zip(seqs.tolist(), pos.tolist()):
            for i in range(L):
                cache.note_write(self.slot_coda(i), b, p)
        return logits[:n], ids[:n]

    # -- prefill -----------------------------------------------------------------------
    def prefill_seq(self, cache, b: int, token_ids) -> torch.Tensor:
        """Whole prompt of sequence b at positions [0, L): fills every slot's
        [0, L) and returns the last position's logits (V,) float32."""
        c, W = self.cfg, self.W
        ids = np.asarray(token_ids, dtype=np.int64).reshape(-1)
        L = len(ids)
        if L == 0 or L > cache.S:
            raise IndexError(f"prompt length {L} must be in [1, {cache.S}]")
        if not 0 <= b < cache.B:
            raise IndexError("sequence index out of range")
        D = c.d_model
        pos = np.arange(L, dtype=np.int64)
        seqs = np.full(L, b, dtype=np.int64)
        n_layers = c.n_prelude + c.T_total * c.n_core + c.n_coda
        slots = np.repeat(np.arange(n_layers, dtype=np.int64)[:, None], L, axis=1)
        rb, fr = self._tables(cache, seqs, pos, slots)
        t32, t64, ids_d = self.staging.upload([np.concatenate([pos, pos + 1]).astype(np.int32),
                                               np.concatenate([rb.reshape(-1), fr.reshape(-1)]), ids])
        pos_d, kvlen_d = t32[:L], t32[L:]
        rb_l = lambda s: t64[s * L: (s + 1) * L]  # noqa: E731
        fr_l = lambda s: t64[(n_layers + s) * L: (n_layers + s + 1) * L]  # noqa: E731
        self._ensure_logits(1)
        sc = self._ensure(L)
        state = torch.empty(L, 2 * D, dtype=self.dtype, device=self.device)  # [s | e] per prompt row
        ops.embed(ids_d, W["wte"], c.emb_scale, out=sc["x"])
        ops.rmsnorm(sc["x"], W["prelude.0.norm_1"], c.norm_eps, n=L, x_out=sc["h"])
        for i in range(c.n_prelude):
            last = i == c.n_prelude - 1
            self._block(f"prelude.{i}.", L, sc, pos_d, kvlen_d, rb_l(i), fr_l(i), L, cache,
                        None if last else W[f"prelude.{i + 1}.norm_1"], final_out=state[:, D:])
        s0 = initial_state_prefill(c, L, self.state_seed, self.state_init)
        state[:, :D].copy_(s0.to(device=self.device, dtype=self.dtype))
        for r in range(c.T_total):
            ops.linear(state, W["adapter"], n=L, out=sc["x"])
            ops.rmsnorm(sc["x"], W["core.0.norm_1"], c.norm_eps, n=L, x_out=sc["h"])
            for l in range(c.n_core):
                s = self.slot_core(r, l)
                last = l == c.n_core - 1
                self._block(f"core.{l}.", L, sc, pos_d, kvlen_d, rb_l(s), fr_l(s), L, cache,
                            None if last else W[f"core.{l + 1}.norm_1"], final_out=state[:, :D])
        ops.rmsnorm(state, W["ln_f"], c.norm_eps, n=L, x_out=sc["x"])
        ops.rmsnorm(sc["x"], W["coda.0.norm_1"], c.norm_eps, n=L, x_out=sc["h"])
        for i in range(c.n_coda):
            s = self.slot_coda(i)
            nxt = W[f"coda.{i + 1}.norm_1"] if i + 1 < c.n_coda else W["ln_f"]
            self._block(f"coda.{i}.", L, sc, pos_d, kvlen_d, rb_l(s), fr_l(s), L, cache, nxt)
        logits = ops.linear(sc["h"][L - 1: L], W["lm_head"], n=1, out=sc["logits"], out_dtype=torch.float32)
        for s in range(n_layers):
            cache.seqlen[s][b] = max(cache.seqlen[s][b], L)
        return logits[0].clone()
