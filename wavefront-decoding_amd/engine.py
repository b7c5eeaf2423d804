"""Device engine: the looped LM's P / R / C passes as fused libwfd launches.

One `LoopedModel` owns the device weights, the RoPE and initial-state (s0)
tables, the wave-state pool and preallocated scratch. A pass runs a *union*
of rows -- any mix of sequences, positions and loop depths -- through:

  prelude_union  wte*emb_scale -> prelude blocks      -> pool[row] = [s0(pos) | e]
  core_union     adapter(pool[row] = [s | e]) -> core blocks (slot by step) -> pool[row][:D]
  coda_union     ln_f(pool[row][:D]) -> coda blocks -> ln_f -> lm_head -> argmax
  prefill_seq    the same blocks over a whole prompt, every slot filled

and every decode block is: linear(Wqkv) with RoPE + cache append fused ->
attn_decode -> linear(proj) -> linear(fc, swiglu) -> linear(mlp_proj), each
residual add and the RMSNorm pair after it -- (norm_2, norm_3), then (norm_4,
the next norm_1) -- folded into the linears around it: the producing linear
(or, above 16 rows, the row kernel norm_prep) writes the residual stream and
the next linear's operand, and the consuming linear scales its rows (see
_prep). The prompt pass (prefill_seq) keeps separate add_rmsnorm launches.

Row tables (positions, slot row bases, append rows, pool rows) are built on
the host per call and read by the kernels as device data. Each row's
arithmetic is independent of the other rows in the union (every kernel is
row-invariant), so a token computed in a wavefront union is bit-identical to
the same token computed alone -- which is what makes wavefront decoding
lossless here.

hipGraph mode (use_graphs=True): each (pass, row bucket, cache) gets one
captured launch sequence over fixed scratch and fixed table buffers; a call
pads its rows to the bucket (a power of two up to 64, then a multiple of 64)
with rows that point at the cache's trash row and the pool's trash row,
refreshes the tables with one host->device copy, and replays. The grid bound for attention is the cache
length, so one graph serves every position, depth mix and rollback.

Wave-state pool: row of (seq b, position p) = b*R + p % R with
R = T_total + 2. At most T_total + 1 consecutive positions of one sequence
are in flight (a token enters only after its predecessor has advanced), so
live tokens never share a row, and a re-entered token after a rollback
reuses its position's row.
"""
from __future__ import annotations

import numpy as np
import torch

from . import _lib, ops
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


class _Captured:
    """One captured pass sequence: fixed device tables, a ring of pinned host
    copies, the graph.

    The device table buffer is baked into the graph; each replay is preceded by
    one host->device copy into it (stream-ordered behind the previous replay).
    The pinned source buffers rotate through a ring, each with an event recorded
    behind its copy, so the host can enqueue several replays ahead of the GPU
    and only waits when it laps the ring. Upload and launch are one native call
    (_tick.launch: event wait, pack, copy, event record, hipGraphLaunch)."""

    DEPTH = 8

    def __init__(self, kind: str, nb: int, cache, n32: int, n64: int, device, tick):
        self.kind, self.nb, self.cache, self.tick = kind, nb, cache, tick
        # one buffer [int64 tables | int32 tables] so a replay needs one host->device copy
        words = n64 + (n32 + 1) // 2
        self.host = [torch.empty(words, dtype=torch.int64).pin_memory() for _ in range(self.DEPTH)]
        self.host_ptr = [h.data_ptr() for h in self.host]
        index = device.index if device.index is not None else torch.cuda.current_device()
        self.events = [tick.event_create(index) for _ in range(self.DEPTH)]
        self.i = 0
        self.dev = torch.empty(words, dtype=torch.int64, device=device)
        self.n32, self.n64 = n32, n64
        self.d64 = self.dev[:n64]
        self.d32 = self.dev[n64:].view(torch.int32)[:n32]
        self.graph: torch.cuda.CUDAGraph | None = None
        self.exec = 0  # the graph's executable (raw handle) once captured

    def launch(self, t64: np.ndarray, t32: np.ndarray, stream: int, replay: bool = True,
               flags: tuple[int, int] = (0, 0)) -> None:
        """Upload the first n64 / n32 words of the host tables and replay the
        graph (replay=False: the upload only); flags = (host address, count)
        of accept flags to clear before the replay."""
        j = self.i
        self.i = (j + 1) % self.DEPTH
        self.tick.launch(self.exec if replay else 0, stream, self.events[j], self.host_ptr[j], self.dev.data_ptr(),
                         t64, self.n64, t32, self.n32, flags[0], flags[1])

    def __del__(self):
        for e in getattr(self, "events", ()):
            try:
                self.tick.event_destroy(e)
            except Exception:  # interpreter shutdown: the runtime may be gone
                pass


# weights read by the linear kernels (the rest -- embedding, norms -- stay plain)
_LINEAR_WEIGHTS = frozenset({"Wqkv", "proj", "fc", "mlp_proj", "adapter", "lm_head"})


# grouped attention only when at least this many (group, kv head) workgroups remain
_GROUP_MIN_WORKGROUPS = 256

# a C row's expected-token entry that asks for no comparison (below every ring handle)
NO_EXPECT = -(1 << 62)

# (min, max) rows of a d_model-output projection that runs split-K; up to 16
# rows one workgroup per tile already walks K in parallel (wide kernel)
_SPLIT_ROWS = (17, 512)


# rows up to which a linear runs as the few-row kernel (one workgroup walks all of K)
_FEW_ROWS = 16


def _few_row_linear(n: int, K: int, dtype: torch.dtype) -> bool:
    """Whether a linear over n rows and K inputs runs as the few-row kernel:
    n <= 16 and at most 3 chunks per sub-slice of the arithmetic contract."""
    kc = 128 if dtype == torch.bfloat16 else 64
    P = K // kc
    Q = (P + 3) // 4
    return n <= _FEW_ROWS and (Q + 3) // 4 <= 3


def _bucket(n: int) -> int:
    """Padded row count of a pass under graphs (one captured graph per
    count): powers of two up to 64, then multiples of 64, the many-row
    linears' row block -- a 150-row union runs 3 row blocks, not the 4 of a
    256-row bucket (padding rows cost the linears a whole block each; the
    attention skips them)."""
    if n > 64:
        return (n + 63) // 64 * 64
    b = 1
    while b < n:
        b *= 2
    return b


class LoopedModel:
    """Device-resident looped LM running unions of rows through libwfd."""

    def __init__(self, cfg: LoopedLMConfig, weights: dict[str, torch.Tensor], device="cuda", *, max_seq_len: int,
                 max_batch: int = 1, state_init: str = "random", state_seed: int = 0, use_graphs: bool = False,
                 max_rows: int | None = None, ring_len: int = 1 << 20, group_attention: bool = True,
                 dense_prompt: bool = True):
        self.cfg = cfg
        self.device = torch.device(device)
        self.dtype = cfg.torch_dtype
        if cfg.d_model > ops.fold_max_d(self.dtype):
            raise ValueError(f"{cfg.name}: d_model={cfg.d_model} is wider than the decode step's folded norm pairs "
                             f"take ({ops.fold_max_d(self.dtype)} for {self.dtype}: one wave holds a row)")
        self.max_seq_len = max_seq_len
        self.max_batch = max_batch
        self.state_init = state_init
        self.state_seed = state_seed
        self.use_graphs = use_graphs
        self.group_attention = group_attention  # rows sharing a slot read its prefix once
        self.group_min_workgroups = _GROUP_MIN_WORKGROUPS
        # row counts at which proj, the MLP down projection and the adapter run
        # split-K (linear_partials) with their K reduction in the next norm:
        # same bits as the one-launch linear, more workgroups per launch
        self.split_rows = _SPLIT_ROWS
        self.W = {}
        # the prompt pass (prefill_seq) runs its linears as plain library GEMMs
        # over row-major copies of the block weights: its rows are computed once
        # and never compared bit for bit with decode rows, and at hundreds to
        # tens of thousands of rows the library GEMM is 2-9x faster
        self.dense_prompt = dense_prompt
        self.Wd: dict[str, torch.Tensor] = {}
        for k, v in weights.items():
            w = v.to(device=self.device, dtype=self.dtype).contiguous()
            leaf = k.rsplit(".", 1)[-1]
            if leaf in _LINEAR_WEIGHTS:  # the kernels' packed layout
                if dense_prompt and leaf != "lm_head":
                    self.Wd[k] = w
                w = ops.pack_linear(w, swiglu=leaf == "fc")
            self.W[k] = w
        cos, sin = rope_tables(max_seq_len, cfg.head_dim, cfg.rope_base)
        self.rope_cos = cos.to(self.device)
        self.rope_sin = sin.to(self.device)
        self.s0 = initial_state_tokens(cfg, range(max_seq_len), state_seed, state_init).to(
            device=self.device, dtype=self.dtype)
        self._s0_prompt: torch.Tensor | None = None  # the prompt pass's s0 stream, see _prompt_s0
        self.R = cfg.T_total + 2
        D = cfg.d_model
        # pool rows: R per sequence + one trash row for padding rows
        self.pool = self._pitched(max_batch * self.R + 1, 2 * D, zero=True)
        self.trash_pool_row = max_batch * self.R
        self.coda_base = cfg.n_prelude + cfg.T_total * cfg.n_core
        k_mult = ops.linear_k_multiple(self.dtype)
        for K in (D, 2 * D, cfg.n_heads * cfg.head_dim, cfg.ffn):
            if K % k_mult:
                raise ValueError(f"{cfg.name}: K={K} is not a multiple of {k_mult} (linear kernel granularity)")
        # decode scratch: fixed capacity (captured graphs keep these addresses)
        self.max_rows = _bucket(max_rows or max_batch * self.R)
        self.sc = self._scratch(self.max_rows)
        # folded norm pairs (decode): the residual stream after proj (r1) and
        # after the MLP (r2), the next linear's operand A, the per-row scales
        # s_a kept for the residual (s1, s2), the precomputed row scales of
        # many-row launches, and the group sums a few-row producer leaves
        cap = self.max_rows
        self.sc["r1"] = torch.empty(cap, D, dtype=self.dtype, device=self.device)
        self.sc["r2"] = torch.empty(cap, D, dtype=self.dtype, device=self.device)
        self.sc["A"] = self._pitched(cap, D)
        f32 = lambda k: torch.zeros(k, dtype=torch.float32, device=self.device)  # noqa: E731
        self.sc["s1"], self.sc["s2"], self.sc["scale"] = f32(cap), f32(cap), f32(cap)
        self.sc["gpart"] = f32(_FEW_ROWS * ops.FOLD_SLOTS * 2)
        self.sc["logits"] = torch.empty(self.max_rows, cfg.vocab_size, dtype=torch.float32, device=self.device)
        self.sc["ids"] = torch.empty(self.max_rows, dtype=torch.int64, device=self.device)
        # column-group argmax bests of a few-row lm_head (at most 16 rows x N / 8 groups)
        self.sc["am_val"] = torch.empty(2 * cfg.vocab_size, dtype=torch.float32, device=self.device)
        self.sc["am_idx"] = torch.empty(2 * cfg.vocab_size, dtype=torch.int32, device=self.device)
        self.attn_ws = torch.zeros(ops.attn_workspace_bytes(self.max_rows, cfg.n_heads, cfg.head_dim, max_seq_len),
                                   dtype=torch.uint8, device=self.device)
        self.staging = _Staging(self.device)
        self._graphs: dict[tuple, _Captured] = {}
        # the native host side of a tick (row tables, upload, graph launch)
        self._tick = _lib.load_tick()
        self._flags_host, self._flags_dev = self._tick.host_alloc(4 * self.max_rows)
        self._dev_index = self.device.index if self.device.index is not None else torch.cuda.current_device()
        self._params: dict[tuple, tuple] = {}
        self._bytes_coef: dict[str, tuple[int, int, int]] = {}
        self._t_passes = 0
        self._t32 = self._t64 = None
        # device token ring: every C pass drops its argmax ids at host-allocated
        # slots; a token is then a handle -(slot + 1) until read back, and the P
        # pass embeds handles straight from the ring (no host round trip per
        # commit). The extra last slot absorbs padding rows.
        self.ring_len = ring_len
        self.tok_ring = torch.zeros(ring_len + 1, dtype=torch.int64, device=self.device)
        self._ring_next = 0
        self.last_c_handles: list[int] | None = None
        # greedy verify flags of the last C pass: the argmax kernel stores them
        # into mapped, coherent pinned host memory, which accept_flags() polls
        # (no device->host copy behind the graph); -1 until written. Every C
        # pass's argmax writes them; _flags_pending marks a C launch whose
        # writes may still be in flight (cleared by a read or a stream wait)
        self._accept_n = self._accept_nb = 0
        self._accept_unread = False
        self._flags_pending = False
        # algorithmic HBM bytes of every pass launched (see pass_bytes)
        self.bytes_moved = 0

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

    def clear_graphs(self) -> None:
        torch.cuda.synchronize()  # no upload may still read a pinned buffer about to be freed
        self._graphs.clear()

    # -- scratch -----------------------------------------------------------------
    def _pitched(self, rows: int, width: int, zero: bool = False) -> torch.Tensor:
        """A (rows, width) view whose row pitch is width + 64 bytes, for the
        buffers the packed linears read as x. Every workgroup of a linear reads
        the same x chunk at about the same time; at a pitch that is a multiple
        of 1 KB (d_model, 2 d_model, ffn) that chunk's rows sit on a few L2
        channels, and the 64-byte skew spreads them (linears at 64-256 rows
        10-25 % faster; a 128-byte skew gains nothing)."""
        pad = 64 // torch.empty(0, dtype=self.dtype).element_size()
        alloc = torch.zeros if zero else torch.empty
        return alloc(rows, width + pad, dtype=self.dtype, device=self.device)[:, :width]

    def _scratch(self, cap: int, dense: bool = False) -> dict[str, torch.Tensor]:
        c = self.cfg
        mk = lambda w: torch.empty(cap, w, dtype=self.dtype, device=self.device)  # noqa: E731
        sc = dict(x=mk(c.d_model), h=self._pitched(cap, c.d_model),
                  q=torch.empty(cap, c.n_heads, c.head_dim, dtype=self.dtype, device=self.device),
                  o=torch.empty(cap, c.n_heads, c.head_dim, dtype=self.dtype, device=self.device),
                  a=mk(c.d_model), u=self._pitched(cap, c.ffn), m=mk(c.d_model))
        # fp32 slice sums of the split-K projections (at most 4 slices)
        sc["part"] = torch.empty(4 * min(cap, self.split_rows[1]) * c.d_model, dtype=torch.float32,
                                 device=self.device)

        if dense:  # the library GEMMs' unfused outputs: q|k|v rows, gate|up rows
            sc["qkv"] = mk((c.n_heads + 2 * c.n_kv_heads) * c.head_dim)
            sc["gu"] = mk(2 * c.ffn)
        return sc

    # -- one SandwichBlock over n rows --------------------------------------------
    def _block(self, prefix: str, n: int, sc, pos_d, kvlen_d, rb_d, fr_d, kv_len_max: int, ws,
               cache: BatchStaticKVCache, next_norm: torch.Tensor | None, final_out=None, final_rows=None,
               segments=None, group_first=None, dense: bool = False):
        """One SandwichBlock over n rows. `segments` = (seg_row_base, seg_q_start,
        seg_pos0, max_seg_len) routes attention through the causal prefill
        kernel (rows grouped by slot at consecutive positions) instead of the
        per-row decode kernel; `group_first` groups decode rows that share a
        slot (one prefix read per group, same bits). `dense` (the prompt pass)
        runs the four linears as library GEMMs over the row-major weights, with
        the RoPE/append and SwiGLU epilogues as their own kernels."""
        c, W = self.cfg, self.W
        x, h = sc["x"], sc["h"]
        if dense:
            qkv = torch.mm(h[:n], self.Wd[prefix + "Wqkv"].t(), out=sc["qkv"][:n])
            q = ops.qkv_rope_append(qkv, pos_d, self.rope_cos, self.rope_sin, fr_d, cache.flat_k, cache.flat_v,
                                    c.n_heads, c.n_kv_heads, c.head_dim, q_out=sc["q"][:n])
        else:
            q = ops.linear_qkv_rope_append(h, W[prefix + "Wqkv"], pos_d, self.rope_cos, self.rope_sin, fr_d,
                                           cache.flat_k, cache.flat_v, c.n_heads, c.n_kv_heads, c.head_dim, n=n,
                                           q_out=sc["q"][:n])
        if segments is not None:
            srb, sqs, sp0, smax = segments
            o = ops.attn_prefill(q, cache.flat_k, cache.flat_v, srb, sqs, sp0, max_seg_len=smax, out=sc["o"][:n])
        else:
            o = ops.attn_decode(q, cache.flat_k, cache.flat_v, rb_d, kvlen_d, kv_len_max=kv_len_max,
                                out=sc["o"][:n], workspace=ws, group_first=group_first)
        if dense:
            a = torch.mm(o.view(n, -1), self.Wd[prefix + "proj"].t(), out=sc["a"][:n])
            ops.add_rmsnorm(a, W[prefix + "norm_2"], c.norm_eps, res=x, w2=W[prefix + "norm_3"], n=n, x_out=x,
                            h_out=h)
        else:
            self._linear_norm(o.view(n, -1), W[prefix + "proj"], n, sc, "a", W[prefix + "norm_2"], res=x,
                              w2=W[prefix + "norm_3"], x_out=x, h_out=h)
        if dense:
            gu = torch.mm(h[:n], self.Wd[prefix + "fc"].t(), out=sc["gu"][:n])
            u = ops.swiglu(gu, n=n, out=sc["u"][:n])
            m = torch.mm(u, self.Wd[prefix + "mlp_proj"].t(), out=sc["m"][:n])
            if next_norm is not None:
                ops.add_rmsnorm(m, W[prefix + "norm_4"], c.norm_eps, res=x, w2=next_norm, n=n, x_out=x, h_out=h)
            else:
                ops.add_rmsnorm(m, W[prefix + "norm_4"], c.norm_eps, res=x, n=n, x_out=final_out,
                                out_rows=final_rows)
        else:
            u = ops.linear(h, W[prefix + "fc"], n=n, out=sc["u"], swiglu=True)
            if next_norm is not None:
                self._linear_norm(u, W[prefix + "mlp_proj"], n, sc, "m", W[prefix + "norm_4"], res=x,
                                  w2=next_norm, x_out=x, h_out=h)
            else:
                self._linear_norm(u, W[prefix + "mlp_proj"], n, sc, "m", W[prefix + "norm_4"], res=x,
                                  x_out=final_out, out_rows=final_rows)

    def _linear_norm(self, xin: torch.Tensor, Wp, n: int, sc, tmp: str, w1: torch.Tensor, *, x_rows=None,
                     keep=None, **norm) -> None:
        """norm(linear(xin) [+ res]) for a d_model-output projection: split-K
        (slice sums, reduced inside the norm) for n in split_rows, else the
        linear into sc[tmp] then the norm -- the same bits either way. `keep`
        also receives the linear's output rows (the adapter's, which are the
        core block's residual)."""
        lo, hi = self.split_rows
        eps = self.cfg.norm_eps
        if lo <= n <= hi:
            S = ops.linear_partials(xin, Wp, sc["part"], n=n, x_rows=x_rows)
            ops.add_rmsnorm_split(sc["part"], S, n, w1, eps, dtype=self.dtype, a_out=keep, **norm)
        else:
            y = ops.linear(xin, Wp, n=n, x_rows=x_rows, out=keep if keep is not None else sc[tmp])
            ops.add_rmsnorm(y, w1, eps, n=n, **norm)

    # -- one SandwichBlock over n decode rows, norms folded into the linears ---------
    def _prep(self, xin: torch.Tensor, Wp, n: int, *, res, r_out: torch.Tensor, x_rows=None, wa=None, wb=None,
              s_slot=None, final=None):
        """A d_model-output linear (proj, the MLP down projection, the adapter)
        and what follows it: r = round(y + x_res) (res = (r, s, w) of the
        residual stream, or None), then either the next linear's operand
        A = round((r * wa) * wb) in sc["A"] -- returning (RowScale that
        linear reads, the residual stream the block adds next) -- or, with
        final = (out, rows, w), the block's last norm round((r * s) * w) into
        out[rows]. Few rows: the linear's own epilogue (linear_prep), r into
        r_out and the group sums (the next residual is (r_out, s_slot, wa),
        s_slot filled by the consumer). Many rows: split-K slices reduced by
        the row kernel (norm_prep), or the one-launch linear then norm_prep,
        which has s_a in hand and writes the normalized residual
        round((r * s_a) * wa) into r_out itself. The same bits in every form."""
        c, sc = self.cfg, self.sc
        D, eps = c.d_model, c.norm_eps
        r_in, s_in, w_in = res if res is not None else (None, None, None)
        fin = final is not None
        if fin:
            h_out, h_rows, wf = final
        if _few_row_linear(n, Wp.K, self.dtype):
            ops.linear_prep(xin, Wp, n=n, x_rows=x_rows, r_in=r_in, s_in=s_in, w_in=w_in, r_out=r_out,
                            a_out=sc["A"], wa=None if fin else wa, wb=wf if fin else wb, part=sc["gpart"])
            if fin:
                ops.norm_prep(n=n, D=D, dtype=self.dtype, eps=eps, a=r_out, wa=wf, h_out=h_out, h_rows=h_rows)
                return None
            return (ops.RowScale(D=D, eps=eps, two=wa is not None, part=sc["gpart"], s_out=s_slot),
                    (r_out, s_slot if wa is not None else None, wa))
        lo, hi = self.split_rows
        src = {}
        if lo <= n <= hi:
            S = ops.linear_partials(xin, Wp, sc["part"], n=n, x_rows=x_rows)
            src = dict(part=sc["part"], nslices=S)
        else:
            src = dict(a=ops.linear(xin, Wp, n=n, x_rows=x_rows, out=sc["a"]))
        if fin:
            ops.norm_prep(n=n, D=D, dtype=self.dtype, eps=eps, r_in=r_in, s_in=s_in, w_in=w_in, wa=wf,
                          h_out=h_out, h_rows=h_rows, **src)
            return None
        ops.norm_prep(n=n, D=D, dtype=self.dtype, eps=eps, r_in=r_in, s_in=s_in, w_in=w_in, a_out=sc["A"],
                      wa=wa, wb=wb, two=wa is not None, scale_out=sc["scale"], h_out=r_out, **src)
        return ops.RowScale(D=D, eps=eps, two=wa is not None, scale=sc["scale"]), (r_out, None, None)

    def _dblock(self, prefix: str, n: int, pos_d, kvlen_d, rb_d, fr_d, kv_len_max: int, cache, inp, res, nxt,
                final=None, group_first=None):
        """One SandwichBlock over n decode rows (huginn_blocks.py:93-103 norms
        and residuals) with its four RMSNorms folded into the linears:
        `inp` is the RowScale of the operand in sc["A"] (None: the plain
        normalized rows in sc["h"]), `res` the residual stream (r, s, w) the
        block adds (s, w None: raw). Returns (inp, res) for the next block --
        the pair (norm_4, nxt) -- or, with final = (out, rows), writes
        norm_4's output there and returns (None, None)."""
        c, W, sc = self.cfg, self.W, self.sc
        xq = sc["h"] if inp is None else sc["A"]
        q = ops.linear_qkv_rope_append(xq, W[prefix + "Wqkv"], pos_d, self.rope_cos, self.rope_sin, fr_d,
                                       cache.flat_k, cache.flat_v, c.n_heads, c.n_kv_heads, c.head_dim, n=n,
                                       q_out=sc["q"][:n], rowscale=inp)
        o = ops.attn_decode(q, cache.flat_k, cache.flat_v, rb_d, kvlen_d, kv_len_max=kv_len_max, out=sc["o"][:n],
                            workspace=self.attn_ws, group_first=group_first)
        rs, mid = self._prep(o.view(n, -1), W[prefix + "proj"], n, res=res, r_out=sc["r1"],
                             wa=W[prefix + "norm_2"], wb=W[prefix + "norm_3"], s_slot=sc["s1"])
        u = ops.linear(sc["A"], W[prefix + "fc"], n=n, out=sc["u"], swiglu=True, rowscale=rs)
        if final is not None:
            self._prep(u, W[prefix + "mlp_proj"], n, res=mid, r_out=sc["r2"], final=(*final, W[prefix + "norm_4"]))
            return None, None
        return self._prep(u, W[prefix + "mlp_proj"], n, res=mid, r_out=sc["r2"], wa=W[prefix + "norm_4"], wb=nxt,
                          s_slot=sc["s2"])

    # -- row tables ------------------------------------------------------------------
    def _layers(self, kind: str) -> int:
        c = self.cfg
        return {"P": c.n_prelude, "R": c.n_core, "C": c.n_coda}[kind]

    def _launch(self, kind: str, cache, nb: int, t32: torch.Tensor, t64: torch.Tensor, kv_max: int,
                grouped: bool = False) -> None:
        """The launch sequence of one pass over nb rows (eager or under capture)."""
        c, W, sc, ws = self.cfg, self.W, self.sc, self.attn_ws
        pos_d, kvlen_d, rows_d = t32[:nb], t32[nb: 2 * nb], t32[2 * nb: 3 * nb]
        nblk = 4 if kind == "C" else 3
        gf = t32[nblk * nb: nblk * nb + nb + 1] if grouped else None
        L = self._layers(kind)
        off = nb if kind == "P" else 0
        rb = lambda l: t64[off + l * nb: off + (l + 1) * nb]  # noqa: E731
        fr = lambda l: t64[off + (L + l) * nb: off + (L + l + 1) * nb]  # noqa: E731
        blk = lambda pre, l, inp, res, nxt, final=None: self._dblock(  # noqa: E731
            pre, nb, pos_d, kvlen_d, rb(l), fr(l), kv_max, cache, inp, res, nxt, final=final, group_first=gf)
        if kind == "P":
            # embed -> x (the first prelude block's raw residual), prelude.0.norm_1
            # -> h, and each token's initial loop state s0[pos] into its
            # wave-state row (the prelude below writes only the row's static half)
            ops.embed_rmsnorm(t64[:nb], W["wte"], c.emb_scale, W["prelude.0.norm_1"], c.norm_eps, h_out=sc["h"],
                              x_out=sc["x"], ring=self.tok_ring, n=nb,
                              copy=(self.s0, pos_d, self.pool, rows_d, c.d_model))
            inp, res = None, (sc["x"], None, None)
            for i in range(L):
                last = i + 1 == L
                inp, res = blk(f"prelude.{i}.", i, inp, res, None if last else W[f"prelude.{i + 1}.norm_1"],
                               final=(self.pool[:, c.d_model:], rows_d) if last else None)
        elif kind == "R":
            # adapter(cat[s, e]) -> the first core block's raw residual, with
            # core.0.norm_1 folded into its Wqkv
            inp, res = self._prep(self.pool, W["adapter"], nb, x_rows=rows_d, res=None, r_out=sc["r2"],
                                  wb=W["core.0.norm_1"])
            for l in range(L):
                last = l + 1 == L
                inp, res = blk(f"core.{l}.", l, inp, res, None if last else W[f"core.{l + 1}.norm_1"],
                               final=(self.pool, rows_d) if last else None)
        else:
            # ln_f -> x (the first coda block's raw residual), coda.0.norm_1 -> h
            ops.add_rmsnorm(self.pool, W["ln_f"], c.norm_eps, w2=W["coda.0.norm_1"], n=nb, a_rows=rows_d,
                            x_out=sc["x"], h_out=sc["h"])
            inp, res = None, (sc["x"], None, None)
            for i in range(L):
                inp, res = blk(f"coda.{i}.", i, inp, res, W[f"coda.{i + 1}.norm_1"] if i + 1 < L else W["ln_f"])
            # lm_head reads the last block's (norm_4, ln_f) pair
            am = dict(out=sc["ids"], ring=self.tok_ring, ring_rows=t32[3 * nb: 4 * nb],
                      expect=t64[2 * L * nb: 2 * L * nb + nb], accept_mapped=(self._flags_dev, self.max_rows))
            G = ops.linear_argmax_groups(nb, W["lm_head"]) if W["lm_head"].dtype == torch.bfloat16 else 0
            if G > 0:  # few rows: the argmax reads each 16-column group's best, not the whole vocabulary
                ops.linear_argmax(sc["A"], W["lm_head"], n=nb, out=sc["logits"], part_val=sc["am_val"],
                                  part_idx=sc["am_idx"], rowscale=inp)
                ops.argmax_groups(sc["am_val"], sc["am_idx"], G, n=nb, **am)
            else:
                ops.linear(sc["A"], W["lm_head"], n=nb, out=sc["logits"], out_dtype=torch.float32, rowscale=inp)
                ops.argmax(sc["logits"], n=nb, **am)

    # -- a tick: row tables, upload, launch -------------------------------------------
    def _tick_params(self, cache) -> tuple:
        """The constants _tick.plan_pass reads (one tuple per cache shape and
        grouping setting)."""
        key = (cache.B, cache.S, cache.trash_row, self.use_graphs, self.group_attention, self.group_min_workgroups)
        prm = self._params.get(key)
        if prm is None:
            c = self.cfg
            prm = (cache.B, cache.S, cache.trash_row, self.R, self.trash_pool_row, c.n_prelude, c.n_core, c.n_coda,
                   c.T_total, self.coda_base, self.ring_len, self.max_batch, self.max_seq_len, self.max_rows,
                   int(self.use_graphs), int(self.group_attention),
                   ops.attn_group_max_rows(c.n_heads, c.n_kv_heads), self.group_min_workgroups, c.n_kv_heads)
            assert len(prm) == self._tick.NUM_PARAMS
            self._params[key] = prm
        return prm

    def _table_scratch(self, passes: int) -> tuple[np.ndarray, np.ndarray]:
        """Host scratch for the tables of `passes` passes (int32, int64), grown on demand."""
        if passes > self._t_passes:
            c, nb = self.cfg, self.max_rows
            lmax = max(c.n_prelude, c.n_core, c.n_coda)
            self._t32 = np.zeros(passes * (5 * nb + 1), dtype=np.int32)
            self._t64 = np.zeros(passes * (2 + 2 * lmax) * nb, dtype=np.int64)
            self._t_passes = passes
        return self._t32, self._t64

    def _launch_plans(self, cache, plans, t32: torch.Tensor, t64: torch.Tensor, kv_max: int | None = None) -> None:
        """Launch the passes in order, each on its slice of the joint tables."""
        o32 = o64 = 0
        for p in plans:
            self._launch(p["kind"], cache, p["nb"], t32[o32: o32 + p["n32"]], t64[o64: o64 + p["n64"]],
                         kv_max if kv_max is not None else p["kv_max"], p["grouped"])
            o32 += p["n32"]
            o64 += p["n64"]

    def _captured(self, cache, plans) -> _Captured:
        """The graph of a pass sequence: one per (cache, [(kind, bucket, grouped)])."""
        key = (id(cache),) + tuple((p["kind"], p["nb"], p["grouped"]) for p in plans)
        g = self._graphs.get(key)
        if g is not None and g.cache is cache:
            return g
        prm = self._tick_params(cache)
        n32 = sum(p["n32"] for p in plans)
        n64 = sum(p["n64"] for p in plans)
        pad32, pad64 = np.zeros(n32, dtype=np.int32), np.zeros(n64, dtype=np.int64)
        o32 = o64 = 0
        for p in plans:  # the same shapes with every row a padding row (and every grouped row its own group)
            _, m32, m64, _, _, _ = self._tick.plan_pass(pad32, o32, pad64, o64, prm, p["kind"], [], [],
                                                        None if p["kind"] == "C" else [], p["nb"],
                                                        int(p["grouped"]), -1)
            o32 += m32
            o64 += m64
        g = _Captured("+".join(p["kind"] for p in plans), plans[0]["nb"], cache, n32, n64, self.device, self._tick)
        g.launch(pad64, pad32, self._raw_stream(), replay=False)
        torch.cuda.synchronize()
        self._launch_plans(cache, plans, g.d32, g.d64, cache.S)                   # warm-up, then capture
        torch.cuda.synchronize()
        g.graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g.graph):
            self._launch_plans(cache, plans, g.d32, g.d64, cache.S)
        torch.cuda.synchronize()
        g.exec = g.graph.raw_cuda_graph_exec()
        self._graphs[key] = g
        return g

    # -- traffic accounting ------------------------------------------------------------
    def _raw_stream(self) -> int:
        """Handle of torch's current stream on the engine's device (the stream
        every launch of the engine is ordered on)."""
        return torch._C._cuda_getCurrentRawStream(self._dev_index)

    def _bytes_terms(self, kind: str) -> tuple[int, int, int]:
        """pass_bytes = fixed + per_row * n + per_key * (keys read), keys read =
        sum over rows of position + 1."""
        t = self._bytes_coef.get(kind)
        if t is None:
            c = self.cfg
            el = torch.empty(0, dtype=self.dtype).element_size()
            D, F, Hd, Kd = c.d_model, c.ffn, c.n_heads * c.head_dim, c.n_kv_heads * c.head_dim
            L = self._layers(kind)
            fixed = L * (c.qkv_dim * D + D * Hd + 2 * F * D + D * F + 4 * D) * el
            # per row: its K/V append; Wqkv x -> q; attention q -> o; proj o -> a;
            # norm (a, x) -> (x, h); fc h -> u; mlp_proj u -> m; norm (m, x) -> (x, h)
            per_row = L * (2 * Kd + 12 * D + 4 * Hd + 2 * F) * el
            per_key = L * 2 * Kd * el
            if kind == "P":
                per_row += 4 * D * el  # embedding row, pool row written (2 D), s0 row
            elif kind == "R":
                fixed += 2 * D * D * el  # adapter weights
                per_row += 3 * D * el    # its x rows and output
            else:
                fixed += (c.vocab_size * D + D) * el  # lm_head, ln_f
                per_row += D * el + c.vocab_size * 4 + 8  # the final norm's row, logits, ids
            t = self._bytes_coef[kind] = (fixed, per_row, per_key)
        return t

    def pass_bytes(self, kind: str, positions) -> int:
        """Algorithmic HBM bytes of one pass over rows at `positions`: every
        weight byte of its layers once (plus the embedding rows for P, the
        adapter for R, ln_f and lm_head for C), each row's slot prefix (K and V
        of keys [0, position]) per layer, its K/V append, and the activation
        rows the layers read and write (x into each linear, its output, the
        norms' inputs and outputs). Padding rows of a captured launch are not
        counted: they are not part of the work."""
        fixed, per_row, per_key = self._bytes_terms(kind)
        n = len(positions)
        return int(fixed + per_row * n + per_key * sum(int(p) + 1 for p in positions))

    # -- P / R / C ---------------------------------------------------------------------
    def _note_writes(self, cache, kind: str, seqs, pos, extra) -> None:
        """The slot lengths the pass's appends extend (the cache's note_write
        per (slot, row), positions already validated)."""
        c = self.cfg
        if kind == "R":
            first = [c.n_prelude + int(s) * c.n_core for s in extra]
            cache.note_writes(first, c.n_core, seqs, pos)
        elif kind == "P":
            cache.note_writes(self.slot_prelude(0), c.n_prelude, seqs, pos)
        else:
            cache.note_writes(self.slot_coda(0), c.n_coda, seqs, pos)

    def run_passes(self, cache, passes) -> tuple[torch.Tensor, torch.Tensor] | None:
        """Several passes as one launch sequence -- one graph replay and one
        table upload -- in order: passes = [(kind, seqs, positions, extra)],
        kind "P" (extra = token ids or ring handles), "R" (extra = steps) or
        "C" (extra = None, or per row the token expected from its argmax -- a
        plain id, a ring handle, or NO_EXPECT -- for a device-side greedy
        verify whose flags `accept_flags()` returns; at most one C, last). A
        scheduler tick (P, R, C) or a whole sequential token (P, T_total x R,
        C) then costs one replay. Every pass is validated and tabled (natively,
        _tick.plan_pass) before anything launches; the slot-length bookkeeping
        and the traffic count run after the launch, while the GPU works.
        Returns what coda_union returns for the C pass, else None."""
        tick = self._tick
        prm = self._tick_params(cache)
        t32, t64 = self._table_scratch(len(passes))
        plans, live, n_c, c_base, c_expect = [], [], 0, -1, False
        o32 = o64 = 0
        last = passes[-1][0] if passes else None
        for kind, seqs, positions, extra in passes:
            n = len(positions)
            if n == 0:
                continue
            if kind == "C":
                if last != "C":
                    raise ValueError("the C pass must come last")
                c_base = self._ring_next if self._ring_next + n <= self.ring_len else -1
            nb, n32, n64, grouped, kv_max, psum = tick.plan_pass(t32, o32, t64, o64, prm, kind, seqs, positions,
                                                                 extra, -1, -1, c_base if kind == "C" else -1)
            plans.append(dict(kind=kind, nb=nb, grouped=grouped, kv_max=kv_max, n32=n32, n64=n64))
            live.append((kind, seqs, positions, extra, n, psum))
            o32 += n32
            o64 += n64
            if kind == "C":
                n_c = n
                c_expect = extra is not None and len(extra) > 0
        # a C pass with expected tokens clears the flags its argmax will write
        # (one per row, padding included); if an earlier C launch may still be
        # writing them (its flags were never read), wait for it first
        nflags = plans[-1]["nb"] if n_c and c_expect else 0
        if nflags and self._flags_pending:
            torch.cuda.current_stream(self.device).synchronize()
            self._flags_pending = False
        if plans:
            if self.use_graphs:
                self._captured(cache, plans).launch(t64, t32, self._raw_stream(), flags=(self._flags_host, nflags))
            else:
                if nflags:
                    self._tick.clear_flags(self._flags_host, nflags)
                d32, d64 = self.staging.upload([t32[:o32], t64[:o64]])
                self._launch_plans(cache, plans, d32, d64)
        if n_c and c_base >= 0:
            self._ring_next = c_base + n_c
        for kind, seqs, positions, extra, n, psum in live:
            fixed, per_row, per_key = self._bytes_terms(kind)
            self.bytes_moved += fixed + per_row * n + per_key * (psum + n)
            self._note_writes(cache, kind, seqs, positions, extra)
        if n_c:
            self.last_c_handles = None if c_base < 0 else [-(c_base + i) - 1 for i in range(n_c)]
            self._accept_n, self._accept_nb = n_c, plans[-1]["nb"]
            self._accept_unread, self._flags_pending = c_expect, True
            return self.sc["logits"][:n_c], self.sc["ids"][:n_c]
        return None

    def accept_flags(self, timeout_s: float = 30.0) -> list[bool]:
        """The greedy verify flags of the last C pass (one per C row; False
        for rows that asked for no comparison): polls the mapped flag buffer
        until the pass's argmax has written every flag. Only after a C pass
        that carried expected tokens, once."""
        if not self._accept_unread:
            raise RuntimeError("the last C pass carried no expected tokens, or its flags were already read")
        # every row's flag, padding rows' included: then no workgroup of this
        # argmax is left to store one after the next pass clears them
        flags = self._tick.wait_flags(self._flags_host, self._accept_nb, timeout_s)
        if flags is None:  # still unwritten: wait for the stream, then read once more
            torch.cuda.current_stream(self.device).synchronize()
            flags = self._tick.wait_flags(self._flags_host, self._accept_nb, 0.0)
            if flags is None:
                raise RuntimeError("the C pass finished without writing its accept flags")
        self._accept_unread = self._flags_pending = False
        return flags[: self._accept_n]

    def __del__(self):
        host = getattr(self, "_flags_host", 0)
        if host:
            try:  # no kernel may still write the flags when they are freed
                torch.cuda.synchronize(self.device)
                self._tick.host_free(host)
            except Exception:  # interpreter shutdown: the runtime may be gone
                pass
            self._flags_host = 0

    def prelude_union(self, cache, seqs, positions, token_ids) -> np.ndarray:
        """Embed + prelude blocks for n new tokens; fills pool[row] = [s0(pos) | e].
        Returns the pool rows."""
        seqs = np.asarray(seqs, dtype=np.int64)
        pos = np.asarray(positions, dtype=np.int64)
        if len(pos) == 0:
            return np.zeros(0, dtype=np.int64)
        self.run_passes(cache, [("P", seqs, pos, token_ids)])
        return seqs * self.R + pos % self.R

    def core_union(self, cache, seqs, positions, steps) -> None:
        """One recurrence for n rows at their own depths: pool[row][:D] advances one step."""
        self.run_passes(cache, [("R", seqs, positions, steps)])

    def coda_union(self, cache, seqs, positions) -> tuple[torch.Tensor, torch.Tensor]:
        """ln_f -> coda blocks -> ln_f -> lm_head -> argmax for n rows. Returns
        (logits (n, V) float32, argmax ids (n,) int64), both device views that
        the next call overwrites. The ids also land in the token ring:
        `last_c_handles` lists their handles (None when the ring is full)."""
        out = self.run_passes(cache, [("C", seqs, positions, None)])
        if out is None:  # empty union
            self.last_c_handles = []
            return self.sc["logits"][:0], self.sc["ids"][:0]
        return out

    # -- token ring --------------------------------------------------------------------
    def reset_token_ring(self) -> None:
        """Start handing out ring slots from 0 (handles of earlier calls become invalid)."""
        self._ring_next = 0

    def resolve_tokens(self, values) -> list[int]:
        """Token ids for a mix of plain ids (>= 0) and ring handles (< 0); one
        device->host read of the used part of the ring."""
        values = list(values)
        slots = [-v - 1 for v in values if v < 0]
        if not slots:
            return values
        host = self.tok_ring[: max(slots) + 1].cpu().numpy()
        return [int(host[-v - 1]) if v < 0 else v for v in values]

    # -- prefill -----------------------------------------------------------------------
    def _prompt_s0(self, L: int) -> torch.Tensor:
        """Rows [0, L) of the prompt pass's initial loop state, on the device.
        It is one stream for every prompt (model.initial_state_prefill), and
        its generator fills rows in order, so rows [0, L) of a longer draw are
        the draw of length L (tested): the stream is drawn once for the longest
        prompt so far (at least doubling) and sliced, not redrawn on the host
        for every prompt."""
        t = self._s0_prompt
        if t is None or t.shape[0] < L:
            n = max(L, min(2 * (0 if t is None else t.shape[0]), self.max_seq_len))
            t = initial_state_prefill(self.cfg, n, self.state_seed, self.state_init).to(device=self.device,
                                                                                        dtype=self.dtype)
            self._s0_prompt = t
        return t[:L]

    def prefill_seq(self, cache, b: int, token_ids) -> torch.Tensor:
        """Whole prompt of sequence b at positions [0, L): fills every slot's
        [0, L) and returns the last position's logits (V,) float32. Runs eagerly
        with its own L-row scratch; with dense_prompt its linears are library
        GEMMs (see __init__), the last position's lm_head row the packed kernel."""
        c, W = self.cfg, self.W
        ids = np.asarray(token_ids, dtype=np.int64).reshape(-1)
        L = len(ids)
        if L == 0 or L > cache.S:
            raise IndexError(f"prompt length {L} must be in [1, {cache.S}]")
        if not 0 <= b < cache.B:
            raise IndexError("sequence index out of range")
        D = c.d_model
        pos = np.arange(L, dtype=np.int64)
        n_layers = c.n_prelude + c.T_total * c.n_core + c.n_coda
        base = (np.arange(n_layers, dtype=np.int64) * cache.B + b) * cache.S  # slot row base per layer slot
        rb = np.repeat(base[:, None], L, axis=1)
        fr = rb + pos[None, :]
        t32, t64, ids_d = self.staging.upload([np.concatenate([pos, pos + 1, [0, L, 0]]).astype(np.int32),
                                               np.concatenate([rb.reshape(-1), fr.reshape(-1), base]), ids])
        pos_d, kvlen_d = t32[:L], t32[L:2 * L]
        rb_l = lambda s: t64[s * L: (s + 1) * L]  # noqa: E731
        fr_l = lambda s: t64[(n_layers + s) * L: (n_layers + s + 1) * L]  # noqa: E731
        # bf16: the whole prompt of a slot is one causal segment for the MFMA
        # prefill kernel; fp32 keeps the per-row decode kernel
        flash = self.dtype == torch.bfloat16 and c.head_dim in (64, 128)
        seg_l = (lambda s: (t64[2 * n_layers * L + s: 2 * n_layers * L + s + 1], t32[2 * L: 2 * L + 2],  # noqa: E731
                            t32[2 * L + 2: 2 * L + 3], L)) if flash else (lambda s: None)
        dense = self.dense_prompt
        sc = self._scratch(L, dense=dense)
        ws = None if flash else torch.zeros(ops.attn_workspace_bytes(L, c.n_heads, c.head_dim, L),
                                            dtype=torch.uint8, device=self.device)
        logits = torch.empty(1, c.vocab_size, dtype=torch.float32, device=self.device)
        state = self._pitched(L, 2 * D)  # [s | e] per prompt row
        ops.embed(ids_d, W["wte"], c.emb_scale, out=sc["x"])
        ops.rmsnorm(sc["x"], W["prelude.0.norm_1"], c.norm_eps, n=L, x_out=sc["h"])
        for i in range(c.n_prelude):
            nxt = W[f"prelude.{i + 1}.norm_1"] if i + 1 < c.n_prelude else None
            self._block(f"prelude.{i}.", L, sc, pos_d, kvlen_d, rb_l(i), fr_l(i), L, ws, cache, nxt,
                        final_out=state[:, D:], segments=seg_l(i), dense=dense)
        state[:, :D].copy_(self._prompt_s0(L))
        for r in range(c.T_total):
            if dense:
                torch.mm(state, self.Wd["adapter"].t(), out=sc["x"][:L])
            else:
                ops.linear(state, W["adapter"], n=L, out=sc["x"])
            ops.rmsnorm(sc["x"], W["core.0.norm_1"], c.norm_eps, n=L, x_out=sc["h"])
            for l in range(c.n_core):
                s = self.slot_core(r, l)
                nxt = W[f"core.{l + 1}.norm_1"] if l + 1 < c.n_core else None
                self._block(f"core.{l}.", L, sc, pos_d, kvlen_d, rb_l(s), fr_l(s), L, ws, cache, nxt,
                            final_out=state[:, :D], segments=seg_l(s), dense=dense)
        ops.add_rmsnorm(state, W["ln_f"], c.norm_eps, w2=W["coda.0.norm_1"], n=L, x_out=sc["x"], h_out=sc["h"])
        for i in range(c.n_coda):
            s = self.slot_coda(i)
            nxt = W[f"coda.{i + 1}.norm_1"] if i + 1 < c.n_coda else W["ln_f"]
            self._block(f"coda.{i}.", L, sc, pos_d, kvlen_d, rb_l(s), fr_l(s), L, ws, cache, nxt, segments=seg_l(s),
                        dense=dense)
        ops.linear(sc["h"][L - 1: L], W["lm_head"], n=1, out=logits, out_dtype=torch.float32)
        for s in range(n_layers):
            cache.seqlen[s][b] = max(cache.seqlen[s][b], L)
        return logits[0]
