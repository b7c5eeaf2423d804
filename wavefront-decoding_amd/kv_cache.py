"""Per-depth slot KV caches over one flat device buffer.

Keeps the reference's invariant -- buffer index == absolute position, one
K/V buffer per (slot, sequence) -- and its slot numbering (prelude i -> i;
core step r layer l -> n_prelude + r*n_core + l; coda i ->
n_prelude + T_total*n_core + i; src/decoding/kv_cache.py:8-22,
huginn_blocks_batch.py:90-100). What changes is the storage: all slots of
all sequences live in one contiguous buffer per K and V, so the decode kernel
reads any slot prefix in place from (row_base, kv_len) tables instead of
gathering and concatenating copies (the pack of batch_kv_cache.py:75-96 /
parcae_blocks.py:458-466 is gone).

Flat row of (slot, seq b, pos) = (slot*B + b)*S + pos
(src/decoding/batch_kv_cache.py:64-65). Layout of the buffers:
  head_major=True (default): (n_slots*B + 1, Hkv, S, Dh) -- one block of S rows
      per (slot, sequence), each head's positions contiguous, so attention
      streams one contiguous run per (query, head);
  head_major=False: (n_slots*B*S + 1, Hkv, Dh) -- token-major, the reference's
      per-slot (S, Hkv, Dh) buffers laid end to end.
`K` / `V` are (n_slots, B, S, Hkv, Dh) views of either layout.

Rollback only truncates the logical lengths (kv_cache.py:158-165,
batch_kv_cache.py:99-105): every read is bounded by the reading query's own
position, so stale rows past a rolled-back length are never read and are
overwritten by the next append at that position.
"""
from __future__ import annotations

import torch

from . import ops


class BatchStaticKVCache:
    """Flat per-(slot, sequence) cache; mirrors src/decoding/batch_kv_cache.py:29-105."""

    def __init__(self, n_slots: int, batch_size: int, n_kv_head: int, head_dim: int, max_seq_len: int,
                 dtype: torch.dtype, device, *, head_major: bool = True):
        self.n_slots = n_slots
        self.B = batch_size
        self.S = max_seq_len
        self.n_kv_head = n_kv_head
        self.head_dim = head_dim
        self.dtype = dtype
        self.device = torch.device(device)
        self.head_major = head_major
        nblk = n_slots * batch_size
        rows = nblk * max_seq_len
        # zero-filled like the reference, so a clamped read never sees NaN garbage;
        # one extra trailing "trash" row (a whole block when head-major) absorbs
        # the appends of padding rows of a captured (fixed-width) launch and is
        # never part of any slot.
        if head_major:
            shape = (nblk + 1, n_kv_head, max_seq_len, head_dim)
            self.flat_k = torch.zeros(shape, dtype=dtype, device=self.device)
            self.flat_v = torch.zeros(shape, dtype=dtype, device=self.device)
            view = lambda t: t[:nblk].view(n_slots, batch_size, n_kv_head, max_seq_len,  # noqa: E731
                                           head_dim).permute(0, 1, 3, 2, 4)
        else:
            self.flat_k = torch.zeros(rows + 1, n_kv_head, head_dim, dtype=dtype, device=self.device)
            self.flat_v = torch.zeros(rows + 1, n_kv_head, head_dim, dtype=dtype, device=self.device)
            view = lambda t: t[:rows].view(n_slots, batch_size, max_seq_len, n_kv_head, head_dim)  # noqa: E731
        self.trash_row = rows
        self.K = view(self.flat_k)
        self.V = view(self.flat_v)
        # logical per-(slot, seq) lengths: bookkeeping and bounds checks only
        self.seqlen = [[0] * batch_size for _ in range(n_slots)]

    # -- indexing -----------------------------------------------------------
    def row_base(self, slot: int, b: int) -> int:
        return (slot * self.B + b) * self.S

    def flat_row(self, slot: int, b: int, pos: int) -> int:
        return (slot * self.B + b) * self.S + pos

    @property
    def nbytes(self) -> int:
        return 2 * self.K.numel() * self.K.element_size()

    def check_position(self, pos: int) -> None:
        if pos < 0 or pos >= self.S:
            raise IndexError(f"position {pos} exceeds max_seq_len={self.S}")

    def note_write(self, slot: int, b: int, pos: int) -> None:
        self.check_position(pos)
        if pos + 1 > self.seqlen[slot][b]:
            self.seqlen[slot][b] = pos + 1

    def note_writes(self, first_slot, n_slots: int, seq_ids, positions) -> None:
        """note_write for slots first_slot .. first_slot + n_slots - 1 of every
        row (first_slot: one int, or one per row), positions already checked."""
        seqlen = self.seqlen
        firsts = [first_slot] * len(positions) if isinstance(first_slot, int) else first_slot
        for s0, b, p in zip(firsts, seq_ids, positions):
            v = int(p) + 1
            for row in seqlen[s0: s0 + n_slots]:
                if row[b] < v:
                    row[b] = v

    # -- reference API --------------------------------------------------------
    def write_prefill(self, slot: int, k: torch.Tensor, v: torch.Tensor, seq_ids=None) -> None:
        """k, v: (B', L, Hkv, Dh) prompt K/V at positions [0, L) of `slot` for
        sequences `seq_ids` (default: all B)."""
        L = k.shape[1]
        if L > self.S:
            raise IndexError(f"prefill length {L} exceeds max_seq_len={self.S}")
        seq_ids = list(range(self.B)) if seq_ids is None else list(seq_ids)
        rows = torch.tensor([self.flat_row(slot, b, p) for b in seq_ids for p in range(L)], dtype=torch.int64,
                            device=self.device)
        ops.kv_append(k.reshape(-1, self.n_kv_head, self.head_dim).contiguous(),
                      v.reshape(-1, self.n_kv_head, self.head_dim).contiguous(), self.flat_k, self.flat_v, rows)
        for b in seq_ids:
            self.seqlen[slot][b] = max(self.seqlen[slot][b], L)

    def write_tokens(self, slots, seq_ids, positions, k: torch.Tensor, v: torch.Tensor) -> None:
        """Scatter n tokens: k, v (n, Hkv, Dh) -> (slots[i], seq_ids[i], positions[i])."""
        for sl, b, p in zip(slots, seq_ids, positions):
            self.note_write(sl, b, p)
        rows = torch.tensor([self.flat_row(sl, b, p) for sl, b, p in zip(slots, seq_ids, positions)],
                            dtype=torch.int64, device=self.device)
        ops.kv_append(k.contiguous(), v.contiguous(), self.flat_k, self.flat_v, rows)

    def gather_pack(self, slots, seq_ids, uptos):
        """Compatibility form of the reference pack (batch_kv_cache.py:75-96):
        copies the n prefixes [0, upto_i] into contiguous K/V + int32 cu_k. The
        decode path never calls it -- the kernel reads the slots in place."""
        lengths = [u + 1 for u in uptos]
        cu = [0]
        for ln in lengths:
            cu.append(cu[-1] + ln)
        pack = lambda t: torch.cat([t[sl, b, :ln] for sl, b, ln in zip(slots, seq_ids, lengths)])  # noqa: E731
        return (pack(self.K), pack(self.V), torch.tensor(cu, dtype=torch.int32, device=self.device), max(lengths))

    def drop_positions_at_and_after(self, b: int, position: int) -> None:
        """Per-sequence rollback: truncate sequence b's logical lengths only."""
        for row in self.seqlen:  # on the host's path from a reject to the next launch
            if row[b] > position:
                row[b] = position

    def reset_lengths(self) -> None:
        """Forget every sequence (buffers are reused as they are; reads are
        bounded by the reading query's position, so stale rows are never read)."""
        self.seqlen = [[0] * self.B for _ in range(self.n_slots)]


class StaticKVCache(BatchStaticKVCache):
    """Single-sequence (B = 1) view with the reference's StaticKVCache methods
    (src/decoding/kv_cache.py:39-175). Slots are preallocated (the flat layout
    needs n_slots up front; the reference allocates them lazily) and negative
    slot ids count from the end, so Huginn's coda ids -1, -2
    (src/decoding/huginn_blocks.py:274,279) address the last two slots."""

    def __init__(self, n_kv_head: int, head_dim: int, max_seq_len: int, dtype: torch.dtype, device, *,
                 n_slots: int, head_major: bool = True):
        super().__init__(n_slots, 1, n_kv_head, head_dim, max_seq_len, dtype, device, head_major=head_major)
        self._seen_tokens = 0

    def _slot(self, step_idx: int) -> int:
        s = step_idx + self.n_slots if step_idx < 0 else step_idx
        if not 0 <= s < self.n_slots:
            raise IndexError(f"slot {step_idx} out of range for {self.n_slots} slots")
        return s

    def write_range(self, step_idx: int, base_pos: int, k: torch.Tensor, v: torch.Tensor) -> None:
        """k, v: (1, T, Hkv, Dh) -> positions [base_pos, base_pos + T)."""
        s = self._slot(step_idx)
        T = k.shape[1]
        self.write_tokens([s] * T, [0] * T, list(range(base_pos, base_pos + T)), k[0], v[0])

    def write_scatter(self, step_idx: int, positions, k: torch.Tensor, v: torch.Tensor) -> None:
        """k, v: (1, nq, Hkv, Dh) at disjoint absolute positions."""
        s = self._slot(step_idx)
        self.write_tokens([s] * len(positions), [0] * len(positions), list(positions), k[0], v[0])

    def gather(self, step_idx: int, upto_pos: int):
        """(1, upto_pos + 1, Hkv, Dh) views of positions [0, upto_pos] (no copy)."""
        s = self._slot(step_idx)
        return self.K[s, :, : upto_pos + 1], self.V[s, :, : upto_pos + 1]

    def drop_positions_at_and_after(self, position: int, b: int | None = None) -> None:  # type: ignore[override]
        super().drop_positions_at_and_after(0 if b is None else b, position)
        self._seen_tokens = position

    def get_seq_length(self) -> int:
        return self._seen_tokens

    def reset(self) -> None:
        self.seqlen = [[0] for _ in range(self.n_slots)]
        self._seen_tokens = 0

    def reset_lengths(self) -> None:
        self.reset()
