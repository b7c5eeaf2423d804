"""The native tick planner (_tick.plan_pass) against a numpy restatement of
the row tables a pass hands its kernels (CPU).

Table layout of a pass over nb rows (rows n..nb-1 padding): int32 [pos |
kv_len | pool_row | ring_slot (C) | group_first (grouped)], int64 [ids (P) |
row_base x L | flat_row x L | expected token (C)], with row_base =
(slot * B + b) * S (src/decoding/batch_kv_cache.py:64-65) and the slot
numbering of src/decoding/kv_cache.py:8-22 (prelude i -> i, core step r layer
l -> n_prelude + r * n_core + l, coda i -> n_prelude + T_total * n_core + i).
"""
from __future__ import annotations

import numpy as np
import pytest

from wavefront_decoding_amd import _lib

NO_EXPECT = -(1 << 62)

# the engine constants, in _tick's parameter order
FIELDS = ["B", "S", "trash_row", "R", "trash_pool_row", "n_prelude", "n_core", "n_coda", "T_total", "coda_base",
          "ring_len", "max_batch", "max_seq_len", "max_rows", "use_graphs", "group_attention", "gmax",
          "group_min_wg", "n_kv_heads"]


def params(**kw) -> dict:
    p = dict(B=4, S=96, n_prelude=2, n_core=4, n_coda=2, T_total=16, ring_len=1000, max_batch=4, max_seq_len=128,
             max_rows=256, use_graphs=1, group_attention=1, gmax=4, group_min_wg=1, n_kv_heads=4)
    p.update(kw)
    n_slots = p["n_prelude"] + p["T_total"] * p["n_core"] + p["n_coda"]
    p.setdefault("trash_row", n_slots * p["B"] * p["S"])
    p["R"] = p["T_total"] + 2
    p.setdefault("trash_pool_row", p["max_batch"] * p["R"])
    p["coda_base"] = p["n_prelude"] + p["T_total"] * p["n_core"]
    return p


def as_tuple(p: dict) -> tuple:
    return tuple(int(p[f]) for f in FIELDS)


def bucket(n: int) -> int:
    if n > 64:
        return (n + 63) // 64 * 64
    b = 1
    while b < n:
        b *= 2
    return b


def ref_groups(p, kind, seqs, steps, nb, force):
    """group_first of a pass (nb + 1 entries) or None: adjacent rows with the
    same key (sequence; for R also the depth) at most gmax rows a group,
    padding rows one by one; only when it leaves >= group_min_wg workgroups."""
    n = len(seqs)
    key = seqs * (p["T_total"] + 1) + steps if kind == "R" else seqs
    if force == 0:
        return None
    if force < 0:
        if not p["group_attention"] or n < 2 or not np.any(key[1:] == key[:-1]):
            return None
    first = [0] if n else []
    for i in range(1, n):
        if key[i] != key[i - 1] or i - first[-1] >= p["gmax"]:
            first.append(i)
    if force < 0 and len(first) * p["n_kv_heads"] < p["group_min_wg"]:
        return None
    first += list(range(n, nb + 1))
    gf = np.full(nb + 1, nb, dtype=np.int32)
    gf[:len(first)] = first
    return gf


def ref_tables(p, kind, seqs, pos, extra, nb_force=-1, grouped_force=-1, ring_base=-1):
    seqs = np.asarray(seqs, dtype=np.int64)
    pos = np.asarray(pos, dtype=np.int64)
    n = len(pos)
    nb = nb_force if nb_force >= 0 else (bucket(n) if p["use_graphs"] else n)
    L = {"P": p["n_prelude"], "R": p["n_core"], "C": p["n_coda"]}[kind]
    steps = np.asarray(extra, dtype=np.int64) if kind == "R" else None
    if kind == "P":
        slots = np.repeat(np.arange(L, dtype=np.int64)[:, None], n, axis=1)
    elif kind == "R":
        slots = p["n_prelude"] + steps[None, :] * p["n_core"] + np.arange(L, dtype=np.int64)[:, None]
    else:
        slots = p["coda_base"] + np.repeat(np.arange(L, dtype=np.int64)[:, None], n, axis=1)
    rb = np.full((L, nb), p["trash_row"], dtype=np.int64)
    rb[:, :n] = (slots * p["B"] + seqs[None, :]) * p["S"]
    fr = rb.copy()
    fr[:, :n] += pos[None, :]
    groups = ref_groups(p, kind, seqs, steps, nb, grouped_force)
    nblk = 4 if kind == "C" else 3
    i32 = np.zeros(nblk * nb + (nb + 1 if groups is not None else 0), dtype=np.int32)
    if groups is not None:
        i32[nblk * nb:] = groups
    i32[:n] = pos
    i32[nb: nb + n] = pos + 1
    i32[nb + n: 2 * nb] = 1
    i32[2 * nb: 2 * nb + n] = seqs * p["R"] + pos % p["R"]
    i32[2 * nb + n: 3 * nb] = p["trash_pool_row"]
    if kind == "C":
        i32[3 * nb: 4 * nb] = p["ring_len"]
        if ring_base >= 0:
            i32[3 * nb: 3 * nb + n] = np.arange(ring_base, ring_base + n, dtype=np.int32)
    parts = [rb.reshape(-1), fr.reshape(-1)]
    if kind == "P":
        idp = np.zeros(nb, dtype=np.int64)
        idp[:n] = extra
        parts.insert(0, idp)
    elif kind == "C":
        exp = np.full(nb, NO_EXPECT, dtype=np.int64)
        if extra is not None and len(extra):
            exp[:n] = extra
        parts.append(exp)
    kv_max = int(pos.max()) + 1 if n else 0
    return nb, i32, np.concatenate(parts), groups is not None, kv_max, int(pos.sum())


@pytest.fixture(scope="module")
def tick():
    t = _lib.load_tick()
    assert t.NUM_PARAMS == len(FIELDS)
    return t


def run(tick, p, kind, seqs, pos, extra, nb_force=-1, grouped_force=-1, ring_base=-1, o32=3, o64=5):
    t32 = np.full(o32 + 4096, -7, dtype=np.int32)
    t64 = np.full(o64 + 8192, -7, dtype=np.int64)
    nb, n32, n64, grouped, kv_max, psum = tick.plan_pass(t32, o32, t64, o64, as_tuple(p), kind, seqs, pos, extra,
                                                         nb_force, grouped_force, ring_base)
    assert (t32[:o32] == -7).all() and (t32[o32 + n32:] == -7).all()  # nothing written outside the pass
    assert (t64[:o64] == -7).all() and (t64[o64 + n64:] == -7).all()
    return nb, t32[o32: o32 + n32], t64[o64: o64 + n64], grouped, kv_max, psum


def check_same(got, want):
    nb, i32, i64, grouped, kv_max, psum = got
    wnb, w32, w64, wgrouped, wkv, wps = want
    assert (nb, grouped, kv_max, psum) == (wnb, wgrouped, wkv, wps)
    np.testing.assert_array_equal(i32, w32)
    np.testing.assert_array_equal(i64, w64)


def random_pass(rng, p, kind, n, sorted_rows):
    seqs = rng.integers(0, p["B"], n)
    if sorted_rows:
        seqs = np.sort(seqs)
    pos = rng.integers(0, p["S"], n)
    if kind == "P":
        extra = rng.integers(-50, 4000, n)  # ids, or ring handles (negative)
    elif kind == "R":
        extra = rng.integers(0, p["T_total"], n)
        if sorted_rows:  # a few rows at the same depth of the same sequence (grouped attention)
            extra = np.sort(extra // 4)
    else:
        extra = None if rng.random() < 0.3 else rng.integers(-60, 4000, n)
    return seqs, pos, extra


@pytest.mark.parametrize("kind", ["P", "R", "C"])
@pytest.mark.parametrize("use_graphs", [1, 0])
def test_random_passes_match_the_restatement(tick, kind, use_graphs):
    rng = np.random.default_rng({"P": 1, "R": 2, "C": 3}[kind] + 10 * use_graphs)
    for case in range(120):
        p = params(use_graphs=use_graphs, gmax=int(rng.choice([1, 2, 4, 8])),
                   group_min_wg=int(rng.choice([1, 8, 64])), group_attention=int(rng.random() < 0.8))
        n = int(rng.choice([0, 1, 2, 3, 5, 8, 13, 17, 40, 64, 65, 100]))
        seqs, pos, extra = random_pass(rng, p, kind, n, sorted_rows=case % 2 == 0)
        rb = int(rng.integers(0, 500)) if kind == "C" and rng.random() < 0.7 else -1
        want = ref_tables(p, kind, seqs, pos, extra, ring_base=rb)
        as_list = lambda a: None if a is None else [int(v) for v in a]  # noqa: E731
        check_same(run(tick, p, kind, as_list(seqs), as_list(pos), as_list(extra), ring_base=rb), want)
        # numpy int64 / int32 arrays and strided views read the same
        check_same(run(tick, p, kind, seqs, pos.astype(np.int32), extra, ring_base=rb), want)
        if n:
            s2, p2 = np.repeat(seqs, 2)[::2], np.repeat(pos, 2)[::2]
            check_same(run(tick, p, kind, s2, p2, extra, ring_base=rb), want)


@pytest.mark.parametrize("kind", ["P", "R", "C"])
def test_padding_tables_of_a_capture(tick, kind):
    """n = 0 with a forced bucket and grouping: every row a padding row aimed
    at the trash row / trash pool row / trash ring slot, each its own group."""
    p = params()
    for nb in (1, 8, 64, 192):
        for g in (0, 1):
            got = run(tick, p, kind, [], [], None if kind == "C" else [], nb_force=nb, grouped_force=g)
            want = ref_tables(p, kind, [], [], None if kind == "C" else [], nb_force=nb, grouped_force=g)
            check_same(got, want)
            nb_, i32, i64, grouped, _, _ = got
            assert nb_ == nb and grouped == bool(g)
            L = {"P": 2, "R": 4, "C": 2}[kind]
            off = nb if kind == "P" else 0
            assert (i64[off: off + 2 * L * nb] == p["trash_row"]).all()
            assert (i32[2 * nb: 3 * nb] == p["trash_pool_row"]).all()
            if g:
                nblk = 4 if kind == "C" else 3
                np.testing.assert_array_equal(i32[nblk * nb:], np.arange(nb + 1))


def test_grouping_thresholds(tick):
    """8 rows of one sequence at one depth: groups of gmax rows; dropped when
    they leave fewer than group_min_wg (group, kv head) workgroups or when
    grouping is off; adjacent rows at different depths never share a group."""
    seqs, pos, steps = [0] * 8, list(range(10, 18)), [3] * 8
    p = params(gmax=4, group_min_wg=8, n_kv_heads=4)
    nb, i32, _, grouped, _, _ = run(tick, p, "R", seqs, pos, steps)
    assert grouped and list(i32[3 * nb: 3 * nb + 3]) == [0, 4, 8]
    assert not run(tick, params(gmax=4, group_min_wg=9, n_kv_heads=4), "R", seqs, pos, steps)[3]
    assert not run(tick, params(group_attention=0), "R", seqs, pos, steps)[3]
    assert not run(tick, params(group_min_wg=1), "R", seqs, pos, list(range(8)))[3]  # every row its own depth
    nb, i32, _, grouped, _, _ = run(tick, params(gmax=8, group_min_wg=1), "C", [0, 0, 1, 1, 1], [5, 6, 7, 8, 9], None)
    assert grouped and list(i32[4 * nb: 4 * nb + 9]) == [0, 2, 5, 6, 7, 8, 8, 8, 8]


def test_rejects_bad_rows(tick):
    p = params()
    with pytest.raises(IndexError, match="position out of range"):
        run(tick, p, "P", [0], [p["S"]], [1])
    with pytest.raises(IndexError, match="position out of range"):
        run(tick, p, "R", [0], [-1], [0])
    with pytest.raises(IndexError, match="sequence index"):
        run(tick, p, "C", [p["B"]], [3], None)
    with pytest.raises(IndexError, match="sequence index"):
        run(tick, params(max_batch=2), "C", [2], [3], None)
    with pytest.raises(ValueError, match="core step"):
        run(tick, p, "R", [0], [3], [p["T_total"]])
    with pytest.raises(ValueError, match="max_rows"):
        run(tick, params(max_rows=64), "C", [0] * 65, [1] * 65, None)
    with pytest.raises(ValueError, match="max_seq_len"):
        run(tick, params(max_seq_len=64), "C", [0], [1], None)
    with pytest.raises(ValueError, match="differs in length"):
        run(tick, p, "P", [0, 0], [1, 2], [5])
    with pytest.raises(ValueError, match="differ in length"):
        run(tick, p, "C", [0], [1, 2], None)
    with pytest.raises(ValueError, match="needs"):
        run(tick, p, "R", [0], [1], None)
    with pytest.raises(ValueError, match="kind"):
        run(tick, p, "X", [0], [1], None)
    with pytest.raises(ValueError, match="below the row count"):
        run(tick, p, "C", [0, 0], [1, 2], None, nb_force=1)
    with pytest.raises(TypeError):
        run(tick, p, "C", [0], ["a"], None)
    with pytest.raises(ValueError, match="scratch too small"):
        tick.plan_pass(np.zeros(4, np.int32), 0, np.zeros(64, np.int64), 0, as_tuple(p), "C", [0] * 2, [1, 2], None,
                       -1, -1, -1)
    with pytest.raises(TypeError):
        tick.plan_pass(np.zeros(64, np.int64), 0, np.zeros(64, np.int64), 0, as_tuple(p), "C", [0], [1], None,
                       -1, -1, -1)


def test_launch_checks_its_arguments_before_any_runtime_call(tick):
    t64, t32 = np.zeros(8, np.int64), np.zeros(8, np.int32)
    with pytest.raises(ValueError, match="null"):
        tick.launch(0, 0, 0, 1, 1, t64, 4, t32, 4, 0, 0)
    with pytest.raises(ValueError, match="beyond the scratch"):
        tick.launch(0, 0, 1, 1, 1, t64, 9, t32, 4, 0, 0)
    with pytest.raises(ValueError, match="accept flag"):
        tick.launch(0, 0, 1, 1, 1, t64, 4, t32, 4, 0, 3)
    with pytest.raises(TypeError):
        tick.launch(0, 0, 1, 1, 1, t64, 4, t32, 4)


def test_accept_flag_polling(tick):
    """clear_flags / wait_flags on ordinary host memory (the engine points
    them at mapped pinned memory the argmax kernel stores into): a flag reads
    -1 until written; the poll returns the flags once all n are written, None
    on timeout."""
    f = np.array([5, 0, 1, 7, 9], dtype=np.int32)
    tick.clear_flags(f.ctypes.data, 4)
    assert f.tolist() == [-1, -1, -1, -1, 9]
    assert tick.wait_flags(f.ctypes.data, 4, 0.01) is None
    f[:3] = [1, 0, 1]
    assert tick.wait_flags(f.ctypes.data, 4, 0.01) is None  # one still unwritten
    f[3] = 0
    assert tick.wait_flags(f.ctypes.data, 4, 0.01) == [True, False, True, False]
    assert tick.wait_flags(f.ctypes.data, 0, 0.0) == []
    with pytest.raises(ValueError):
        tick.wait_flags(0, 2, 0.0)
    with pytest.raises(ValueError):
        tick.clear_flags(f.ctypes.data, -1)


def test_note_writes_matches_note_write():
    """The slot-length bookkeeping of a pass (BatchStaticKVCache.note_writes)
    extends exactly the lengths a note_write per (slot, row) would."""
    import torch

    from wavefront_decoding_amd.kv_cache import BatchStaticKVCache

    rng = np.random.default_rng(4)
    a = BatchStaticKVCache(20, 3, 1, 8, 64, torch.float32, "cpu")
    b = BatchStaticKVCache(20, 3, 1, 8, 64, torch.float32, "cpu")
    for _ in range(200):
        n = int(rng.integers(1, 6))
        seqs, pos = rng.integers(0, 3, n), rng.integers(0, 64, n)
        nsl = int(rng.integers(1, 5))
        if rng.random() < 0.5:
            first = int(rng.integers(0, 20 - nsl + 1))
            a.note_writes(first, nsl, seqs, pos)
            firsts = [first] * n
        else:
            firsts = [int(f) for f in rng.integers(0, 20 - nsl + 1, n)]
            a.note_writes(firsts, nsl, seqs.tolist(), pos.tolist())
        for f, sq, p in zip(firsts, seqs, pos):
            for sl in range(f, f + nsl):
                b.note_write(sl, int(sq), int(p))
        if rng.random() < 0.1:
            bq, at = int(rng.integers(0, 3)), int(rng.integers(0, 64))
            a.drop_positions_at_and_after(bq, at)
            b.drop_positions_at_and_after(bq, at)
        assert a.seqlen == b.seqlen
