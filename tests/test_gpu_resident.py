"""Resident block tables (the device step descriptor) against the oracle's
allocator, and the ops that read them: the device slot mapping against the
host claim, and attention by rows against attention by explicit tables.

Bar: bit-exact everywhere (tables, lengths and cells are integers; attention
by rows must give the bits of attention by tables on the same inputs).
"""

from __future__ import annotations

import numpy as np
import pytest

from helpers import BLOCK, append_rows, attention_close, fill_sequences, tables_and_lens

pytestmark = pytest.mark.gpu


def _caches(kv_dim, n_blocks, dtype="f16", seed=0):
    from langtrain_studio_amd import KvCache
    from oracle import OracleKv

    order = np.random.default_rng(seed).permutation(n_blocks)
    g = KvCache(1, kv_dim, n_blocks * BLOCK, dtype=dtype, device=0)
    o = OracleKv(1, kv_dim, n_blocks * BLOCK, dtype=dtype)
    g.init_free_order(order)
    o.init_free_order(order)
    return g, o


def _check_resident(g, o, live):
    """Every live sequence's resident row equals the oracle's table; rows not
    held by a live sequence read as empty."""
    tables, lengths = g.resident_tables()
    rows = g.seq_rows(live)
    assert (rows >= 0).all()
    assert len(set(rows.tolist())) == len(rows), "two live sequences share a row"
    for s, r in zip(live, rows):
        want = o.block_table(int(s))
        assert lengths[r] == want.size, (s, r)
        np.testing.assert_array_equal(tables[r, :want.size], want, err_msg=f"seq {s} row {r}")
    held = np.zeros(lengths.size, dtype=bool)
    held[rows] = True
    assert (lengths[~held] == 0).all()


def test_resident_tables_follow_appends_forks_truncates(gpu):
    """Random traffic of the engine's kinds (append in steps, fork by share,
    copy-on-write on the forks' first append, truncate, remove): after every
    step the resident rows equal the oracle's tables, and only changed entries
    are uploaded."""
    rng = np.random.default_rng(7)
    kv_dim, n_blocks = 64, 4096
    g, o = _caches(kv_dim, n_blocks)
    caches = [("gpu", g), ("oracle", o)]
    lens = {s: int(rng.integers(1, 300)) for s in range(40)}
    fill_sequences(caches, lens, rng, kv_dim)
    _check_resident(g, o, sorted(lens))
    next_id = 100
    for step in range(12):
        # forks of a random parent, then one decode token for every sequence
        for _ in range(3):
            src = int(rng.choice(sorted(lens)))
            dst = next_id
            next_id += 1
            n = int(rng.integers(1, lens[src] + 1))
            g.share(src, dst, n)
            o.share(src, dst, n)
            lens[dst] = n
        seqs = np.array(sorted(lens), dtype=np.uint32)
        pos = np.array([lens[int(s)] for s in seqs], dtype=np.uint64)
        before = g.table_uploads()
        append_rows(caches, seqs, pos, rng, kv_dim)
        for s in seqs:
            lens[int(s)] += 1
        # truncate some, remove some
        for s in rng.choice(seqs, size=4, replace=False):
            s = int(s)
            if rng.random() < 0.5:
                g.truncate(s, 0)
                o.truncate(s, 0)
                del lens[s]
            else:
                cut = int(rng.integers(1, lens[s] + 1))
                g.truncate(s, cut)
                o.truncate(s, cut)
                lens[s] = cut
        _check_resident(g, o, sorted(lens))
        # one token per sequence adds at most one table entry each, plus
        # the forks' copied tables and one length per touched row
        grew = g.table_uploads() - before
        assert grew <= 2 * len(lens) + sum(o.block_table(int(s)).size for s in seqs) + 64


def test_resident_tables_grow_in_rows_and_width(gpu):
    """More sequences than the initial 64 rows and a table wider than the
    initial 64 blocks: the tables are reallocated and still match."""
    rng = np.random.default_rng(8)
    kv_dim = 32
    g, o = _caches(kv_dim, 2048)
    caches = [("gpu", g), ("oracle", o)]
    fill_sequences(caches, {s: 3 for s in range(80)}, rng, kv_dim)
    _check_resident(g, o, list(range(80)))
    fill_sequences(caches, {500: 70 * BLOCK + 5}, rng, kv_dim)
    _check_resident(g, o, list(range(80)) + [500])
    tables, _ = g.resident_tables()
    assert tables.shape[0] >= 81 and tables.shape[1] >= 71


def test_removed_rows_are_reused(gpu):
    rng = np.random.default_rng(9)
    g, o = _caches(32, 256)
    caches = [("gpu", g), ("oracle", o)]
    fill_sequences(caches, {1: 20, 2: 40, 3: 5}, rng, 32)
    r2 = int(g.seq_rows([2])[0])
    g.truncate(2, 0)
    o.truncate(2, 0)
    assert g.seq_rows([2])[0] == -1
    fill_sequences(caches, {7: 33}, rng, 32)
    assert g.seq_rows([7])[0] == r2
    _check_resident(g, o, [1, 3, 7])


def test_slot_mapping_equals_host_claim(gpu):
    """The device slot mapping from (row, position) equals what append_batch
    returned for the same tokens; unknown rows and positions past a table
    give -1."""
    import torch

    rng = np.random.default_rng(10)
    kv_dim = 64
    g, o = _caches(kv_dim, 1024)
    caches = [("gpu", g), ("oracle", o)]
    fill_sequences(caches, {s: int(rng.integers(1, 200)) for s in range(12)}, rng, kv_dim)
    g.share(3, 50, 37)
    o.share(3, 50, 37)
    seqs = np.array(list(range(12)) + [50] * 20, dtype=np.uint32)
    pos = np.array([g.len(int(s)) for s in range(12)] + list(range(37, 57)), dtype=np.uint64)
    sm, _ = append_rows(caches, seqs, pos, rng, kv_dim)  # forks copy on write here
    rows = g.seq_rows(seqs)
    d_rows = torch.from_numpy(rows).to(gpu)
    d_pos = torch.from_numpy(pos.astype(np.int64)).to(gpu)
    got = g.slot_mapping(d_rows, d_pos).cpu().numpy()
    np.testing.assert_array_equal(got, sm)
    bad_rows = torch.tensor([-1, 10_000, int(rows[0])], dtype=torch.int32, device=gpu)
    bad_pos = torch.tensor([0, 0, g.len(0) + 10 * BLOCK], dtype=torch.int64, device=gpu)
    np.testing.assert_array_equal(g.slot_mapping(bad_rows, bad_pos).cpu().numpy(), [-1, -1, -1])


@pytest.mark.parametrize("dtype,head_dim,group", [("f16", 128, 4), ("f16", 64, 7), ("f32", 128, 4),
                                                 ("f32", 64, 8), ("q8_0", 128, 4), ("q8_0", 64, 1)])
def test_attention_rows_equals_tables(gpu, dtype, head_dim, group):
    """Attention by resident rows gives the bits of attention by explicit
    tables, and both agree with the oracle; a row of -1 with length 0 gives
    zeros."""
    import torch

    rng = np.random.default_rng(head_dim + group)
    n_kv = 2
    kv_dim = n_kv * head_dim
    n_heads = group * n_kv
    lens = [1, 16, 17, 300, 1031, 2100, 64]
    g, o = _caches(kv_dim, sum(-(-n // BLOCK) for n in lens) + 16, dtype)
    fill_sequences([("gpu", g), ("oracle", o)], dict(enumerate(lens)), rng, kv_dim)
    seqs = list(range(len(lens)))
    tables, la = tables_and_lens(g, seqs, lens)
    q = rng.standard_normal((len(lens) + 1, n_heads * head_dim), dtype=np.float32)
    d_q = torch.from_numpy(q).to(gpu)
    by_tables = g.decode_attention(0, d_q[:-1].contiguous(), torch.from_numpy(tables).to(gpu),
                                   torch.from_numpy(la).to(gpu), n_heads, head_dim).cpu().numpy()
    rows = np.append(g.seq_rows(seqs), -1).astype(np.int32)
    la_rows = np.append(la, 0).astype(np.int32)
    by_rows = g.decode_attention_rows(0, d_q, torch.from_numpy(rows).to(gpu),
                                      torch.from_numpy(la_rows).to(gpu), n_heads, head_dim).cpu().numpy()
    np.testing.assert_array_equal(by_rows[:-1].view(np.uint32), by_tables.view(np.uint32))
    assert (by_rows[-1] == 0).all()
    want = o.attention_tables(0, tables, la, q[:-1], n_heads, head_dim, threads=8)
    attention_close(by_rows[:-1], want, dtype)


def test_attention_rows_after_decode_steps(gpu):
    """A decode loop that only appends and reads rows: every step's attention
    by rows equals the oracle's, with table uploads only when a sequence
    crosses into a new block."""
    import torch

    rng = np.random.default_rng(12)
    n_heads, n_kv, head_dim = 8, 2, 128
    kv_dim = n_kv * head_dim
    g, o = _caches(kv_dim, 512)
    caches = [("gpu", g), ("oracle", o)]
    lens = {s: int(rng.integers(1, 200)) for s in range(16)}
    fill_sequences(caches, lens, rng, kv_dim)
    seqs = np.array(sorted(lens), dtype=np.uint32)
    d_rows = torch.from_numpy(g.seq_rows(seqs)).to(gpu)
    for step in range(20):
        pos = np.array([lens[int(s)] for s in seqs], dtype=np.uint64)
        new_blocks = int((pos % BLOCK == 0).sum())
        g.sync_tables()
        before = g.table_uploads()
        append_rows(caches, seqs, pos, rng, kv_dim)
        for s in seqs:
            lens[int(s)] += 1
        q = rng.standard_normal((seqs.size, n_heads * head_dim), dtype=np.float32)
        la = np.array([lens[int(s)] for s in seqs], dtype=np.int32)
        out = g.decode_attention_rows(0, torch.from_numpy(q).to(gpu), d_rows, torch.from_numpy(la).to(gpu),
                                      n_heads, head_dim).cpu().numpy()
        assert g.table_uploads() - before == 2 * new_blocks  # entry + length per new block
        tables = g.block_tables(seqs)
        want = o.attention_tables(0, tables, la, q, n_heads, head_dim, threads=8)
        attention_close(out, want, "f16")
