"""Faults the device ops cannot return themselves, reported by
ltkv_synchronize where the reference panics.

The reference indexes a sequence's blocks with every position it reads
(kv.rs:133-150, `rows`): an index past them panics. Here the tables are
caller data on the device, so attention reads a bad entry as block 0 and
gather copies nothing for it; both set a fault bit that the next
ltkv_synchronize turns into LTKV_ERR_RANGE (and clears). A fused append whose
cell is not position len - 1 of its table (the precondition of
ltkv_append_decode_attention) is reported as LTKV_ERR_ARG. The queries of the
batch that read valid entries are unaffected. Nothing here faults the GPU:
every bad entry is clamped or skipped by the kernels' own bounds checks.
"""

from __future__ import annotations

import numpy as np
import pytest

from helpers import BLOCK, attention_close, fill_sequences, tables_and_lens

pytestmark = pytest.mark.gpu


def _caches(kv_dim, n_blocks, dtype, rng):
    from langtrain_studio_amd import KvCache
    from oracle import OracleKv

    g = KvCache(1, kv_dim, n_blocks * BLOCK, dtype=dtype, device=0)
    o = OracleKv(1, kv_dim, n_blocks * BLOCK, dtype=dtype)
    order = rng.permutation(n_blocks)
    g.init_free_order(order)
    o.init_free_order(order)
    return g, o


def _expect(g, code):
    from langtrain_studio_amd import KvError

    with pytest.raises(KvError) as ei:
        g.synchronize()
    assert ei.value.code == code, ei.value
    g.synchronize()  # reported once, then cleared


@pytest.mark.parametrize("dtype,head_dim,group", [("f16", 128, 4), ("f16", 128, 7), ("q8_0", 128, 4),
                                                  ("f32", 64, 8), ("f32", 128, 4)])
@pytest.mark.parametrize("bad", [-3, "past"])
def test_attention_reports_out_of_range_entry(gpu, dtype, head_dim, group, bad):
    import torch

    from langtrain_studio_amd._lib import ERR_RANGE

    rng = np.random.default_rng(51)
    n_kv = 2
    kv_dim, n_heads = n_kv * head_dim, group * n_kv
    n_blocks = 200
    lens = [300, 900, 40]
    g, o = _caches(kv_dim, n_blocks, dtype, rng)
    fill_sequences([("gpu", g), ("oracle", o)], dict(enumerate(lens)), rng, kv_dim)
    tables, la = tables_and_lens(g, range(3), lens)
    q = rng.standard_normal((3, n_heads * head_dim), dtype=np.float32)
    want = o.attention_tables(0, tables, la, q, n_heads, head_dim, threads=8)
    bad_tables = tables.copy()
    bad_tables[1, 30] = -3 if bad == -3 else n_blocks + 7  # inside query 1's 900 tokens
    out = g.decode_attention(0, torch.from_numpy(q).to(gpu), torch.from_numpy(bad_tables).to(gpu),
                             torch.from_numpy(la).to(gpu), n_heads, head_dim).cpu().numpy()
    _expect(g, ERR_RANGE)
    attention_close(out[[0, 2]], want[[0, 2]], dtype)  # the other queries are unaffected
    # entries past a query's length are never read: no fault
    pad = tables.copy()
    pad[2, 3:] = n_blocks + 100
    g.decode_attention(0, torch.from_numpy(q).to(gpu), torch.from_numpy(pad).to(gpu),
                       torch.from_numpy(la).to(gpu), n_heads, head_dim)
    g.synchronize()


def test_gather_reports_out_of_range_entry(gpu):
    import torch

    from langtrain_studio_amd._lib import ERR_RANGE

    rng = np.random.default_rng(52)
    kv_dim, n_blocks = 256, 64
    g, o = _caches(kv_dim, n_blocks, "f16", rng)
    lens = [40, 100]
    fill_sequences([("gpu", g), ("oracle", o)], dict(enumerate(lens)), rng, kv_dim)
    tables, la = tables_and_lens(g, range(2), lens)
    tables[1, 2] = n_blocks  # tokens 32..47 of sequence 1
    offs = np.array([0, 40], dtype=np.int64)
    k_out = torch.full((140, kv_dim), -1.0, dtype=torch.float16, device=gpu)
    v_out = torch.full((140, kv_dim), -1.0, dtype=torch.float16, device=gpu)
    g.gather(0, torch.from_numpy(tables).to(gpu), torch.from_numpy(la).to(gpu), torch.from_numpy(offs).to(gpu),
             k_out, v_out)
    _expect(g, ERR_RANGE)
    kh = k_out.cpu().numpy().view(np.uint16)
    ok, _ = o.pool(0)
    rows0 = np.concatenate([ok[b] for b in tables[0, :3]])[:40]
    np.testing.assert_array_equal(kh[:40], rows0)  # sequence 0 gathered
    assert (kh[40 + 32:40 + 48] == np.float16(-1.0).view(np.uint16)).all()  # the bad block: untouched


def test_resident_row_out_of_range_reports(gpu):
    import torch

    from langtrain_studio_amd._lib import ERR_RANGE

    rng = np.random.default_rng(53)
    kv_dim, n_blocks = 1024, 64
    g, _ = _caches(kv_dim, n_blocks, "f16", rng)
    fill_sequences([("gpu", g)], {0: 50, 1: 70}, rng, kv_dim)
    rows = g.seq_rows([0, 1]).astype(np.int32)
    q = torch.from_numpy(rng.standard_normal((3, 32 * 128), dtype=np.float32)).to(gpu)
    r = torch.from_numpy(np.array([rows[0], 5000, rows[1]], dtype=np.int32)).to(gpu)
    lens = torch.from_numpy(np.array([50, 0, 70], dtype=np.int32)).to(gpu)
    g.decode_attention_rows(0, q, r, lens, 32, 128)
    g.synchronize()  # a free row with length 0 reads nothing: no fault
    lens = torch.from_numpy(np.array([50, 20, 70], dtype=np.int32)).to(gpu)
    g.decode_attention_rows(0, q, r, lens, 32, 128)
    _expect(g, ERR_RANGE)


def test_fused_append_wrong_cell_reports(gpu):
    import torch

    from langtrain_studio_amd._lib import ERR_ARG

    rng = np.random.default_rng(54)
    kv_dim, n_blocks = 1024, 128
    g, _ = _caches(kv_dim, n_blocks, "f16", rng)
    lens = [100, 33, 260]
    fill_sequences([("gpu", g)], dict(enumerate(lens)), rng, kv_dim)
    seqs = np.arange(3, dtype=np.uint32)
    sm = g.append_batch(seqs, np.array(lens, dtype=np.uint64))
    new_lens = np.array(lens, dtype=np.int32) + 1
    tables, la = tables_and_lens(g, range(3), new_lens)
    k = torch.from_numpy(rng.standard_normal((3, kv_dim), dtype=np.float32)).to(gpu)
    q = torch.from_numpy(rng.standard_normal((3, 32 * 128), dtype=np.float32)).to(gpu)
    dt, dl = torch.from_numpy(tables).to(gpu), torch.from_numpy(la).to(gpu)
    g.append_decode_attention(0, torch.from_numpy(sm).to(gpu), k, k, q, dt, dl, 32, 128)
    g.synchronize()  # the claim's own cells: no fault
    sm2 = g.append_batch(seqs, np.array(new_lens, dtype=np.uint64))
    tables, la = tables_and_lens(g, range(3), new_lens + 1)
    wrong = sm2.copy()
    wrong[1] = sm2[0]  # query 1 handed query 0's cell
    g.append_decode_attention(0, torch.from_numpy(wrong).to(gpu), k, k, q, torch.from_numpy(tables).to(gpu),
                              torch.from_numpy(la).to(gpu), 32, 128)
    _expect(g, ERR_ARG)
