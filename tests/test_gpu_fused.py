"""The decode step's append fused into decode attention
(ltkv_append_decode_attention) against the same step as two launches
(ltkv_write, then ltkv_decode_attention): pools and outputs bit-identical,
and the output within the attention tolerance of the oracle."""

from __future__ import annotations

import numpy as np
import pytest

from helpers import BLOCK, attention_close, fill_sequences

pytestmark = pytest.mark.gpu


def _pair(dtype, kv_dim, n_blocks, order):
    from langtrain_studio_amd import KvCache

    caches = []
    for _ in range(2):
        c = KvCache(1, kv_dim, n_blocks * BLOCK, dtype=dtype, device=0)
        c.init_free_order(order)
        caches.append(c)
    return caches


def _step(gpu, dtype, head_dim, group, n_kv, ctx, partition=0, seed=0, skip=()):
    import torch

    from oracle import OracleKv

    rng = np.random.default_rng(seed)
    kv_dim = n_kv * head_dim
    n_heads = group * n_kv
    n = len(ctx)
    blocks = sum(-(-(c + 1) // BLOCK) for c in ctx) + 8
    order = rng.permutation(blocks)
    a, b = _pair(dtype, kv_dim, blocks, order)
    o = OracleKv(1, kv_dim, blocks * BLOCK, dtype=dtype)
    o.init_free_order(order)
    if partition:
        a.set_attention_partition(partition)
        b.set_attention_partition(partition)
    fill_sequences([("gpu", a), ("gpu", b), ("oracle", o)], dict(enumerate(ctx)), rng, kv_dim)
    seqs = np.arange(n, dtype=np.uint32)
    pos = np.array(ctx, dtype=np.uint64)
    sm = a.append_batch(seqs, pos)
    np.testing.assert_array_equal(b.append_batch(seqs, pos), sm)
    o.append_batch(seqs, pos)
    sm = sm.copy()
    for i in skip:
        sm[i] = -1  # a skipped cell: nothing written, the stale cell is read
    lens = np.array([c + 1 for c in ctx], dtype=np.int32)
    tables = a.block_tables(seqs)
    k = rng.standard_normal((n, kv_dim), dtype=np.float32)
    v = rng.standard_normal((n, kv_dim), dtype=np.float32)
    q = rng.standard_normal((n, n_heads * head_dim), dtype=np.float32)
    d = {x: torch.from_numpy(y).to(gpu) for x, y in (("sm", sm), ("k", k), ("v", v), ("q", q),
                                                       ("t", tables), ("l", lens))}
    a.write_batch(0, d["sm"], d["k"], d["v"])
    two = a.decode_attention(0, d["q"], d["t"], d["l"], n_heads, head_dim).cpu().numpy()
    one = b.append_decode_attention(0, d["sm"], d["k"], d["v"], d["q"], d["t"], d["l"], n_heads,
                                    head_dim).cpu().numpy()
    np.testing.assert_array_equal(one.view(np.uint32), two.view(np.uint32))
    for pa, pb in zip(a.read_pool(0), b.read_pool(0)):
        np.testing.assert_array_equal(pa, pb)
    o.write_batch(0, sm, k, v)
    if not skip:
        want = o.attention_tables(0, tables, lens, q, n_heads, head_dim, threads=8)
        attention_close(one, want, dtype)


@pytest.mark.parametrize("head_dim,group,n_kv", [(128, 4, 8), (128, 7, 4), (64, 8, 2), (64, 2, 4),
                                                 (128, 1, 2)])
def test_fused_step_equals_write_then_attention(gpu, head_dim, group, n_kv):
    # new tokens at slot 0 of a new block (ctx % 16 == 0), mid-block, the
    # first token of a sequence, and long contexts split over partitions
    ctx = [0, 15, 16, 17, 31, 32, 300, 1023, 1024, 2047, 4100]
    _step(gpu, "f16", head_dim, group, n_kv, ctx, seed=head_dim + group)


@pytest.mark.parametrize("partition", [64, 1024])
def test_fused_step_fixed_partitions(gpu, partition):
    _step(gpu, "f16", 128, 4, 8, [5, 64, 65, 700, 2049], partition=partition, seed=partition)


def test_fused_step_partition_runs(gpu):
    # 16 queries of ~2k tokens in 64-token partitions: more than twice the
    # wave slots in partition items, so waves take runs of partitions and the
    # one whose run ends the query writes the new row
    _step(gpu, "f16", 128, 4, 8, [1990 + 37 * i for i in range(16)], partition=64, seed=9)


def test_fused_step_skipped_cells(gpu):
    _step(gpu, "f16", 128, 4, 8, [10, 40, 300], seed=3, skip=(1,))


@pytest.mark.parametrize("dtype", ["q8_0", "f32"])
def test_fused_step_other_dtypes_are_two_launches(gpu, dtype):
    _step(gpu, dtype, 128, 4, 2, [0, 17, 300], seed=4)
