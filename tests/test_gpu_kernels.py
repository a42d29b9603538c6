"""Parity of the HIP kernels (through the C ABI) against the CPU oracle.

Bar: bit-exact for append (write), copy-on-write/block copy, gather and block
tables; attention within max abs 1e-3 (f32 KV) / 2e-2 (f16 KV) and relative
L2 1e-3 of the oracle's restatement of model.rs:431-475.
"""

from __future__ import annotations

import numpy as np
import pytest

from helpers import BLOCK, attention_close, fill_sequences, tables_and_lens

pytestmark = pytest.mark.gpu


def _caches(n_layers, kv_dim, n_tokens, dtype, order=None):
    from langtrain_studio_amd import KvCache
    from oracle import OracleKv

    g = KvCache(n_layers, kv_dim, n_tokens, dtype=dtype, device=0)
    o = OracleKv(n_layers, kv_dim, n_tokens, dtype=dtype)
    if order is not None:
        g.init_free_order(order)
        o.init_free_order(order)
    return g, o


def _bits(a):
    return a.view(np.uint16) if a.dtype == np.uint16 else a.view(np.uint32)


def _assert_pools_equal(g, o, layers):
    for layer in layers:
        gk, gv = g.read_pool(layer)
        ok, ov = o.pool(layer)
        np.testing.assert_array_equal(_bits(gk), _bits(ok), err_msg=f"K pool, layer {layer}")
        np.testing.assert_array_equal(_bits(gv), _bits(ov), err_msg=f"V pool, layer {layer}")


# ---------------------------------------------------------------------------- write (kernel 1)
@pytest.mark.parametrize("dtype", ["f16", "f32"])
def test_write_bitexact_special_values(gpu, dtype):
    rng = np.random.default_rng(1)
    kv_dim, n_blocks = 256, 64
    order = rng.permutation(n_blocks)
    g, o = _caches(2, kv_dim, n_blocks * BLOCK, dtype, order)
    fill_sequences([("gpu", g), ("oracle", o)], {0: 37, 5: 16, 9: 100, 3: 1}, rng, kv_dim,
                   layers=(0, 1), special=True)
    g.synchronize()
    _assert_pools_equal(g, o, (0, 1))


def test_write_skips_negative_and_out_of_range_slots(gpu):
    import torch

    from langtrain_studio_amd import KvCache

    g = KvCache(1, 64, 4 * BLOCK, device=0)
    sm = torch.tensor([-1, 3, 4 * BLOCK, 5, -7], dtype=torch.int32, device=gpu)
    k = torch.full((5, 64), 2.0, device=gpu)
    g.write_batch(0, sm, k, k)
    pk, pv = g.read_pool(0)
    flat = pk.reshape(-1, 64)
    written = {3, 5}
    for cell in range(4 * BLOCK):
        want = 0x4000 if cell in written else 0  # 2.0 in f16 is 0x4000
        assert (flat[cell] == want).all(), cell


def test_write_row_strided_source(gpu):
    import torch

    from langtrain_studio_amd import KvCache
    from oracle import OracleKv

    rng = np.random.default_rng(2)
    g = KvCache(1, 128, 8 * BLOCK, device=0)
    o = OracleKv(1, 128, 8 * BLOCK)
    sm = g.append_batch([0] * 20, np.arange(20))
    o.append_batch([0] * 20, np.arange(20))
    src = rng.standard_normal((20, 160), dtype=np.float32)  # row stride 160 > kv_dim
    g.write_batch(0, torch.from_numpy(sm).to(gpu), torch.from_numpy(src).to(gpu), torch.from_numpy(src).to(gpu))
    o.write_batch(0, sm, src[:, :128], src[:, :128])
    _assert_pools_equal(g, o, (0,))


@pytest.mark.parametrize("dtype", ["f16", "f32"])
def test_write_bulk_streaming(gpu, dtype):
    """An append whose sources exceed the 256 MB last-level cache (40 000 rows
    of kv_dim 1024, 328 MB of f32 K and V) takes the streaming form (two rows
    a thread, non-temporal loads): the pools equal the oracle's bit for bit,
    skipped and out-of-range slots are left alone (including a missing
    second row of an odd count), then a second streaming append and a
    cached-size one follow."""
    import torch

    rng = np.random.default_rng(43)
    kv_dim, n = 1024, 40000
    n_blocks = n // BLOCK + 64
    g, o = _caches(1, kv_dim, n_blocks * BLOCK, dtype, rng.permutation(n_blocks))
    seqs = np.repeat(np.arange(n // 500, dtype=np.uint32), 500)
    pos = np.tile(np.arange(500, dtype=np.uint64), n // 500)
    sm = g.append_batch(seqs, pos)
    np.testing.assert_array_equal(sm, o.append_batch(seqs, pos))
    sm = sm.copy()
    sm[rng.choice(n, 50, replace=False)] = -1
    sm[rng.choice(n, 5, replace=False)] = n_blocks * BLOCK + 3
    for rows in (n, 33001, 4000):
        k = rng.standard_normal((rows, kv_dim), dtype=np.float32)
        v = rng.standard_normal((rows, kv_dim), dtype=np.float32)
        g.write_batch(0, torch.from_numpy(sm[:rows]).to(gpu), torch.from_numpy(k).to(gpu),
                      torch.from_numpy(v).to(gpu))
        o.write_batch(0, np.where(sm[:rows] >= n_blocks * BLOCK, -1, sm[:rows]), k, v)  # skipped on the GPU
        _assert_pools_equal(g, o, (0,))


@pytest.mark.parametrize("dtype,kv_dim,n", [("f16", 1024, 40000), ("f32", 1024, 3001), ("q8_0", 256, 5000),
                                             ("f16", 12, 777)])
def test_write_ordered_equals_write(gpu, dtype, kv_dim, n):
    """ltkv_write_ordered over ltkv_cell_order's rows writes the oracle's
    cells bit for bit (streaming and cached forms, q8_0 quants and scales,
    rows that move element-wise), skipped and out-of-range cells left alone;
    order entries outside the batch are skipped."""
    import torch

    rng = np.random.default_rng(n + kv_dim)
    n_blocks = n // BLOCK + 64
    g, o = _caches(1, kv_dim, n_blocks * BLOCK, dtype, rng.permutation(n_blocks))
    per = 500 if n >= 500 else 37
    seqs = np.repeat(np.arange(-(-n // per), dtype=np.uint32), per)[:n]
    pos = np.concatenate([np.arange(per, dtype=np.uint64)] * -(-n // per))[:n]
    sm = g.append_batch(seqs, pos)
    np.testing.assert_array_equal(sm, o.append_batch(seqs, pos))
    sm = sm.copy()
    sm[rng.choice(n, 50, replace=False)] = -1
    sm[rng.choice(n, 5, replace=False)] = n_blocks * BLOCK + 3
    order = g.cell_order(sm)
    assert order.size == n - int((sm < 0).sum()) - int((sm >= n_blocks * BLOCK).sum())
    d_order = torch.from_numpy(np.concatenate([order, np.array([-1, n, n + 7], np.int32)])).to(gpu)
    k = rng.standard_normal((n, kv_dim), dtype=np.float32)
    v = rng.standard_normal((n, kv_dim), dtype=np.float32)
    g.write_batch_ordered(0, torch.from_numpy(sm).to(gpu), torch.from_numpy(k).to(gpu),
                          torch.from_numpy(v).to(gpu), d_order)
    o.write_batch(0, np.where(sm >= n_blocks * BLOCK, -1, sm), k, v)
    _assert_pools_equal(g, o, (0,))
    if dtype == "q8_0":
        for a, b in zip(g.read_scales(0), o.scales(0)):
            np.testing.assert_array_equal(a, b.transpose(0, 2, 1))


# ---------------------------------------------------------------------------- kv.rs tests, on the GPU cache
def test_share_then_diverge_copies_on_write(gpu):
    """kv.rs:202-217 with the K/V data living in HBM, at the test's own kv_dim 4."""
    from langtrain_studio_amd import KvCache
    from oracle import f16_to_f32

    kv = KvCache(1, 4, 256, device=0)

    def fill(seq, n, base):
        for p in range(kv.len(seq), n):
            b, s = kv.append(seq, p)
            x = np.full(kv.kv_dim, base + p, dtype=np.float32)
            kv.write(0, b, s, x, x)

    fill(0, 20, 0.0)
    kv.share(0, 1, 20)
    free_before = kv.free_blocks()
    b, s = kv.append(1, 20)
    kv.write(0, b, s, np.full(4, 1000.0, np.float32), np.full(4, 1000.0, np.float32))
    assert kv.free_blocks() == free_before - 1
    a = f16_to_f32(kv.rows(0, 0, 20)[0][:, 0])
    c = f16_to_f32(kv.rows(0, 1, 21)[0][:, 0])
    np.testing.assert_array_equal(a, c[:20])
    assert c[20] == 1000.0
    assert kv.len(0) == 20


def test_truncate_frees_blocks(gpu):
    """kv.rs:219-229 on the GPU cache, at the test's own kv_dim 4."""
    from langtrain_studio_amd import KvCache, NonContiguous

    kv = KvCache(1, 4, 64, device=0)
    for p in range(40):
        b, s = kv.append(3, p)
        x = np.full(4, float(p), np.float32)
        kv.write(0, b, s, x, x)
    assert kv.free_blocks() == 1
    kv.truncate(3, 10)
    assert kv.free_blocks() == 3
    kv.truncate(3, 0)
    assert kv.free_blocks() == 4
    with pytest.raises(NonContiguous):
        kv.append(3, 5)


# ---------------------------------------------------------------------------- copy-on-write / copy (kernel 2)
@pytest.mark.parametrize("dtype", ["f16", "f32"])
def test_copy_on_write_matches_oracle(gpu, dtype):
    """Prefix sharing, divergence and truncation, three layers: pools and
    tables stay bit-identical to the oracle after every step."""
    import torch

    rng = np.random.default_rng(3)
    kv_dim, n_blocks, layers = 64, 96, (0, 1, 2)
    g, o = _caches(3, kv_dim, n_blocks * BLOCK, dtype, rng.permutation(n_blocks))
    fill_sequences([("gpu", g), ("oracle", o)], {0: 45, 1: 16}, rng, kv_dim, layers=layers)
    for dst in (2, 3, 4, 5):
        g.share(0, dst, 45)
        o.share(0, dst, 45)
    g.share(1, 6, 16)
    o.share(1, 6, 16)
    g.share(0, 7, 30)  # shares a partially used block in the middle of seq 0
    o.share(0, 7, 30)
    for step in range(6):
        seqs = [0, 2, 3, 4, 5, 6, 7]
        pos = [g.len(s) for s in seqs]
        sm_g = g.append_batch(seqs, pos)
        sm_o = o.append_batch(seqs, pos)
        np.testing.assert_array_equal(sm_g, sm_o)
        for layer in layers:
            k = rng.standard_normal((len(seqs), kv_dim), dtype=np.float32)
            v = rng.standard_normal((len(seqs), kv_dim), dtype=np.float32)
            g.write_batch(layer, torch.from_numpy(sm_g).to(gpu), torch.from_numpy(k).to(gpu),
                          torch.from_numpy(v).to(gpu))
            o.write_batch(layer, sm_o, k, v)
        if step == 2:
            g.truncate(3, 20)
            o.truncate(3, 20)
            g.share(5, 3, 40)
            o.share(5, 3, 40)
        assert g.cow_copies() == o.cow_copies()
        assert g.free_blocks() == o.free_blocks()
        for s in range(8):
            np.testing.assert_array_equal(g.block_table(s), o.block_table(s))
        _assert_pools_equal(g, o, layers)
    assert g.cow_copies() >= 6


def test_copy_blocks_bulk(gpu):
    import torch

    from langtrain_studio_amd import KvCache

    rng = np.random.default_rng(4)
    kv_dim, n_blocks = 1024, 300
    g = KvCache(2, kv_dim, n_blocks * BLOCK, device=0)
    seq_lens = {0: n_blocks * BLOCK}
    fill_sequences([("gpu", g)], seq_lens, rng, kv_dim, layers=(0, 1))
    before = [g.read_pool(l) for l in (0, 1)]
    perm = rng.permutation(n_blocks)
    src, dst = perm[:100], perm[100:200]
    pairs = torch.from_numpy(np.stack([src, dst], 1).astype(np.int32)).to(gpu)
    g.copy_blocks(pairs)
    for l in (0, 1):
        k, v = g.read_pool(l)
        wk, wv = before[l][0].copy(), before[l][1].copy()
        wk[dst] = before[l][0][src]
        wv[dst] = before[l][1][src]
        np.testing.assert_array_equal(k, wk)
        np.testing.assert_array_equal(v, wv)


@pytest.mark.parametrize("dtype", ["f16", "q8_0"])
def test_copy_blocks_destination_ordered(gpu, dtype):
    """Batches of 4096 pairs and more are bucketed by destination on the
    device before the copy: the pools (and q8_0 scales) equal the oracle's
    block copies bit for bit, invalid pairs are skipped, and the bucket
    counts start from zero again on the next call (three calls in a row:
    above, at and below the ordering threshold)."""
    import torch

    rng = np.random.default_rng(41)
    kv_dim, n_blocks = 64, 12000
    g, o = _caches(2, kv_dim, n_blocks * BLOCK, dtype, rng.permutation(n_blocks))
    fill_sequences([("gpu", g), ("oracle", o)], {s: 16 * BLOCK for s in range(n_blocks // 16)}, rng, kv_dim,
                   layers=(0, 1))
    for n_pairs in (5000, 4096, 100):
        perm = rng.permutation(n_blocks).astype(np.int32)
        pairs = np.stack([perm[:n_pairs], perm[n_pairs:2 * n_pairs]], 1)
        bad = np.array([[-1, 5], [7, n_blocks], [3, 3], [n_blocks + 9, 2]], dtype=np.int32)
        pairs = np.concatenate([pairs, bad])[rng.permutation(n_pairs + len(bad))]
        g.copy_blocks(torch.from_numpy(np.ascontiguousarray(pairs)).to(gpu))
        o.copy_blocks(pairs)
        _assert_pools_equal(g, o, (0, 1))
        if dtype == "q8_0":
            for layer in (0, 1):
                gks, gvs = g.read_scales(layer)
                oks, ovs = o.scales(layer)
                np.testing.assert_array_equal(gks, oks.transpose(0, 2, 1))  # [block][group][slot]
                np.testing.assert_array_equal(gvs, ovs.transpose(0, 2, 1))


# ---------------------------------------------------------------------------- gather (kernel 3)
@pytest.mark.parametrize("dtype", ["f16", "f32"])
def test_gather_ragged_matches_rows(gpu, dtype):
    import torch

    rng = np.random.default_rng(5)
    kv_dim, n_blocks = 512, 256
    g, o = _caches(1, kv_dim, n_blocks * BLOCK, dtype, rng.permutation(n_blocks))
    lens = {0: 1, 1: 15, 2: 16, 3: 17, 4: 333, 5: 1000, 6: 64}
    fill_sequences([("gpu", g), ("oracle", o)], lens, rng, kv_dim)
    seqs = [0, 1, 2, 3, 4, 5, 6, 9]  # seq 9 is unknown: length 0
    want_lens = [lens.get(s, 0) for s in seqs]
    tables, lens_arr = tables_and_lens(g, seqs, want_lens, stride=70)
    offs = np.concatenate([[0], np.cumsum(want_lens)[:-1]]).astype(np.int64)
    total = int(sum(want_lens))
    tdt = torch.float16 if dtype == "f16" else torch.float32
    k_out = torch.full((total + 3, kv_dim), -1.0, dtype=tdt, device=gpu)
    v_out = torch.full((total + 3, kv_dim), -1.0, dtype=tdt, device=gpu)
    g.gather(0, torch.from_numpy(tables).to(gpu), torch.from_numpy(lens_arr).to(gpu),
             torch.from_numpy(offs).to(gpu), k_out, v_out)
    kh = k_out.cpu().numpy()
    vh = v_out.cpu().numpy()
    npdt = np.uint16 if dtype == "f16" else np.uint32
    for s, n, off in zip(seqs, want_lens, offs):
        if n == 0:
            continue
        wk, wv = o.rows(0, s, n)
        np.testing.assert_array_equal(kh[off:off + n].view(npdt), _bits(wk))
        np.testing.assert_array_equal(vh[off:off + n].view(npdt), _bits(wv))
    # rows past the gathered total are untouched
    assert (kh[total:] == -1).all() and (vh[total:] == -1).all()


@pytest.mark.parametrize("dtype", ["f16", "q8_0"])
def test_empty_batches_change_nothing(gpu, dtype):
    """Every device op with an empty batch (n = 0: empty tensors, so null
    device pointers) succeeds, launches nothing and leaves the pools and the
    fault word as they were, as the reference's loops over an empty batch do
    (model.rs:380-475 with no tokens)."""
    import torch

    rng = np.random.default_rng(17)
    kv_dim, head_dim, n_heads = 256, 64, 8
    g, o = _caches(1, kv_dim, 32 * BLOCK, dtype, rng.permutation(32))
    fill_sequences([("gpu", g), ("oracle", o)], {0: 40, 1: 7}, rng, kv_dim)
    g.synchronize()
    before = [p.copy() for p in g.read_pool(0)]
    i32 = torch.zeros(0, dtype=torch.int32, device=gpu)
    f32 = torch.zeros((0, kv_dim), dtype=torch.float32, device=gpu)
    q = torch.zeros((0, n_heads * head_dim), dtype=torch.float32, device=gpu)
    tables = torch.zeros((0, 4), dtype=torch.int32, device=gpu)
    assert g.append_batch(np.zeros(0, np.uint32), np.zeros(0, np.uint64)).size == 0
    g.write_batch(0, i32, f32, f32)
    g.write_batch_ordered(0, i32, f32, f32, i32)
    g.rope_init(10000.0, head_dim, head_dim, False, 64)
    g.write_rope(0, i32, i32, f32, f32, q, n_heads)
    g.copy_blocks(torch.zeros((0, 2), dtype=torch.int32, device=gpu))
    assert g.decode_attention(0, q, tables, i32, n_heads, head_dim).numel() == 0
    assert g.decode_attention(0, q, tables, i32, n_heads, head_dim, noalloc=True).numel() == 0
    assert g.decode_attention_rows(0, q, i32, i32, n_heads, head_dim).numel() == 0
    assert g.slot_mapping(i32, torch.zeros(0, dtype=torch.int64, device=gpu)).numel() == 0
    if dtype == "f16":
        assert g.append_decode_attention(0, i32, f32, f32, q, tables, i32, n_heads, head_dim).numel() == 0
        g.gather(0, tables, i32, torch.zeros(0, dtype=torch.int64, device=gpu),
                 torch.zeros((1, kv_dim), dtype=torch.float16, device=gpu),
                 torch.zeros((1, kv_dim), dtype=torch.float16, device=gpu))
    g.plan_attention([], [], n_heads, head_dim)
    assert g.planned_attention(0, q).numel() == 0
    g.synchronize()  # no fault recorded
    after = g.read_pool(0)
    for b, a in zip(before, after):
        np.testing.assert_array_equal(a.view(np.uint8), b.view(np.uint8))


def test_rows_host_convenience(gpu):
    rng = np.random.default_rng(6)
    g, o = _caches(2, 128, 64 * BLOCK, "f16", rng.permutation(64))
    fill_sequences([("gpu", g), ("oracle", o)], {4: 77, 8: 3}, rng, 128, layers=(0, 1))
    for layer in (0, 1):
        for s, n in ((4, 77), (4, 50), (8, 3)):
            gk, gv = g.rows(layer, s, n)
            ok, ov = o.rows(layer, s, n)
            np.testing.assert_array_equal(gk, ok)
            np.testing.assert_array_equal(gv, ov)


# ---------------------------------------------------------------------------- attention (kernel 4)
def _attention_case(gpu, dtype, head_dim, group, n_kv_heads, lens, partition, seed):
    import torch

    rng = np.random.default_rng(seed)
    kv_dim = n_kv_heads * head_dim
    n_heads = group * n_kv_heads
    blocks = sum(-(-n // BLOCK) for n in lens) + 8
    g, o = _caches(1, kv_dim, blocks * BLOCK, dtype, rng.permutation(blocks))
    if partition:
        g.set_attention_partition(partition)
    fill_sequences([("gpu", g), ("oracle", o)], dict(enumerate(lens)), rng, kv_dim)
    seqs = list(range(len(lens)))
    tables, lens_arr = tables_and_lens(g, seqs, lens)
    q = rng.standard_normal((len(lens), n_heads * head_dim), dtype=np.float32)
    out = g.decode_attention(0, torch.from_numpy(q).to(gpu), torch.from_numpy(tables).to(gpu),
                             torch.from_numpy(lens_arr).to(gpu), n_heads, head_dim).cpu().numpy()
    want = o.attention_tables(0, tables, lens_arr, q, n_heads, head_dim, threads=8)
    return out, want


@pytest.mark.parametrize("dtype,head_dim", [("f16", 128), ("f16", 64), ("f32", 64), ("f32", 128)])
@pytest.mark.parametrize("group", [1, 4, 7, 8])
def test_attention_shapes(gpu, dtype, head_dim, group):
    lens = [1, 2, 15, 16, 17, 63, 300, 1031]
    out, want = _attention_case(gpu, dtype, head_dim, group, 2, lens, 0, seed=group * 10 + head_dim)
    attention_close(out, want, dtype)


@pytest.mark.parametrize("head_dim", [64, 128])
@pytest.mark.parametrize("group,n_kv", [(2, 2), (3, 4), (2, 3), (4, 5), (1, 1), (5, 4), (6, 2),
                                         (7, 4), (7, 3), (8, 2)])
def test_attention_head_pairs_f16(gpu, head_dim, group, n_kv):
    """f16 waves read two adjacent kv heads when the group has at most 4
    query heads and the kv heads pair up (even count), one otherwise."""
    lens = [1, 16, 33, 300, 1031, 2100]
    out, want = _attention_case(gpu, "f16", head_dim, group, n_kv, lens, 0, seed=group * 7 + n_kv)
    attention_close(out, want, "f16")


@pytest.mark.parametrize("partition", [0, 64, 128])
def test_attention_head_pairs_large_batch(gpu, partition):
    """64 queries of the Llama-3-8B shape (f16 waves of two kv heads, one
    wave per SIMD) against the oracle, with the default and fixed
    partitions."""
    rng = np.random.default_rng(partition + 5)
    lens = [int(x) for x in rng.integers(1, 400, size=64)]
    out, want = _attention_case(gpu, "f16", 128, 4, 8, lens, partition, seed=partition + 6)
    attention_close(out, want, "f16")


@pytest.mark.parametrize("partition", [64, 128, 256, 512, 4096])
def test_attention_partitions(gpu, partition):
    lens = [5, 64, 65, 257, 700, 2049]
    out, want = _attention_case(gpu, "f16", 128, 4, 8, lens, partition, seed=partition)
    attention_close(out, want, "f16")


@pytest.mark.parametrize("dtype,engine,lens,fixed", [
    ("f16", "auto", [1537, 1600, 1580], 448),     # ceil(len/4) in (384, 448]
    ("f16", "auto", [2, 40, 255, 256], 64),       # the 64-token floor
    ("f16", "auto", [2048, 2000, 1985], 512),     # four equal partitions up to 2048 tokens
    ("f16", "auto", [2049, 3000, 4096], 1024),    # f16 matrix cores: 1024 tokens past 2048
    ("f16", "auto", [4097, 9000, 5000], 1024),    # beyond 4096 tokens
    ("f16", "valu", [3000, 2990, 2945], 768),     # the vector-ALU engine: four up to 4096
    ("f16", "valu", [4097, 5000], 1024),
    ("q8_0", "auto", [3000, 2990, 2945], 768),    # q8_0 pools: four up to 4096
    ("q8_0", "auto", [4097, 6000], 1024),
    ("f32", "auto", [3000, 2990], 768),           # f32 pools: four up to 4096
])
def test_attention_default_policy_is_per_query_partition(gpu, dtype, engine, lens, fixed):
    """With no fixed partition a query of len tokens is split into partitions
    of roundup64(ceil(len/4)) tokens (at least 64), and of 1024 tokens past
    4096 tokens, or past 2048 tokens on f16 pools on the matrix cores: the
    output equals, bit for bit, the one with that partition fixed."""
    import torch

    rng = np.random.default_rng(fixed + len(lens))
    kv_dim = 1024
    blocks = sum(-(-n // BLOCK) for n in lens) + 4
    g, o = _caches(1, kv_dim, blocks * BLOCK, dtype, rng.permutation(blocks))
    if engine != "auto":
        g.set_attention_engine(engine)
    fill_sequences([("gpu", g), ("oracle", o)], dict(enumerate(lens)), rng, kv_dim)
    tables, la = tables_and_lens(g, list(range(len(lens))), lens)
    q = torch.from_numpy(rng.standard_normal((len(lens), 32 * 128), dtype=np.float32)).to(gpu)
    dt, dl = torch.from_numpy(tables).to(gpu), torch.from_numpy(la).to(gpu)
    auto = g.decode_attention(0, q, dt, dl, 32, 128).cpu().numpy()
    g.set_attention_partition(fixed)
    pinned = g.decode_attention(0, q, dt, dl, 32, 128).cpu().numpy()
    np.testing.assert_array_equal(auto.view(np.uint32), pinned.view(np.uint32))
    want = o.attention_tables(0, tables, la, q.cpu().numpy(), 32, 128, threads=8)
    attention_close(auto, want, dtype)


def test_attention_config_tinyllama_f32(gpu):
    """TinyLlama-shaped layer, f32 KV: 32 q heads, 4 kv heads, head_dim 64;
    4 sequences with contexts U[128,512] over a permuted 1024-block pool;
    append one token per sequence, then one decode step (scale 1/8)."""
    import torch

    from langtrain_studio_amd import KvCache
    from oracle import OracleKv

    rng = np.random.default_rng(11)
    n_heads, n_kv, hd = 32, 4, 64
    kv_dim = n_kv * hd
    g = KvCache(1, kv_dim, 1024 * BLOCK, dtype="f32", device=0)
    o = OracleKv(1, kv_dim, 1024 * BLOCK, dtype="f32")
    order = rng.permutation(1024)
    g.init_free_order(order)
    o.init_free_order(order)
    ctx = rng.integers(128, 513, 4)
    fill_sequences([("gpu", g), ("oracle", o)], {s: int(n) for s, n in enumerate(ctx)}, rng, kv_dim)
    seqs = np.arange(4, dtype=np.uint32)
    pos = ctx.astype(np.uint64)
    sm = g.append_batch(seqs, pos)
    np.testing.assert_array_equal(sm, o.append_batch(seqs, pos))
    k = rng.standard_normal((4, kv_dim), dtype=np.float32)
    v = rng.standard_normal((4, kv_dim), dtype=np.float32)
    g.write_batch(0, torch.from_numpy(sm).to(gpu), torch.from_numpy(k).to(gpu), torch.from_numpy(v).to(gpu))
    o.write_batch(0, sm, k, v)
    q = rng.standard_normal((4, n_heads * hd), dtype=np.float32)
    tables, lens = tables_and_lens(g, seqs, pos + 1)
    out = g.decode_attention(0, torch.from_numpy(q).to(gpu), torch.from_numpy(tables).to(gpu),
                             torch.from_numpy(lens).to(gpu), n_heads, hd, scale=0.125).cpu().numpy()
    want = o.attention(0, seqs, pos, q, n_heads, hd, scale=0.125, threads=8)
    attention_close(out, want, "f32")
    _assert_pools_equal(g, o, (0,))


def test_attention_single_position_returns_v_row(gpu):
    """len == 1: the softmax weight is exactly 1, so the output is the V row."""
    import torch

    from oracle import f16_to_f32

    rng = np.random.default_rng(12)
    g, o = _caches(1, 256, 8 * BLOCK, "f16")
    _, rows = fill_sequences([("gpu", g), ("oracle", o)], {0: 1, 1: 1}, rng, 256)
    tables, lens = tables_and_lens(g, [0, 1], [1, 1])
    q = rng.standard_normal((2, 8 * 128), dtype=np.float32)
    out = g.decode_attention(0, torch.from_numpy(q).to(gpu), torch.from_numpy(tables).to(gpu),
                             torch.from_numpy(lens).to(gpu), 8, 128).cpu().numpy()
    vrow = f16_to_f32(o.rows(0, 0, 1)[1][0]), f16_to_f32(o.rows(0, 1, 1)[1][0])
    for i in range(2):
        want = np.concatenate([np.tile(vrow[i][h * 128:(h + 1) * 128], 4) for h in range(2)])
        np.testing.assert_array_equal(out[i], want)


def test_attention_equal_keys_average_values(gpu):
    """All K rows equal: uniform weights, so the output is the mean of V."""
    import torch

    from oracle import f16_to_f32

    rng = np.random.default_rng(13)
    kv_dim, n = 128, 200
    g, o = _caches(1, kv_dim, 16 * BLOCK, "f16")
    sm = g.append_batch([0] * n, np.arange(n))
    o.append_batch([0] * n, np.arange(n))
    k = np.tile(rng.standard_normal((1, kv_dim), dtype=np.float32), (n, 1))
    v = rng.standard_normal((n, kv_dim), dtype=np.float32)
    g.write_batch(0, torch.from_numpy(sm).to(gpu), torch.from_numpy(k).to(gpu), torch.from_numpy(v).to(gpu))
    tables, lens = tables_and_lens(g, [0], [n])
    q = rng.standard_normal((1, 4 * 128), dtype=np.float32)
    out = g.decode_attention(0, torch.from_numpy(q).to(gpu), torch.from_numpy(tables).to(gpu),
                             torch.from_numpy(lens).to(gpu), 4, 128).cpu().numpy()
    vm = f16_to_f32(g.rows(0, 0, n)[1]).astype(np.float64).mean(0)
    np.testing.assert_allclose(out[0], np.tile(vm, 4), atol=2e-5, rtol=0)


def test_attention_physical_placement_invariance(gpu):
    """The same logical contents under two different block placements give
    bit-identical outputs (the kernel depends only on the block table)."""
    import torch

    from langtrain_studio_amd import KvCache

    rng = np.random.default_rng(14)
    lens = [700, 33, 1500, 16]
    kv_dim, blocks = 1024, 256
    outs = []
    q = rng.standard_normal((4, 32 * 128), dtype=np.float32)
    data_seed = 99
    for order_seed in (1, 2):
        g = KvCache(1, kv_dim, blocks * BLOCK, device=0)
        g.init_free_order(np.random.default_rng(order_seed).permutation(blocks))
        fill_sequences([("gpu", g)], dict(enumerate(lens)), np.random.default_rng(data_seed), kv_dim)
        tables, la = tables_and_lens(g, range(4), lens)
        outs.append(g.decode_attention(0, torch.from_numpy(q).to(gpu), torch.from_numpy(tables).to(gpu),
                                       torch.from_numpy(la).to(gpu), 32, 128).cpu().numpy())
        assert not np.array_equal(tables[:, 0], np.arange(4))  # placements really differ
    np.testing.assert_array_equal(outs[0], outs[1])


@pytest.mark.parametrize("dtype", ["f16", "q8_0", "f32"])
@pytest.mark.parametrize("n_batch", [5, 200, 300])
def test_attention_batch_independence(gpu, dtype, n_batch):
    """A query's output is bit-identical alone and inside a batch (the
    reference's batching property, engine/README.md:102), for small batches
    and for ones that fill every SIMD: batches of up to 256 queries take
    their work items longest first (200: four 64-query rounds of the order
    scan), larger ones in query order, a query alone in query order."""
    import torch

    rng = np.random.default_rng(15 + n_batch)
    lens = [2000, 9, 513, 4096, 77] + [int(x) for x in rng.integers(1, 600, size=n_batch - 5)]
    blocks = sum(-(-n // BLOCK) for n in lens) + 8
    g, _ = _caches(1, 1024, blocks * BLOCK, dtype, rng.permutation(blocks))
    fill_sequences([("gpu", g)], dict(enumerate(lens)), rng, 1024)
    q = rng.standard_normal((n_batch, 32 * 128), dtype=np.float32)
    tables, la = tables_and_lens(g, range(n_batch), lens)
    dq, dt, dl = (torch.from_numpy(x).to(gpu) for x in (q, tables, la))
    full = g.decode_attention(0, dq, dt, dl, 32, 128).cpu().numpy()
    for i in range(5):
        one = g.decode_attention(0, dq[i:i + 1].contiguous(), dt[i:i + 1, :-(-lens[i] // BLOCK)].contiguous(),
                                 dl[i:i + 1].contiguous(), 32, 128).cpu().numpy()
        np.testing.assert_array_equal(one[0].view(np.uint32), full[i].view(np.uint32))


@pytest.mark.parametrize("dtype", ["f16", "q8_0"])
def test_attention_partition_runs_match_single_partitions(gpu, dtype):
    """A batch with at least twice as many partition items as the chip holds
    waves (fixed 64-token partitions, 24 queries of 1.5-3k tokens: ~4k-7k
    items times the kv-head groups on 1024 or 2048 wave slots) has each wave
    stream a run of consecutive partitions, writing each partition's partial
    as it passes; every query's output equals, bit for bit, the one it gets
    alone (a wave per partition), and the batch is within the tolerance of
    the oracle."""
    import torch

    rng = np.random.default_rng(77)
    lens = [int(x) for x in rng.integers(1500, 3000, size=24)]
    lens[3] = 1  # a one-token query among them
    blocks = sum(-(-n // BLOCK) for n in lens) + 8
    g, o = _caches(1, 1024, blocks * BLOCK, dtype, rng.permutation(blocks))
    g.set_attention_partition(64)
    fill_sequences([("gpu", g), ("oracle", o)], dict(enumerate(lens)), rng, 1024)
    q = rng.standard_normal((len(lens), 32 * 128), dtype=np.float32)
    tables, la = tables_and_lens(g, range(len(lens)), lens)
    dq, dt, dl = (torch.from_numpy(x).to(gpu) for x in (q, tables, la))
    full = g.decode_attention(0, dq, dt, dl, 32, 128).cpu().numpy()
    for i in (0, 3, 11, 23):
        one = g.decode_attention(0, dq[i:i + 1].contiguous(), dt[i:i + 1].contiguous(),
                                 dl[i:i + 1].contiguous(), 32, 128).cpu().numpy()
        np.testing.assert_array_equal(one[0].view(np.uint32), full[i].view(np.uint32))
    # the same batch by resident rows (the runs read the same table entries)
    rows = torch.from_numpy(g.seq_rows(list(range(len(lens)))).astype(np.int32)).to(gpu)
    by_rows = g.decode_attention_rows(0, dq, rows, dl, 32, 128).cpu().numpy()
    np.testing.assert_array_equal(by_rows.view(np.uint32), full.view(np.uint32))
    want = o.attention_tables(0, tables, la, q, 32, 128, threads=8)
    attention_close(full, want, dtype)


def test_attention_workspace_reuse_across_shapes(gpu):
    """Calls of different batch sizes and table widths alternate on one cache
    (its partition workspace and counters are reused); each must match."""
    import torch

    rng = np.random.default_rng(17)
    lens = [3000, 40, 700, 1500, 5, 2222]
    g, o = _caches(1, 1024, 800 * BLOCK, "f16", rng.permutation(800))
    fill_sequences([("gpu", g), ("oracle", o)], dict(enumerate(lens)), rng, 1024)
    q = rng.standard_normal((6, 32 * 128), dtype=np.float32)
    for pick in ([0, 1, 2, 3, 4, 5], [1], [3, 0], [4], [5, 2, 1], [0, 1, 2, 3, 4, 5], [2]):
        tables, la = tables_and_lens(g, pick, [lens[i] for i in pick])
        qq = q[pick]
        out = g.decode_attention(0, torch.from_numpy(qq).to(gpu), torch.from_numpy(tables).to(gpu),
                                 torch.from_numpy(la).to(gpu), 32, 128).cpu().numpy()
        want = o.attention_tables(0, tables, la, qq, 32, 128, threads=8)
        attention_close(out, want, "f16")


def test_attention_stale_nonfinite_slots_are_ignored(gpu):
    """Cells past a sequence's length may hold stale non-finite data; they
    must not leak into the output."""
    import torch

    rng = np.random.default_rng(16)
    kv_dim = 128
    g, o = _caches(1, kv_dim, 8 * BLOCK, "f16")
    sm = g.append_batch([0] * 16, np.arange(16))
    o.append_batch([0] * 16, np.arange(16))
    k = rng.standard_normal((16, kv_dim), dtype=np.float32)
    v = rng.standard_normal((16, kv_dim), dtype=np.float32)
    k[9:] = np.inf
    v[9:] = np.nan
    g.write_batch(0, torch.from_numpy(sm).to(gpu), torch.from_numpy(k).to(gpu), torch.from_numpy(v).to(gpu))
    o.write_batch(0, sm, k, v)
    g.truncate(0, 9)
    o.truncate(0, 9)
    tables, lens = tables_and_lens(g, [0], [9])
    q = rng.standard_normal((1, 128), dtype=np.float32)
    out = g.decode_attention(0, torch.from_numpy(q).to(gpu), torch.from_numpy(tables).to(gpu),
                             torch.from_numpy(lens).to(gpu), 1, 128).cpu().numpy()
    want = o.attention_tables(0, tables, lens, q, 1, 128)
    attention_close(out, want, "f16")


def test_attention_zero_length_gives_zeros(gpu):
    import torch

    g, _ = _caches(1, 128, 8 * BLOCK, "f16")
    q = torch.ones((2, 256), device=gpu)
    tables = torch.full((2, 4), -1, dtype=torch.int32, device=gpu)
    lens = torch.zeros(2, dtype=torch.int32, device=gpu)
    out = g.decode_attention(0, q, tables, lens, 2, 128)
    assert (out.cpu().numpy() == 0).all()


# ---------------------------------------------------------------------------- fused RoPE + append
@pytest.mark.parametrize("dtype,n_heads,n_kv,head_dim,rope_dim,neox,base", [
    ("f16", 32, 8, 128, 128, False, 500000.0),   # Llama-3-8B
    ("f16", 28, 4, 128, 128, True, 1000000.0),   # Qwen2.5-7B (NeoX pairs)
    ("f16", 8, 2, 128, 64, True, 10000.0),       # partial rotary
    ("f32", 32, 4, 64, 64, False, 10000.0),      # TinyLlama, f32 cells
])
def test_write_rope_bit_exact(gpu, dtype, n_heads, n_kv, head_dim, rope_dim, neox, base):
    """model.rs:414-429 fused: q rotated in place and k rotated into its cell
    (then f32->f16 RNE), v appended; pools and q bit-identical to the oracle
    for positions up to 32767, including skipped slots."""
    import torch

    rng = np.random.default_rng(head_dim + rope_dim + n_heads)
    kv_dim = n_kv * head_dim
    g, o = _caches(1, kv_dim, 600 * BLOCK, dtype, rng.permutation(600))
    g.rope_init(base, rope_dim, head_dim, neox, 32768)
    lens = {0: 700, 1: 1200, 2: 33}
    seqs = np.concatenate([np.full(n, s, dtype=np.uint32) for s, n in lens.items()])
    pos = np.concatenate([np.arange(n, dtype=np.uint64) for n in lens.values()])
    sm = g.append_batch(seqs, pos)
    assert np.array_equal(sm, o.append_batch(seqs, pos))
    sm[5] = -1  # a skipped row
    n = sm.size
    k = rng.standard_normal((n, kv_dim), dtype=np.float32) * 3
    v = rng.standard_normal((n, kv_dim), dtype=np.float32)
    q = rng.standard_normal((n, n_heads * head_dim), dtype=np.float32)
    p32 = pos.astype(np.int32) * 23 % 32768  # positions need not follow the cells here
    dq = torch.from_numpy(q).to(gpu)
    g.write_rope(0, torch.from_numpy(sm).to(gpu), torch.from_numpy(p32).to(gpu), torch.from_numpy(k).to(gpu),
                 torch.from_numpy(v).to(gpu), q=dq, n_heads=n_heads)
    qo = q.copy()
    o.write_rope_batch(0, sm, p32, k, v, base, rope_dim, head_dim, neox, q=qo, n_heads=n_heads)
    np.testing.assert_array_equal(_bits(dq.cpu().numpy()), _bits(qo))
    gk, gv = g.read_pool(0)
    ok, ov = o.pool(0)
    np.testing.assert_array_equal(_bits(gk), _bits(ok))
    np.testing.assert_array_equal(_bits(gv), _bits(ov))


def test_write_rope_equals_write_of_rotated_rows(gpu):
    """Without q, the fused launch writes exactly what ltkv_write writes for
    rows rotated by the oracle; positions outside the table write nothing."""
    import torch

    rng = np.random.default_rng(7)
    kv_dim, hd = 512, 128
    g, o = _caches(1, kv_dim, 64 * BLOCK, "f16")
    g.rope_init(10000.0, hd, hd, False, 4096)
    sm = g.append_batch(np.zeros(40, np.uint32), np.arange(40, dtype=np.uint64))
    o.append_batch(np.zeros(40, np.uint32), np.arange(40, dtype=np.uint64))
    k = rng.standard_normal((40, kv_dim), dtype=np.float32)
    v = rng.standard_normal((40, kv_dim), dtype=np.float32)
    pos = np.arange(40, dtype=np.int32) * 100
    pos[3] = 4096  # outside the table: skipped
    pos[4] = -1
    g.write_rope(0, torch.from_numpy(sm).to(gpu), torch.from_numpy(pos).to(gpu), torch.from_numpy(k).to(gpu),
                 torch.from_numpy(v).to(gpu))
    keep = np.ones(40, bool)
    keep[[3, 4]] = False
    sm_o = sm.copy()
    sm_o[~keep] = -1
    o.write_rope_batch(0, sm_o, np.where(keep, pos, 0), k, v, 10000.0, hd, hd, False)
    gk, gv = g.read_pool(0)
    ok, ov = o.pool(0)
    np.testing.assert_array_equal(gk, ok)
    np.testing.assert_array_equal(gv, ov)
