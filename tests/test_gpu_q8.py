"""Q8_0 KV cache (int8 quants plus one f16 scale per 32 elements) through the
C ABI against the oracle: append and copy-on-write bit-exact in quants and
scales (quant.rs:785-791 quantisation, quant.rs:188-193 block format);
attention within max abs 1e-3 and relative L2 1e-3 of the oracle's attention
(model.rs:431-475) over the same dequantised rows d * q."""

from __future__ import annotations

import numpy as np
import pytest

from helpers import BLOCK, attention_close, fill_sequences, tables_and_lens

pytestmark = pytest.mark.gpu


def _caches(n_layers, kv_dim, n_tokens, order=None):
    from langtrain_studio_amd import KvCache
    from oracle import OracleKv

    g = KvCache(n_layers, kv_dim, n_tokens, dtype="q8_0", device=0)
    o = OracleKv(n_layers, kv_dim, n_tokens, dtype="q8_0")
    if order is not None:
        g.init_free_order(order)
        o.init_free_order(order)
    return g, o


def _assert_q8_equal(g, o, layers):
    for layer in layers:
        gk, gv = g.read_pool(layer)
        ok, ov = o.pool(layer)
        np.testing.assert_array_equal(gk, ok, err_msg=f"K quants, layer {layer}")
        np.testing.assert_array_equal(gv, ov, err_msg=f"V quants, layer {layer}")
        gks, gvs = g.read_scales(layer)  # [block][group][slot]
        oks, ovs = o.scales(layer)       # [block][slot][group]
        np.testing.assert_array_equal(gks, oks.transpose(0, 2, 1), err_msg=f"K scales, layer {layer}")
        np.testing.assert_array_equal(gvs, ovs.transpose(0, 2, 1), err_msg=f"V scales, layer {layer}")


def q8_rows(rng, n, kv_dim):
    """Rows whose 32-element blocks hit each case of quant.rs:785-791: exact
    ties at amax 127 (round half away from zero), NaN elements (ignored by
    the amax, quantised to 0), +-inf (d = inf, id = 0), zeros (d = 0), a
    subnormal amax (1 / d overflows, quants saturate at 127 / -128), a
    negative maximum, huge values (d overflows f16), an all-NaN block, and
    ordinary blocks."""
    x = (rng.standard_normal((n, kv_dim)) * 3).astype(np.float32)
    blocks = x.reshape(n, kv_dim // 32, 32)
    ties = np.array([0.5, -0.5, 1.5, -1.5, 2.5, -2.5, 126.5, -126.5, 63.5, -63.5, 1.0, 0.0], np.float32)
    tiny = np.array([1e-40, -1e-40, 5e-41, -7e-41, 0.0], np.float32)
    for r in range(n):
        for b in range(blocks.shape[1]):
            blk = blocks[r, b]
            kind = (r * blocks.shape[1] + b) % 9
            if kind == 0:
                blk[:] = rng.choice(ties, 32)
                blk[rng.integers(0, 32)] = 127.0 if rng.random() < 0.5 else -127.0
            elif kind == 1:
                blk[rng.integers(0, 32, 3)] = np.nan
            elif kind == 2:
                blk[rng.integers(0, 32)] = np.inf if rng.random() < 0.5 else -np.inf
            elif kind == 3:
                blk[:] = rng.choice(np.array([0.0, -0.0], np.float32), 32)
            elif kind == 4:
                blk[:] = rng.choice(tiny, 32)
            elif kind == 5:
                blk[rng.integers(0, 32)] = -50.0
            elif kind == 6:
                blk *= np.float32(1e37)
            elif kind == 7:
                blk[:] = np.nan
    return x


def _write(caches, sm, layer, k, v):
    import torch

    for kind, c in caches:
        if kind == "gpu":
            dev = torch.device("cuda", c.device)
            c.write_batch(layer, torch.from_numpy(sm).to(dev), torch.from_numpy(k).to(dev),
                          torch.from_numpy(v).to(dev))
        else:
            c.write_batch(layer, sm, k, v)


# ---------------------------------------------------------------------------- append (kernel 1)
@pytest.mark.parametrize("kv_dim", [32, 256, 1024])
def test_q8_write_bitexact_special_blocks(gpu, kv_dim):
    rng = np.random.default_rng(kv_dim)
    n_blocks = 48
    g, o = _caches(2, kv_dim, n_blocks * BLOCK, rng.permutation(n_blocks))
    seqs = np.concatenate([np.full(n, s, np.uint32) for s, n in ((0, 37), (5, 16), (9, 100), (3, 1))])
    pos = np.concatenate([np.arange(n, dtype=np.uint64) for n in (37, 16, 100, 1)])
    sm = g.append_batch(seqs, pos)
    np.testing.assert_array_equal(o.append_batch(seqs, pos), sm)
    for layer in (0, 1):
        _write([("gpu", g), ("oracle", o)], sm, layer, q8_rows(rng, sm.size, kv_dim),
               q8_rows(rng, sm.size, kv_dim))
    g.synchronize()
    _assert_q8_equal(g, o, (0, 1))
    # every case of the quantiser occurred
    k, _ = g.read_pool(0)
    assert (k == 127).any() and (k == -128).any() and (k == 0).any()


def test_q8_write_skips_bad_slots_and_host_row(gpu):
    import torch

    from oracle import OracleKv

    from langtrain_studio_amd import KvCache

    g = KvCache(1, 64, 4 * BLOCK, dtype="q8_0", device=0)
    o = OracleKv(1, 64, 4 * BLOCK, dtype="q8_0")
    sm = torch.tensor([-1, 3, 4 * BLOCK, 5, -7], dtype=torch.int32, device=gpu)
    k = torch.full((5, 64), 2.0, device=gpu)
    g.write_batch(0, sm, k, k)
    o.write_batch(0, np.array([-1, 3, -1, 5, -1], np.int32), np.full((5, 64), 2.0, np.float32),
                  np.full((5, 64), 2.0, np.float32))
    row = np.linspace(-4, 4, 64).astype(np.float32)
    g.write(0, 2, 7, row, -row)
    o.write(0, 2, 7, row, -row)
    _assert_q8_equal(g, o, (0,))
    gk, _ = g.read_pool(0)
    assert (gk.reshape(-1, 64)[3] == 127).all()  # 2.0 / (2.0 / 127)


# ---------------------------------------------------------------------------- copy-on-write (kernel 2)
def test_q8_copy_on_write_carries_scales(gpu):
    rng = np.random.default_rng(12)
    kv_dim, n_blocks, layers = 256, 96, (0, 1)
    g, o = _caches(2, kv_dim, n_blocks * BLOCK, rng.permutation(n_blocks))
    both = [("gpu", g), ("oracle", o)]
    fill_sequences(both, {5: 40, 6: 3}, rng, kv_dim, layers=layers)
    for rnd in range(3):
        for s in (1, 2, 3):
            g.share(5, s, 37 + rnd)
            o.share(5, s, 37 + rnd)
        seqs = [1, 2, 3, 1, 2]
        lens = {s: g.len(s) for s in (1, 2, 3)}
        pos = []
        for s in seqs:
            pos.append(lens[s])
            lens[s] += 1
        sm = g.append_batch(seqs, pos)
        np.testing.assert_array_equal(o.append_batch(seqs, pos), sm)
        for layer in layers:
            _write(both, sm, layer, q8_rows(rng, len(seqs), kv_dim), q8_rows(rng, len(seqs), kv_dim))
        assert g.cow_copies() == o.cow_copies()
        _assert_q8_equal(g, o, layers)
    assert g.cow_copies() >= 9


def test_q8_copy_blocks_bulk(gpu):
    import torch

    from langtrain_studio_amd import KvCache

    rng = np.random.default_rng(13)
    kv_dim, n_blocks = 512, 200
    g = KvCache(2, kv_dim, n_blocks * BLOCK, dtype="q8_0", device=0)
    fill_sequences([("gpu", g)], {0: n_blocks * BLOCK}, rng, kv_dim, layers=(0, 1))
    before = [(g.read_pool(l), g.read_scales(l)) for l in (0, 1)]
    perm = rng.permutation(n_blocks)
    src, dst = perm[:70], perm[70:140]
    g.copy_blocks(torch.from_numpy(np.stack([src, dst], 1).astype(np.int32)).to(gpu))
    for l in (0, 1):
        for got, was in zip(g.read_pool(l) + g.read_scales(l), before[l][0] + before[l][1]):
            want = was.copy()
            want[dst] = was[src]
            np.testing.assert_array_equal(got, want)


# ---------------------------------------------------------------------------- attention (kernel 4)
def _q8_attention(gpu, head_dim, group, n_kv_heads, lens, partition, seed):
    import torch

    rng = np.random.default_rng(seed)
    kv_dim = n_kv_heads * head_dim
    n_heads = group * n_kv_heads
    blocks = sum(-(-n // BLOCK) for n in lens) + 8
    g, o = _caches(1, kv_dim, blocks * BLOCK, rng.permutation(blocks))
    if partition:
        g.set_attention_partition(partition)
    fill_sequences([("gpu", g), ("oracle", o)], dict(enumerate(lens)), rng, kv_dim)
    tables, lens_arr = tables_and_lens(g, list(range(len(lens))), lens)
    q = rng.standard_normal((len(lens), n_heads * head_dim), dtype=np.float32)
    out = g.decode_attention(0, torch.from_numpy(q).to(gpu), torch.from_numpy(tables).to(gpu),
                             torch.from_numpy(lens_arr).to(gpu), n_heads, head_dim).cpu().numpy()
    want = o.attention_tables(0, tables, lens_arr, q, n_heads, head_dim, threads=8)
    return out, want


@pytest.mark.parametrize("head_dim", [64, 128])
@pytest.mark.parametrize("group", [1, 4, 7, 8])
def test_q8_attention_shapes(gpu, head_dim, group):
    lens = [1, 2, 15, 16, 17, 63, 300, 1031]
    out, want = _q8_attention(gpu, head_dim, group, 2, lens, 0, seed=group * 10 + head_dim)
    attention_close(out, want, "q8_0")


@pytest.mark.parametrize("head_dim", [64, 128])
@pytest.mark.parametrize("group,n_kv", [(2, 2), (3, 4), (2, 3), (4, 5), (6, 2), (7, 4), (7, 3)])
def test_q8_attention_head_pairs(gpu, head_dim, group, n_kv):
    """q8_0 waves over two adjacent kv heads (even count, group at most 4)
    and over one (odd count or larger group)."""
    lens = [1, 16, 33, 300, 1031, 2100]
    out, want = _q8_attention(gpu, head_dim, group, n_kv, lens, 0, seed=group * 7 + n_kv)
    attention_close(out, want, "q8_0")


@pytest.mark.parametrize("partition", [64, 512, 4096])
def test_q8_attention_partitions_llama_shape(gpu, partition):
    lens = [5, 64, 65, 257, 700, 2049]
    out, want = _q8_attention(gpu, 128, 4, 8, lens, partition, seed=partition)
    attention_close(out, want, "q8_0")


@pytest.mark.parametrize("head_dim", [64, 128])
def test_q8_attention_ignores_stale_nonfinite_slots(gpu, head_dim):
    """Slots past a query's length hold inf rows (scale inf, quants 0, so
    d * q is NaN): the result must equal the one over the valid prefix."""
    import torch

    rng = np.random.default_rng(head_dim + 1)
    kv_dim, n_heads = 2 * head_dim, 8
    g, o = _caches(1, kv_dim, 8 * BLOCK)
    sm = g.append_batch([0] * 20, np.arange(20))
    o.append_batch([0] * 20, np.arange(20))
    k = rng.standard_normal((20, kv_dim), dtype=np.float32)
    v = rng.standard_normal((20, kv_dim), dtype=np.float32)
    k[17:] = np.inf
    v[17:] = np.inf
    _write([("gpu", g), ("oracle", o)], sm, 0, k, v)
    tables, lens = tables_and_lens(g, [0], [17])
    q = rng.standard_normal((1, n_heads * head_dim), dtype=np.float32)
    out = g.decode_attention(0, torch.from_numpy(q).to(gpu), torch.from_numpy(tables).to(gpu),
                             torch.from_numpy(lens).to(gpu), n_heads, head_dim).cpu().numpy()
    want = o.attention_tables(0, tables, lens, q, n_heads, head_dim)
    attention_close(out, want, "q8_0")


def test_q8_planned_attention_equals_decode(gpu):
    """The planned path on a q8_0 cache: without groups it gives the decode
    kernel's bits; with the forks grouped it stays within the bar."""
    import torch

    rng = np.random.default_rng(31)
    kv_dim, head_dim, n_heads = 1024, 128, 32
    g, o = _caches(1, kv_dim, 600 * BLOCK, rng.permutation(600))
    fill_sequences([("gpu", g), ("oracle", o)], {0: 2000}, rng, kv_dim)
    for s in range(1, 9):
        g.share(0, s, 1990)
        o.share(0, s, 1990)
    seqs = list(range(1, 9))
    pos = [1990] * 8
    from helpers import append_rows
    append_rows([("gpu", g), ("oracle", o)], seqs, pos, rng, kv_dim)
    lens = [g.len(s) for s in seqs]
    st = g.plan_attention(seqs, lens, n_heads, head_dim, shared_prefix=False)
    assert st["groups"] == 0
    q = torch.from_numpy(rng.standard_normal((8, n_heads * head_dim), dtype=np.float32)).to(gpu)
    got = g.planned_attention(0, q).cpu().numpy()
    tables, la = tables_and_lens(g, seqs, lens)
    ref = g.decode_attention(0, q, torch.from_numpy(tables).to(gpu), torch.from_numpy(la).to(gpu),
                             n_heads, head_dim).cpu().numpy()
    np.testing.assert_array_equal(got, ref)
    want = o.attention_tables(0, tables, la, q.cpu().numpy(), n_heads, head_dim, threads=8)
    attention_close(got, want, "q8_0")
    st = g.plan_attention(seqs, lens, n_heads, head_dim)
    assert st["groups"] == 1
    attention_close(g.planned_attention(0, q).cpu().numpy(), want, "q8_0")


def test_q8_unsupported_ops_raise(gpu):
    import torch

    from langtrain_studio_amd import KvCache, KvError

    with pytest.raises(KvError, match="multiple of 32"):
        KvCache(1, 48, 64, dtype="q8_0", device=0)
    g = KvCache(1, 64, 4 * BLOCK, dtype="q8_0", device=0)
    g.append_batch([0] * 3, np.arange(3))
    with pytest.raises(KvError, match="Q8_0"):
        g.rows(0, 0, 3)
    t = torch.zeros((1, 1), dtype=torch.int32, device=gpu)
    l = torch.ones(1, dtype=torch.int32, device=gpu)
    off = torch.zeros(1, dtype=torch.int64, device=gpu)
    out = torch.zeros((4, 64), dtype=torch.int8, device=gpu)
    with pytest.raises(KvError, match="Q8_0"):
        g.gather(0, t, l, off, out, out.clone())
    h = KvCache(1, 96, 4 * BLOCK, dtype="q8_0", device=0)
    h.rope_init(10000.0, 48, 48, False, 16)  # head_dim 48: not whole scale groups
    x = torch.zeros((1, 96), device=gpu)
    with pytest.raises(KvError, match="multiple of 32"):
        h.write_rope(0, t.reshape(1), t.reshape(1), x, x)


# ---------------------------------------------------------------------------- fused RoPE append (f2 on q8_0)
@pytest.mark.parametrize("n_heads,n_kv,head_dim,rope_dim,neox,base", [
    (32, 8, 128, 128, False, 500000.0),   # Llama-3-8B
    (28, 4, 128, 128, True, 1000000.0),   # Qwen2.5-7B (NeoX pairs)
    (8, 2, 128, 64, True, 10000.0),       # partial rotary: groups on one side of rope_dim / 2
    (4, 2, 64, 48, True, 10000.0),        # groups straddling rope_dim / 2 and rope_dim
    (4, 2, 64, 48, False, 10000.0),       # interleaved pairs, a group straddling rope_dim
])
def test_q8_write_rope_bit_exact(gpu, n_heads, n_kv, head_dim, rope_dim, neox, base):
    """K rotated (model.rs:291-308) then quantised per 32 elements, V
    quantised, Q rotated in place: quants, scales and Q bit-identical to the
    oracle (rotation, then quantize_block), skipped rows included."""
    import torch

    rng = np.random.default_rng(head_dim * 7 + rope_dim)
    kv_dim = n_kv * head_dim
    g, o = _caches(1, kv_dim, 300 * BLOCK, rng.permutation(300))
    g.rope_init(base, rope_dim, head_dim, neox, 32768)
    lens = {0: 700, 1: 900, 2: 33}
    seqs = np.concatenate([np.full(n, s, dtype=np.uint32) for s, n in lens.items()])
    pos = np.concatenate([np.arange(n, dtype=np.uint64) for n in lens.values()])
    sm = g.append_batch(seqs, pos)
    np.testing.assert_array_equal(o.append_batch(seqs, pos), sm)
    sm[7] = -1
    n = sm.size
    k = q8_rows(rng, n, kv_dim)
    k[~np.isfinite(k)] = 1.0  # rotation mixes elements: keep K finite (V keeps the special blocks)
    v = q8_rows(rng, n, kv_dim)
    q = rng.standard_normal((n, n_heads * head_dim), dtype=np.float32)
    p32 = pos.astype(np.int32) * 37 % 32768
    dq = torch.from_numpy(q).to(gpu)
    g.write_rope(0, torch.from_numpy(sm).to(gpu), torch.from_numpy(p32).to(gpu), torch.from_numpy(k).to(gpu),
                 torch.from_numpy(v).to(gpu), q=dq, n_heads=n_heads)
    qo = q.copy()
    o.write_rope_batch(0, sm, p32, k, v, base, rope_dim, head_dim, neox, q=qo, n_heads=n_heads)
    np.testing.assert_array_equal(dq.cpu().numpy().view(np.uint32), qo.view(np.uint32))
    _assert_q8_equal(g, o, (0,))
