"""Planned attention on the GPU (ltkv_plan_attention + ltkv_planned_attention)
against the oracle's attention closure (model.rs:431-475 over kv.rs tables):
without prefix groups it is the decode kernel on host-built tables (bit-exact
with ltkv_decode_attention); with them, the shared blocks of forked sequences
go through the matrix-core kernel once per group and are merged with each
query's own blocks (attention tolerance)."""

import numpy as np
import pytest

from helpers import BLOCK, append_rows, attention_close, fill_sequences, tables_and_lens

pytestmark = pytest.mark.gpu


def _caches(n_layers, kv_dim, n_tokens, dtype, rng):
    from langtrain_studio_amd import KvCache
    from oracle import OracleKv

    g = KvCache(n_layers, kv_dim, n_tokens, dtype=dtype, device=0)
    o = OracleKv(n_layers, kv_dim, n_tokens, dtype=dtype)
    order = rng.permutation(g.n_blocks)
    g.init_free_order(order)
    o.init_free_order(order)
    return g, o


def _forked(rng, kv_dim, dtype, spec, singles=(), n_layers=1):
    """spec: (root, prefix_len, [(child, extra_tokens), ...]) -- the root holds
    prefix_len tokens, each child shares them (kv.rs:172-183) and appends its
    own tokens (copy-on-write of the shared partial block, kv.rs:95-110).
    singles: (seq, len) sequences that share nothing."""
    need = sum(p + sum(e for _, e in kids) + 16 * (len(kids) + 1) for _, p, kids in spec)
    need += sum(n + 16 for _, n in singles) + 64 * BLOCK
    g, o = _caches(n_layers, kv_dim, need, dtype, rng)
    both = [("gpu", g), ("oracle", o)]
    layers = tuple(range(n_layers))
    for root, prefix, kids in spec:
        append_rows(both, [root] * prefix, np.arange(prefix), rng, kv_dim, layers)
        for child, extra in kids:
            g.share(root, child, prefix)
            o.share(root, child, prefix)
            if extra:
                append_rows(both, [child] * extra, np.arange(prefix, prefix + extra), rng, kv_dim, layers)
    if singles:
        fill_sequences(both, dict(singles), rng, kv_dim, layers)
    assert g.cow_copies() == o.cow_copies()
    return g, o


def _run(gpu, g, o, seqs, lens, n_heads, head_dim, rng, shared=True, layer=0, dtype="f16", f16p=False):
    import torch

    q = rng.standard_normal((len(seqs), n_heads * head_dim), dtype=np.float32)
    stats = g.plan_attention(seqs, lens, n_heads, head_dim, shared_prefix=shared, f16_products=f16p)
    out = g.planned_attention(layer, torch.from_numpy(q).to(gpu)).cpu().numpy()
    tables, la = tables_and_lens(g, seqs, lens)
    want = o.attention_tables(layer, tables, la, q, n_heads, head_dim, threads=8)
    attention_close(out, want, dtype)
    return stats, q, out, tables, la


def test_planned_without_groups_is_the_decode_kernel(gpu):
    """Host-built tables, one upload: bit-identical to ltkv_decode_attention."""
    import torch

    rng = np.random.default_rng(40)
    lens = [1, 17, 300, 1031, 2500, 64]
    g, o = _caches(1, 1024, (sum(lens) // BLOCK + 32) * BLOCK, "f16", rng)
    fill_sequences([("gpu", g), ("oracle", o)], dict(enumerate(lens)), rng, 1024)
    seqs = list(range(len(lens)))
    _, q, out, tables, la = _run(gpu, g, o, seqs, lens, 32, 128, rng, shared=False)
    ref = g.decode_attention(0, torch.from_numpy(q).to(gpu), torch.from_numpy(tables).to(gpu),
                             torch.from_numpy(la).to(gpu), 32, 128).cpu().numpy()
    np.testing.assert_array_equal(out, ref)


@pytest.mark.parametrize("n_kids,prefix", [(70, 2040), (3, 100), (256, 504)])
def test_prefix_sharing_forks(gpu, n_kids, prefix):
    """Sequences forked from one prefix with private suffixes (Llama-3-8B
    heads, f16): one group over the common full blocks; output within the
    attention tolerance of the oracle and of the per-query decode kernel."""
    import torch

    rng = np.random.default_rng(n_kids + prefix)
    kids = [(1 + i, int(rng.integers(1, 71))) for i in range(n_kids)]
    g, o = _forked(rng, 1024, "f16", [(0, prefix, kids)])
    seqs = [s for s, _ in kids]
    lens = [g.len(s) for s in seqs]
    stats, q, out, tables, la = _run(gpu, g, o, seqs, lens, 32, 128, rng)
    assert stats["groups"] == 1 and stats["grouped"] == n_kids
    assert stats["shared_blocks"] == prefix // BLOCK
    ref = g.decode_attention(0, torch.from_numpy(q).to(gpu), torch.from_numpy(tables).to(gpu),
                             torch.from_numpy(la).to(gpu), 32, 128).cpu().numpy()
    attention_close(out, ref, "f16")


@pytest.mark.parametrize("head_dim,group", [(128, 1), (128, 4), (128, 7), (128, 8), (64, 4), (64, 8)])
def test_prefix_groups_shapes(gpu, head_dim, group):
    """Two groups, their roots, sequences sharing nothing, a fork with an
    empty suffix (its whole context is shared) and an empty read, for each
    supported head shape."""
    rng = np.random.default_rng(head_dim * 10 + group)
    n_kv = 2
    kv_dim = n_kv * head_dim
    spec = [(0, 333, [(1, 5), (2, 0), (3, 40), (4, 16)]),
            (10, 1200, [(11 + i, int(rng.integers(0, 50))) for i in range(20)])]
    g, o = _forked(rng, kv_dim, "f16", spec, singles=[(50, 700), (51, 3)])
    seqs = [0, 1, 2, 3, 4, 10] + [11 + i for i in range(20)] + [50, 51, 2]
    lens = [g.len(s) for s in seqs]
    lens[-1] = 0  # an empty read of a grouped sequence
    stats, *_ = _run(gpu, g, o, seqs, lens, group * n_kv, head_dim, rng)
    assert stats["groups"] == 2


def test_plan_serves_every_layer_and_replans(gpu):
    """One plan for several layers; a second plan of another batch reuses
    the buffers."""
    import torch

    rng = np.random.default_rng(41)
    kids = [(1 + i, int(rng.integers(1, 40))) for i in range(12)]
    g, o = _forked(rng, 1024, "f16", [(0, 900, kids)], singles=[(40, 2000)], n_layers=3)
    seqs = [s for s, _ in kids] + [40]
    lens = [g.len(s) for s in seqs]
    q = rng.standard_normal((len(seqs), 32 * 128), dtype=np.float32)
    g.plan_attention(seqs, lens, 32, 128)
    tables, la = tables_and_lens(g, seqs, lens)
    for layer in (2, 0, 1):
        out = g.planned_attention(layer, torch.from_numpy(q).to(gpu)).cpu().numpy()
        want = o.attention_tables(layer, tables, la, q, 32, 128, threads=8)
        attention_close(out, want, "f16")
    _run(gpu, g, o, seqs[:3], lens[:3], 32, 128, rng, layer=1)
    _run(gpu, g, o, seqs[::-1], lens[::-1], 32, 128, rng, layer=2)


def test_stale_plan_is_rejected(gpu):
    import torch

    from langtrain_studio_amd import KvError

    rng = np.random.default_rng(42)
    g, o = _forked(rng, 1024, "f16", [(0, 100, [(1, 3), (2, 3)])])
    g.plan_attention([1, 2], [g.len(1), g.len(2)], 32, 128)
    g.append(1, g.len(1))
    q = torch.zeros((2, 32 * 128), dtype=torch.float32, device=gpu)
    with pytest.raises(KvError, match="stale"):
        g.planned_attention(0, q)


def test_f32_pools_plan_without_groups(gpu):
    """f32 pools ignore the shared-prefix flag: bit-identical to the decode kernel."""
    import torch

    rng = np.random.default_rng(43)
    g, o = _forked(rng, 256, "f32", [(0, 300, [(1, 4), (2, 9)])])
    seqs = [0, 1, 2]
    lens = [g.len(s) for s in seqs]
    stats, q, out, tables, la = _run(gpu, g, o, seqs, lens, 32, 64, rng, dtype="f32")
    assert stats["groups"] == 0
    ref = g.decode_attention(0, torch.from_numpy(q).to(gpu), torch.from_numpy(tables).to(gpu),
                             torch.from_numpy(la).to(gpu), 32, 64).cpu().numpy()
    np.testing.assert_array_equal(out, ref)


@pytest.mark.parametrize("dtype", ["f16", "q8_0"])
@pytest.mark.parametrize("head_dim,group", [(128, 4), (128, 7), (64, 8)])
def test_prefix_groups_f16_products(gpu, dtype, head_dim, group):
    """LTKV_PLAN_F16_PRODUCTS: the grouped products on f16-rounded Q and
    weights stay within the attention tolerance of the oracle (f16 pools:
    max abs 2e-2, relative L2 1e-3; q8_0: the f32 bar on max abs), and
    really differ from the f32-accurate products (the flag takes effect)."""
    import torch

    rng = np.random.default_rng(head_dim + group + (7 if dtype == "q8_0" else 0))
    n_kv = 2
    kv_dim = n_kv * head_dim
    spec = [(0, 1200, [(1 + i, int(rng.integers(0, 60))) for i in range(40)])]
    g, o = _forked(rng, kv_dim, dtype, spec, singles=[(60, 300)])
    seqs = [1 + i for i in range(40)] + [60]
    lens = [g.len(s) for s in seqs]
    n_heads = group * n_kv
    stats, q, fast, tables, la = _run(gpu, g, o, seqs, lens, n_heads, head_dim, rng, dtype=dtype, f16p=True)
    assert stats["groups"] == 1
    g.plan_attention(seqs, lens, n_heads, head_dim, shared_prefix=True)
    exact = g.planned_attention(0, torch.from_numpy(q).to(gpu)).cpu().numpy()
    rel = np.linalg.norm(fast - exact) / np.linalg.norm(exact)
    assert 1e-6 < rel < 1e-3, rel


@pytest.mark.parametrize("n_heads,n_kv,head_dim,ctx,chunk", [(28, 4, 128, 1000, 512), (32, 4, 64, 700, 100)])
def test_prefill_chunk_f16_products(gpu, n_heads, n_kv, head_dim, ctx, chunk):
    """Causal groups of a prefill chunk with LTKV_PLAN_F16_PRODUCTS, within
    the attention tolerance of the oracle."""
    rng = np.random.default_rng(ctx + chunk + head_dim + 1)
    g, o, seqs, lens = _prefill_state(rng, n_kv * head_dim, [(0, ctx, chunk)])
    stats, *_ = _run(gpu, g, o, seqs, lens, n_heads, head_dim, rng, f16p=True)
    assert stats["groups"] == 1 and stats["grouped"] == chunk


# ---------------------------------------------------------------------------- chunked prefill
def _prefill_state(rng, kv_dim, chunks, decode=(), dtype="f16"):
    """chunks: (seq, context, chunk_len) -- the sequence holds `context`
    tokens, then appends a chunk of chunk_len tokens (the step's prefill
    chunk, model.rs:380-429); decode: (seq, len) sequences appending one token."""
    need = sum(c + n + 32 for _, c, n in chunks) + sum(n + 32 for _, n in decode) + 64 * BLOCK
    g, o = _caches(1, kv_dim, need, dtype, rng)
    both = [("gpu", g), ("oracle", o)]
    for s, ctx, _ in chunks:
        if ctx:
            append_rows(both, [s] * ctx, np.arange(ctx), rng, kv_dim)
    if decode:
        fill_sequences(both, dict(decode), rng, kv_dim)
    seqs, pos = [], []
    for s, ctx, n in chunks:
        seqs += [s] * n
        pos += list(range(ctx, ctx + n))
    for s, n in decode:
        seqs.append(s)
        pos.append(n)
    append_rows(both, seqs, pos, rng, kv_dim)
    return g, o, seqs, [p + 1 for p in pos]


@pytest.mark.parametrize("n_heads,n_kv,head_dim,ctx,chunk", [
    (28, 4, 128, 1000, 512),   # Qwen2.5-7B heads, a 512-token chunk after 1000 tokens
    (32, 8, 128, 0, 300),      # the first chunk of a prompt
    (32, 8, 128, 2047, 33),
    (32, 4, 64, 700, 100),
    (16, 2, 64, 64, 200),
])
def test_prefill_chunk_causal(gpu, n_heads, n_kv, head_dim, ctx, chunk):
    """Every token of a prefill chunk attends to its own prefix (causal
    within the chunk) through one causal group on the matrix cores."""
    rng = np.random.default_rng(ctx + chunk + head_dim)
    g, o, seqs, lens = _prefill_state(rng, n_kv * head_dim, [(0, ctx, chunk)])
    stats, *_ = _run(gpu, g, o, seqs, lens, n_heads, head_dim, rng)
    assert stats["groups"] == 1 and stats["grouped"] == chunk


def test_prefill_chunks_with_one_long_context(gpu):
    """Several prefill chunks, one after a context much longer than the
    others: the planner cuts only that chunk's range (it exceeds the mean
    load of a work-group slot), and with no decode queries the per-query
    pass is the merge alone, which folds every group partial."""
    rng = np.random.default_rng(46)
    g, o, seqs, lens = _prefill_state(rng, 4 * 128, [(0, 3000, 128), (1, 200, 128), (2, 90, 96), (3, 0, 64)])
    stats, *_ = _run(gpu, g, o, seqs, lens, 28, 128, rng)
    assert stats["groups"] == 4 and stats["grouped"] == 128 + 128 + 96 + 64


def test_mixed_step_prefill_decode_and_forks(gpu):
    """A continuous-batching step: two prefill chunks, decode queries that
    share nothing, and decode queries of forked sequences, in one plan."""
    rng = np.random.default_rng(44)
    kv_dim = 4 * 128
    g, o, seqs, lens = _prefill_state(rng, kv_dim, [(0, 600, 128), (1, 0, 64)],
                                      decode=[(5, 900), (6, 33), (7, 1500)])
    both = [("gpu", g), ("oracle", o)]
    append_rows(both, [20] * 400, np.arange(400), rng, kv_dim)
    for child in (21, 22, 23):
        g.share(20, child, 400)
        o.share(20, child, 400)
        append_rows(both, [child], [400], rng, kv_dim)
    seqs = seqs + [21, 22, 23]
    lens = lens + [401, 401, 401]
    stats, *_ = _run(gpu, g, o, seqs, lens, 28, 128, rng)
    assert stats["groups"] == 3 and stats["grouped"] == 128 + 64 + 3


def test_decode_queries_in_a_mixed_plan_match_the_decode_kernel(gpu):
    """Prefill chunks (completed by their causal groups) next to decode
    queries with long contexts: the per-query pass covers only the decode
    queries, with the per-query partition policy, so their outputs equal the
    decode kernel's bit for bit; the chunk tokens match the oracle."""
    import torch

    rng = np.random.default_rng(45)
    kv_dim, n_heads, hd = 4 * 128, 28, 128
    g, o, seqs, lens = _prefill_state(rng, kv_dim, [(0, 900, 96), (1, 40, 64)],
                                      decode=[(5, 1300), (6, 2100), (7, 700)])
    stats, q, out, tables, la = _run(gpu, g, o, seqs, lens, n_heads, hd, rng)
    assert stats["groups"] == 2 and stats["grouped"] == 160
    dec = slice(160, 163)
    ref = g.decode_attention(0, torch.from_numpy(q[dec].copy()).to(gpu), torch.from_numpy(tables[dec].copy()).to(gpu),
                             torch.from_numpy(la[dec].copy()).to(gpu), n_heads, hd).cpu().numpy()
    np.testing.assert_array_equal(out[dec], ref)


def test_continuous_batching_churn_matches_oracle(gpu):
    """Config-4 semantics at small scale, 6 steps: each step appends a prefill
    chunk of one stream and a token per decode sequence (fused RoPE append),
    decode sequences finish (blocks freed LIFO, kv.rs:76-81) and arrivals
    reuse them; tables and pools stay bit-identical to the oracle and every
    step's attention (per-query and planned) is within tolerance."""
    import torch

    rng = np.random.default_rng(46)
    n_heads, n_kv, hd = 28, 4, 128
    kv_dim = n_kv * hd
    g, o = _caches(1, kv_dim, 300 * BLOCK, "f16", rng)
    both = [("gpu", g), ("oracle", o)]
    g.rope_init(1e6, hd, hd, True, 4096)
    dec = list(range(6))
    fill_sequences(both, {s: int(rng.integers(20, 200)) for s in dec}, rng, kv_dim)
    stream, next_id = 100, 200
    for step in range(6):
        seqs = [stream] * 48 + dec
        pos = list(range(g.len(stream), g.len(stream) + 48)) + [g.len(s) for s in dec]
        sm = g.append_batch(seqs, pos)
        np.testing.assert_array_equal(sm, o.append_batch(seqs, pos))
        k = rng.standard_normal((len(seqs), kv_dim), dtype=np.float32)
        v = rng.standard_normal((len(seqs), kv_dim), dtype=np.float32)
        q = rng.standard_normal((len(seqs), n_heads * hd), dtype=np.float32)
        dq = torch.from_numpy(q.copy()).to(gpu)
        g.write_rope(0, torch.from_numpy(sm).to(gpu), torch.from_numpy(np.array(pos, np.int32)).to(gpu),
                     torch.from_numpy(k).to(gpu), torch.from_numpy(v).to(gpu), q=dq, n_heads=n_heads)
        o.write_rope_batch(0, sm, np.array(pos, np.int32), k, v, 1e6, hd, hd, True, q=q, n_heads=n_heads)
        np.testing.assert_array_equal(dq.cpu().numpy().view(np.uint32), q.view(np.uint32))
        lens = [p + 1 for p in pos]
        tables, la = tables_and_lens(g, seqs, lens)
        want = o.attention_tables(0, tables, la, q, n_heads, hd, threads=8)
        flat = g.decode_attention(0, dq, torch.from_numpy(tables).to(gpu), torch.from_numpy(la).to(gpu),
                                  n_heads, hd).cpu().numpy()
        attention_close(flat, want, "f16")
        g.plan_attention(seqs, lens, n_heads, hd)
        attention_close(g.planned_attention(0, dq).cpu().numpy(), want, "f16")
        for i, s in enumerate(dec):  # a third finish; arrivals take their place
            if rng.random() < 0.34:
                g.truncate(s, 0)
                o.truncate(s, 0)
                dec[i] = next_id
                fill_sequences(both, {next_id: int(rng.integers(1, 120))}, rng, kv_dim)
                next_id += 1
        if g.len(stream) > 200:  # the prompt is done: a new stream starts
            g.truncate(stream, 0)
            o.truncate(stream, 0)
            stream += 1
        assert g.free_blocks() == o.free_blocks()
        for s in dec + [stream]:
            np.testing.assert_array_equal(g.block_table(s), o.block_table(s))
        gk, gv = g.read_pool(0)
        ok, ov = o.pool(0)
        np.testing.assert_array_equal(gk, ok)
        np.testing.assert_array_equal(gv, ov)


# ---------------------------------------------------------------------------- q8_0 groups
@pytest.mark.parametrize("n_kids,prefix", [(70, 2040), (3, 100)])
def test_q8_prefix_sharing_forks(gpu, n_kids, prefix):
    """Forks of one prefix on a q8_0 cache: the group kernel stages the int8
    tiles as f16 with their scales; within the f32 bar of the oracle over the
    dequantised rows."""
    rng = np.random.default_rng(n_kids + prefix + 1)
    kids = [(1 + i, int(rng.integers(1, 71))) for i in range(n_kids)]
    g, o = _forked(rng, 1024, "q8_0", [(0, prefix, kids)])
    seqs = [s for s, _ in kids]
    lens = [g.len(s) for s in seqs]
    stats, *_ = _run(gpu, g, o, seqs, lens, 32, 128, rng, dtype="q8_0")
    assert stats["groups"] == 1 and stats["grouped"] == n_kids


@pytest.mark.parametrize("head_dim,group", [(128, 1), (128, 4), (128, 8), (64, 4), (64, 8)])
def test_q8_prefix_groups_shapes(gpu, head_dim, group):
    """Two groups, roots, unshared sequences, a fork with an empty suffix and
    an empty read, on q8_0 pools."""
    rng = np.random.default_rng(head_dim * 10 + group + 1)
    n_kv = 2
    kv_dim = n_kv * head_dim
    spec = [(0, 333, [(1, 5), (2, 0), (3, 40), (4, 16)]),
            (10, 1200, [(11 + i, int(rng.integers(0, 50))) for i in range(20)])]
    g, o = _forked(rng, kv_dim, "q8_0", spec, singles=[(50, 700), (51, 3)])
    seqs = [0, 1, 2, 3, 4, 10] + [11 + i for i in range(20)] + [50, 51, 2]
    lens = [g.len(s) for s in seqs]
    lens[-1] = 0
    stats, *_ = _run(gpu, g, o, seqs, lens, group * n_kv, head_dim, rng, dtype="q8_0")
    assert stats["groups"] == 2


@pytest.mark.parametrize("n_heads,n_kv,head_dim,ctx,chunk", [
    (28, 4, 128, 1000, 512),
    (32, 8, 128, 0, 300),
    (32, 4, 64, 700, 100),
])
def test_q8_prefill_chunk_causal(gpu, n_heads, n_kv, head_dim, ctx, chunk):
    rng = np.random.default_rng(ctx + chunk + head_dim + 1)
    g, o, seqs, lens = _prefill_state(rng, n_kv * head_dim, [(0, ctx, chunk)], dtype="q8_0")
    stats, *_ = _run(gpu, g, o, seqs, lens, n_heads, head_dim, rng, dtype="q8_0")
    assert stats["groups"] == 1 and stats["grouped"] == chunk
