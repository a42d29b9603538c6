"""Query rows beyond the f16 range of the matrix-core operands. The kernels
feed q * scale * log2 e to the products as f16 hi + lo parts, and f16 stops
at 65 504 (|q| >= ~5.1e5 at head_dim 128); the reference computes the scores
in f32 (model.rs:450,455-461), so such rows must still give its finite
result. Query heads scaled by 6e5 .. 3e7 (and one row with a single huge
element) go through every path that feeds Q to the matrix cores: decode
attention on f16 and q8_0 pools (two kv heads a wave and one), the fused
append + attention, and planned attention's grouped kernel (prefix groups
with f32-accurate and f16 products, a causal prefill chunk). Each output is
within the attention tolerance of the oracle, and on the decode kernels the
heads left in range keep their bits."""

from __future__ import annotations

import numpy as np
import pytest

from helpers import BLOCK, attention_close, fill_sequences, tables_and_lens
from test_gpu_planned import _forked, _prefill_state

pytestmark = pytest.mark.gpu

FACTORS = (6e5, 2e6, 3e7)


def _big(q, n_heads, head_dim):
    """q with every third (query, head) row scaled out of the f16 range and
    one element of row (0, 1) set to 1e7; returns it and the scaled-head mask."""
    q = q.copy()
    n = q.shape[0]
    mask = np.zeros((n, n_heads), dtype=bool)
    for i in range(n):
        for h in range(n_heads):
            if (i + h) % 3 == 0:
                q[i, h * head_dim:(h + 1) * head_dim] *= FACTORS[(i + h) % len(FACTORS)]
                mask[i, h] = True
    q[0, head_dim + 5] = 1e7
    mask[0, 1] = True
    return q, mask


def _decode(gpu, g, q, tables, la, n_heads, head_dim):
    import torch

    return g.decode_attention(0, torch.from_numpy(q).to(gpu), torch.from_numpy(tables).to(gpu),
                              torch.from_numpy(la).to(gpu), n_heads, head_dim).cpu().numpy()


@pytest.mark.parametrize("dtype", ["f16", "q8_0"])
@pytest.mark.parametrize("head_dim,group,n_kv", [(128, 4, 8), (128, 7, 4), (64, 8, 2), (128, 2, 4)])
def test_decode_attention_q_beyond_f16(gpu, dtype, head_dim, group, n_kv):
    from langtrain_studio_amd import KvCache
    from oracle import OracleKv

    rng = np.random.default_rng(900 + head_dim + group)
    kv_dim, n_heads = n_kv * head_dim, n_kv * group
    lens = [1, 17, 300, 1031, 2500, 4100, 64, 5000]
    n_tokens = (sum(-(-n // BLOCK) for n in lens) + 8) * BLOCK
    g = KvCache(1, kv_dim, n_tokens, dtype=dtype, device=0)
    o = OracleKv(1, kv_dim, n_tokens, dtype=dtype)
    order = rng.permutation(g.n_blocks)
    g.init_free_order(order)
    o.init_free_order(order)
    fill_sequences([("gpu", g), ("oracle", o)], dict(enumerate(lens)), rng, kv_dim)
    tables, la = tables_and_lens(g, range(len(lens)), lens)
    q = rng.standard_normal((len(lens), n_heads * head_dim), dtype=np.float32)
    qb, mask = _big(q, n_heads, head_dim)
    print(f"q range decode {dtype} hd {head_dim} group {group}", flush=True)
    out = _decode(gpu, g, qb, tables, la, n_heads, head_dim)
    want = o.attention_tables(0, tables, la, qb, n_heads, head_dim, threads=8)
    attention_close(out, want, dtype)
    # heads inside the range: the same bits as with every head inside it
    ref = _decode(gpu, g, q, tables, la, n_heads, head_dim)
    keep = np.repeat(~mask, head_dim, axis=1)
    np.testing.assert_array_equal(out.view(np.uint32)[keep], ref.view(np.uint32)[keep])


def test_fused_step_q_beyond_f16(gpu):
    import torch

    from langtrain_studio_amd import KvCache
    from oracle import OracleKv

    rng = np.random.default_rng(950)
    head_dim, n_kv, n_heads = 128, 8, 32
    kv_dim = n_kv * head_dim
    ctx = [0, 15, 300, 2047, 4100]
    n_tokens = (sum(-(-(c + 1) // BLOCK) for c in ctx) + 8) * BLOCK
    g = KvCache(1, kv_dim, n_tokens, dtype="f16", device=0)
    o = OracleKv(1, kv_dim, n_tokens, dtype="f16")
    order = rng.permutation(g.n_blocks)
    g.init_free_order(order)
    o.init_free_order(order)
    fill_sequences([("gpu", g), ("oracle", o)], dict(enumerate(ctx)), rng, kv_dim)
    seqs = np.arange(len(ctx), dtype=np.uint32)
    pos = np.array(ctx, dtype=np.uint64)
    sm = g.append_batch(seqs, pos)
    np.testing.assert_array_equal(o.append_batch(seqs, pos), sm)
    lens = np.array([c + 1 for c in ctx], dtype=np.int32)
    tables = g.block_tables(seqs)
    k = rng.standard_normal((len(ctx), kv_dim), dtype=np.float32)
    v = rng.standard_normal((len(ctx), kv_dim), dtype=np.float32)
    qb, _ = _big(rng.standard_normal((len(ctx), n_heads * head_dim), dtype=np.float32), n_heads, head_dim)
    d = {x: torch.from_numpy(y).to(gpu) for x, y in (("sm", sm), ("k", k), ("v", v), ("q", qb),
                                                       ("t", tables), ("l", lens))}
    out = g.append_decode_attention(0, d["sm"], d["k"], d["v"], d["q"], d["t"], d["l"], n_heads,
                                    head_dim).cpu().numpy()
    o.write_batch(0, sm, k, v)
    want = o.attention_tables(0, tables, lens, qb, n_heads, head_dim, threads=8)
    attention_close(out, want, "f16")


def _planned(gpu, g, o, seqs, lens, n_heads, head_dim, rng, dtype, f16p):
    import torch

    qb, _ = _big(rng.standard_normal((len(seqs), n_heads * head_dim), dtype=np.float32), n_heads, head_dim)
    stats = g.plan_attention(seqs, lens, n_heads, head_dim, shared_prefix=True, f16_products=f16p)
    assert stats["groups"] >= 1
    out = g.planned_attention(0, torch.from_numpy(qb).to(gpu)).cpu().numpy()
    tables, la = tables_and_lens(g, seqs, lens)
    want = o.attention_tables(0, tables, la, qb, n_heads, head_dim, threads=8)
    attention_close(out, want, dtype)


@pytest.mark.parametrize("dtype", ["f16", "q8_0"])
@pytest.mark.parametrize("f16p", [False, True])
def test_prefix_group_q_beyond_f16(gpu, dtype, f16p):
    rng = np.random.default_rng(960 + f16p)
    kids = [(1 + i, int(rng.integers(0, 40))) for i in range(40)]
    g, o = _forked(rng, 1024, dtype, [(0, 1500, kids)], singles=[(90, 333)])
    seqs = [s for s, _ in kids] + [90]
    print(f"q range prefix group {dtype} f16p={f16p}", flush=True)
    _planned(gpu, g, o, seqs, [g.len(s) for s in seqs], 32, 128, rng, dtype, f16p)


def test_prefill_chunk_q_beyond_f16(gpu):
    rng = np.random.default_rng(970)
    g, o, seqs, lens = _prefill_state(rng, 4 * 128, [(0, 700, 300)], decode=[(5, 900)])
    _planned(gpu, g, o, seqs, lens, 28, 128, rng, "f16", False)
