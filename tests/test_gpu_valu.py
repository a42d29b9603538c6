"""The vector-ALU decode attention engine on f16 pools (ltkv_set_attention_engine
with LTKV_ENGINE_VALU: wave-wide dot products and shuffle reductions, no
matrix cores) against the oracle's attention closure (model.rs:431-475 over
kv.rs tables), within the attention tolerance, through every entry point that
takes it: per-query decode attention, attention by resident rows, the fused
append (two launches on this engine) and the per-query pass of planned
attention (group partials folded by the merge). A query's result stays
independent of the rest of the batch."""

import numpy as np
import pytest

from helpers import BLOCK, append_rows, attention_close, fill_sequences, tables_and_lens

pytestmark = pytest.mark.gpu


def _caches(kv_dim, n_tokens, rng, dtype="f16"):
    from langtrain_studio_amd import KvCache
    from oracle import OracleKv

    g = KvCache(1, kv_dim, n_tokens, dtype=dtype, device=0)
    o = OracleKv(1, kv_dim, n_tokens, dtype=dtype)
    order = rng.permutation(g.n_blocks)
    g.init_free_order(order)
    o.init_free_order(order)
    g.set_attention_engine("valu")
    return g, o


@pytest.mark.parametrize("head_dim", [64, 128])
@pytest.mark.parametrize("group", [1, 4, 7, 8])
def test_valu_engine_shapes(gpu, head_dim, group):
    import torch

    rng = np.random.default_rng(300 + head_dim + group)
    n_kv = 2
    kv_dim, n_heads = n_kv * head_dim, n_kv * group
    lens = [1, 2, 15, 16, 17, 63, 300, 1031, 4100]
    g, o = _caches(kv_dim, (sum(-(-n // BLOCK) for n in lens) + 8) * BLOCK, rng)
    fill_sequences([("gpu", g), ("oracle", o)], dict(enumerate(lens)), rng, kv_dim)
    tables, la = tables_and_lens(g, range(len(lens)), lens)
    q = rng.standard_normal((len(lens), n_heads * head_dim), dtype=np.float32)
    out = g.decode_attention(0, torch.from_numpy(q).to(gpu), torch.from_numpy(tables).to(gpu),
                             torch.from_numpy(la).to(gpu), n_heads, head_dim).cpu().numpy()
    want = o.attention_tables(0, tables, la, q, n_heads, head_dim, threads=8)
    attention_close(out, want, "f16")


def test_valu_engine_differs_from_the_matrix_cores_within_tolerance(gpu):
    """Both engines on the same Llama-3-8B-shaped step: each within the bar of
    the oracle, and not the same bits (the setting takes effect)."""
    import torch

    rng = np.random.default_rng(311)
    lens = [int(x) for x in rng.integers(2048, 4097, size=8)]
    g, o = _caches(1024, (sum(-(-n // BLOCK) for n in lens) + 8) * BLOCK, rng)
    fill_sequences([("gpu", g), ("oracle", o)], dict(enumerate(lens)), rng, 1024)
    tables, la = tables_and_lens(g, range(len(lens)), lens)
    q = rng.standard_normal((len(lens), 32 * 128), dtype=np.float32)
    dq, dt, dl = (torch.from_numpy(x).to(gpu) for x in (q, tables, la))
    valu = g.decode_attention(0, dq, dt, dl, 32, 128).cpu().numpy()
    g.set_attention_engine("auto")
    mfma = g.decode_attention(0, dq, dt, dl, 32, 128).cpu().numpy()
    want = o.attention_tables(0, tables, la, q, 32, 128, threads=8)
    attention_close(valu, want, "f16")
    attention_close(mfma, want, "f16")
    assert not np.array_equal(valu.view(np.uint32), mfma.view(np.uint32))


def test_valu_engine_batch_independence(gpu):
    import torch

    rng = np.random.default_rng(312)
    lens = [2000, 9, 513, 4096, 77] + [int(x) for x in rng.integers(1, 600, size=60)]
    g, _ = _caches(1024, (sum(-(-n // BLOCK) for n in lens) + 8) * BLOCK, rng)
    fill_sequences([("gpu", g)], dict(enumerate(lens)), rng, 1024)
    tables, la = tables_and_lens(g, range(len(lens)), lens)
    q = rng.standard_normal((len(lens), 32 * 128), dtype=np.float32)
    dq, dt, dl = (torch.from_numpy(x).to(gpu) for x in (q, tables, la))
    full = g.decode_attention(0, dq, dt, dl, 32, 128).cpu().numpy()
    for i in range(5):
        one = g.decode_attention(0, dq[i:i + 1].contiguous(), dt[i:i + 1, :-(-lens[i] // BLOCK)].contiguous(),
                                 dl[i:i + 1].contiguous(), 32, 128).cpu().numpy()
        np.testing.assert_array_equal(one[0].view(np.uint32), full[i].view(np.uint32))


def test_valu_engine_fused_step_and_resident_rows(gpu):
    """The fused decode step runs as write + attention on this engine: pools
    and outputs equal the two calls; attention by resident rows equals
    attention by tables, and both match the oracle."""
    import torch

    rng = np.random.default_rng(313)
    lens = [40, 700, 1500, 3000, 17, 64]
    kv_dim, n_heads, hd = 512, 16, 128
    g, o = _caches(kv_dim, (sum(-(-n // BLOCK) for n in lens) + 16) * BLOCK, rng)
    fill_sequences([("gpu", g), ("oracle", o)], dict(enumerate(lens)), rng, kv_dim)
    seqs = np.arange(len(lens), dtype=np.uint32)
    pos = np.array(lens, dtype=np.uint64)
    sm_g = g.append_batch(seqs, pos)
    sm_o = o.append_batch(seqs, pos)
    np.testing.assert_array_equal(sm_g, sm_o)
    kn = rng.standard_normal((len(lens), kv_dim), dtype=np.float32)
    vn = rng.standard_normal((len(lens), kv_dim), dtype=np.float32)
    o.write_batch(0, sm_o, kn, vn)
    new_lens = [n + 1 for n in lens]
    tables, la = tables_and_lens(g, seqs, new_lens)
    q = rng.standard_normal((len(lens), n_heads * hd), dtype=np.float32)
    d = {k: torch.from_numpy(v).to(gpu) for k, v in dict(q=q, t=tables, l=la, sm=sm_g, k=kn, v=vn).items()}
    out = g.append_decode_attention(0, d["sm"], d["k"], d["v"], d["q"], d["t"], d["l"], n_heads, hd).cpu().numpy()
    gk, gv = g.read_pool(0)
    ok, ov = o.pool(0)
    np.testing.assert_array_equal(gk.view(np.uint16), ok.view(np.uint16))
    np.testing.assert_array_equal(gv.view(np.uint16), ov.view(np.uint16))
    again = g.decode_attention(0, d["q"], d["t"], d["l"], n_heads, hd).cpu().numpy()
    np.testing.assert_array_equal(out.view(np.uint32), again.view(np.uint32))
    rows = torch.from_numpy(g.seq_rows(seqs)).to(gpu)
    by_row = g.decode_attention_rows(0, d["q"], rows, d["l"], n_heads, hd).cpu().numpy()
    np.testing.assert_array_equal(by_row.view(np.uint32), out.view(np.uint32))
    want = o.attention_tables(0, tables, la, q, n_heads, hd, threads=8)
    attention_close(out, want, "f16")


def test_valu_engine_planned_prefix_groups(gpu):
    """Planned attention with a prefix group: the shared blocks on the matrix
    cores, each query's remainder on the vector-ALU kernel, the group
    partials folded by the merge; within the bar of the oracle."""
    import torch

    rng = np.random.default_rng(314)
    kv_dim, n_heads, hd = 1024, 32, 128
    prefix, kids = 1000, [(1 + i, int(rng.integers(1, 70))) for i in range(40)]
    need = prefix + sum(e for _, e in kids) + 16 * (len(kids) + 1) + 64 * BLOCK
    g, o = _caches(kv_dim, need, rng)
    both = [("gpu", g), ("oracle", o)]
    append_rows(both, [0] * prefix, np.arange(prefix), rng, kv_dim)
    for child, extra in kids:
        g.share(0, child, prefix)
        o.share(0, child, prefix)
        append_rows(both, [child] * extra, np.arange(prefix, prefix + extra), rng, kv_dim)
    seqs = [s for s, _ in kids]
    lens = [g.len(s) for s in seqs]
    q = rng.standard_normal((len(seqs), n_heads * hd), dtype=np.float32)
    stats = g.plan_attention(seqs, lens, n_heads, hd, shared_prefix=True)
    assert stats["groups"] == 1
    out = g.planned_attention(0, torch.from_numpy(q).to(gpu)).cpu().numpy()
    tables, la = tables_and_lens(g, seqs, lens)
    want = o.attention_tables(0, tables, la, q, n_heads, hd, threads=8)
    attention_close(out, want, "f16")
