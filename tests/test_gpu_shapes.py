"""Shapes outside the tuned kernels, against the oracle.

The reference takes any shape: model.rs:401-402 reads head_dim and the group
from the model and the closure (model.rs:431-475) loops over whatever they
are; its own cache test uses kv_dim 4 (kv.rs:202-229). Rows whose byte length
is not a multiple of 16 move element by element (append, gather, rows), and
attention with a head_dim other than 64 / 128 or a group above 8 runs on the
generic kernel; the bar is the same as for the tuned kernels: bit-exact
pools and rows, attention within max abs 2e-2 (f16) / 1e-3 (f32, q8_0) and
relative L2 1e-3.
"""

from __future__ import annotations

import numpy as np
import pytest

from helpers import BLOCK, attention_close, fill_sequences, tables_and_lens

pytestmark = pytest.mark.gpu


def _caches(kv_dim, n_blocks, dtype, rng, layers=1):
    from langtrain_studio_amd import KvCache
    from oracle import OracleKv

    g = KvCache(layers, kv_dim, n_blocks * BLOCK, dtype=dtype, device=0)
    o = OracleKv(layers, kv_dim, n_blocks * BLOCK, dtype=dtype)
    order = rng.permutation(n_blocks)
    g.init_free_order(order)
    o.init_free_order(order)
    return g, o


def _bits(a):
    return a.view(np.uint16) if a.dtype.itemsize == 2 else a.view(np.uint32)


@pytest.mark.parametrize("dtype", ["f16", "f32"])
@pytest.mark.parametrize("kv_dim", [4, 12, 20, 100])
def test_write_gather_rows_any_kv_dim(gpu, dtype, kv_dim):
    import torch

    rng = np.random.default_rng(kv_dim)
    n_blocks = 80
    g, o = _caches(kv_dim, n_blocks, dtype, rng, layers=2)
    lens = {0: 1, 1: 15, 2: 16, 3: 17, 4: 333, 5: 50}
    fill_sequences([("gpu", g), ("oracle", o)], lens, rng, kv_dim, layers=(0, 1), special=True)
    for layer in (0, 1):
        gk, gv = g.read_pool(layer)
        ok, ov = o.pool(layer)
        np.testing.assert_array_equal(_bits(gk), _bits(ok))
        np.testing.assert_array_equal(_bits(gv), _bits(ov))
    seqs = list(lens)
    want_lens = [lens[s] for s in seqs]
    tables, la = tables_and_lens(g, seqs, want_lens, stride=25)
    offs = np.concatenate([[0], np.cumsum(want_lens)[:-1]]).astype(np.int64)
    total = int(sum(want_lens))
    tdt = torch.float16 if dtype == "f16" else torch.float32
    k_out = torch.full((total + 3, kv_dim), -1.0, dtype=tdt, device=gpu)
    v_out = torch.full((total + 3, kv_dim), -1.0, dtype=tdt, device=gpu)
    g.gather(1, torch.from_numpy(tables).to(gpu), torch.from_numpy(la).to(gpu), torch.from_numpy(offs).to(gpu),
             k_out, v_out)
    kh, vh = k_out.cpu().numpy(), v_out.cpu().numpy()
    for s, off, n in zip(seqs, offs, want_lens):
        rk, rv = o.rows(1, s, n)
        np.testing.assert_array_equal(_bits(kh[off:off + n]), _bits(rk))
        np.testing.assert_array_equal(_bits(vh[off:off + n]), _bits(rv))
        gk, gv = g.rows(1, s, n)
        np.testing.assert_array_equal(_bits(gk), _bits(rk))
    assert (kh[total:] == -1).all()
    g.synchronize()


@pytest.mark.parametrize("dtype", ["f16", "f32", "q8_0"])
@pytest.mark.parametrize("head_dim,group,n_kv", [(32, 4, 2), (96, 5, 1), (80, 16, 2), (256, 8, 1),
                                                 (128, 12, 1), (64, 32, 1), (160, 2, 2), (1024, 2, 1)])
def test_attention_any_shape(gpu, dtype, head_dim, group, n_kv):
    import torch

    kv_dim = head_dim * n_kv
    if dtype == "q8_0" and kv_dim % 32:
        pytest.skip("q8_0 rows are whole 32-element groups")
    rng = np.random.default_rng(head_dim * 7 + group)
    n_heads = group * n_kv
    lens = [0, 1, 15, 16, 17, 300, 1031]
    blocks = sum(-(-n // BLOCK) for n in lens) + 8
    g, o = _caches(kv_dim, blocks, dtype, rng)
    fill_sequences([("gpu", g), ("oracle", o)], dict(enumerate(lens)), rng, kv_dim)
    tables, la = tables_and_lens(g, range(len(lens)), lens)
    q = rng.standard_normal((len(lens), n_heads * head_dim), dtype=np.float32)
    out = g.decode_attention(0, torch.from_numpy(q).to(gpu), torch.from_numpy(tables).to(gpu),
                             torch.from_numpy(la).to(gpu), n_heads, head_dim).cpu().numpy()
    want = o.attention_tables(0, tables, la, q, n_heads, head_dim, threads=8)
    attention_close(out, want, dtype)
    assert (out[0] == 0).all()  # an empty context yields zeros
    # a query alone gives the same bits (one work-group per query head)
    one = g.decode_attention(0, torch.from_numpy(q[5:6]).to(gpu), torch.from_numpy(tables[5:6]).to(gpu),
                             torch.from_numpy(la[5:6]).to(gpu), n_heads, head_dim).cpu().numpy()
    np.testing.assert_array_equal(one[0].view(np.uint32), out[5].view(np.uint32))
    g.synchronize()


def test_attention_head_dim_beyond_limit_is_refused(gpu):
    """head_dim 1024 is the largest the kernels take; 1056 (a multiple of 32
    past it) is refused with LTKV_ERR_ARG before anything is launched."""
    import torch

    from langtrain_studio_amd import KvError

    rng = np.random.default_rng(3)
    g, o = _caches(1056, 4, "f16", rng)
    fill_sequences([("gpu", g), ("oracle", o)], {0: 5}, rng, 1056)
    tables, la = tables_and_lens(g, [0], [5])
    q = torch.zeros((1, 1056), dtype=torch.float32, device=gpu)
    with pytest.raises(KvError, match="at most 1024"):
        g.decode_attention(0, q, torch.from_numpy(tables).to(gpu), torch.from_numpy(la).to(gpu), 1, 1056)
    g.synchronize()


@pytest.mark.parametrize("head_dim,group", [(96, 5), (128, 12)])
def test_fused_step_and_plan_any_shape(gpu, head_dim, group):
    """The fused append + attention entry and planned attention (with the
    shared-prefix flag) take the generic kernel for such shapes: the same
    bits as write then decode attention, and forks planned per query."""
    import torch

    rng = np.random.default_rng(head_dim + group)
    n_kv = 2
    kv_dim, n_heads = head_dim * n_kv, group * n_kv
    g, o = _caches(kv_dim, 200, "f16", rng)
    lens = {0: 130, 1: 47, 2: 300}
    fill_sequences([("gpu", g), ("oracle", o)], lens, rng, kv_dim)
    for c in (g, o):
        c.share(2, 3, 300)
        c.share(2, 4, 250)
    seqs = np.array([0, 1, 2, 3, 4], dtype=np.uint32)
    pos = np.array([130, 47, 300, 300, 250], dtype=np.uint64)
    sm = g.append_batch(seqs, pos)
    np.testing.assert_array_equal(sm, o.append_batch(seqs, pos))
    k = rng.standard_normal((5, kv_dim), dtype=np.float32)
    v = rng.standard_normal((5, kv_dim), dtype=np.float32)
    q = rng.standard_normal((5, n_heads * head_dim), dtype=np.float32)
    new_lens = (pos + 1).astype(np.int32)
    tables, la = tables_and_lens(g, seqs, new_lens)
    dq, dt, dl = (torch.from_numpy(x).to(gpu) for x in (q, tables, la))
    fused = g.append_decode_attention(0, torch.from_numpy(sm).to(gpu), torch.from_numpy(k).to(gpu),
                                      torch.from_numpy(v).to(gpu), dq, dt, dl, n_heads, head_dim).cpu().numpy()
    o.write_batch(0, sm, k, v)
    want = o.attention_tables(0, tables, la, q, n_heads, head_dim, threads=8)
    attention_close(fused, want, "f16")
    plain = g.decode_attention(0, dq, dt, dl, n_heads, head_dim).cpu().numpy()
    np.testing.assert_array_equal(plain.view(np.uint32), fused.view(np.uint32))
    g.plan_attention(list(seqs), list(new_lens), n_heads, head_dim, shared_prefix=True)
    planned = g.planned_attention(0, dq).cpu().numpy()
    attention_close(planned, want, "f16")
    assert g.plan_stats()["groups"] == 0
    g.synchronize()
