"""A decode step (append + decode attention, and attention by resident rows)
captured in a HIP graph: every replay, with eager work and synchronisation
between replays, gives the eager step's bits. The library records no memset
or host synchronisation inside these calls, so the step can be replayed by
an engine that captures its decode loop."""

from __future__ import annotations

import numpy as np
import pytest

from helpers import BLOCK, fill_sequences, tables_and_lens

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("dtype", ["f16", "q8_0"])
def test_decode_step_graph_replays_match_eager(gpu, dtype):
    import torch

    from langtrain_studio_amd import KvCache

    rng = np.random.default_rng(3)
    n_heads, n_kv, hd = 32, 8, 128
    kvd = n_kv * hd
    lens0 = [int(x) for x in rng.integers(100, 1500, size=12)]
    blocks = sum(-(-(n + 1) // BLOCK) for n in lens0) + 8
    kv = KvCache(1, kvd, blocks * BLOCK, dtype=dtype, device=0, stream=torch.cuda.current_stream())
    kv.init_free_order(rng.permutation(blocks))
    fill_sequences([("gpu", kv)], dict(enumerate(lens0)), rng, kvd)
    seqs = np.arange(12, dtype=np.uint32)
    sm = torch.from_numpy(kv.append_batch(seqs, np.array(lens0, np.uint64))).to(gpu)
    tables, la = tables_and_lens(kv, seqs, [n + 1 for n in lens0])
    d_tables, d_lens = torch.from_numpy(tables).to(gpu), torch.from_numpy(la).to(gpu)
    d_rows = torch.from_numpy(kv.seq_rows(seqs)).to(gpu)
    k = torch.randn((12, kvd), device=gpu)
    v = torch.randn((12, kvd), device=gpu)
    q = torch.randn((12, n_heads * hd), device=gpu)
    out = torch.empty_like(q)
    out_rows = torch.empty_like(q)

    def step():
        kv.write_batch(0, sm, k, v)
        kv.decode_attention(0, q, d_tables, d_lens, n_heads, hd, out=out)
        kv.decode_attention_rows(0, q, d_rows, d_lens, n_heads, hd, out=out_rows)

    step()  # eager, warm: workspace sized, resident tables uploaded
    torch.cuda.synchronize()
    want, want_rows = out.clone(), out_rows.clone()

    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        kv.set_stream(torch.cuda.current_stream())  # the capture stream
        step()
    kv.set_stream(torch.cuda.current_stream())
    for r in range(4):
        out.zero_()
        out_rows.zero_()
        q.mul_(1.0)  # eager work between replays
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        np.testing.assert_array_equal(out.cpu().numpy().view(np.uint32), want.cpu().numpy().view(np.uint32),
                                      err_msg=f"replay {r}")
        np.testing.assert_array_equal(out_rows.cpu().numpy().view(np.uint32),
                                      want_rows.cpu().numpy().view(np.uint32), err_msg=f"replay {r} (rows)")
