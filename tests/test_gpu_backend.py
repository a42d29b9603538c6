"""PagedKvBackend driven like the engine drives NativeBackend: prefill
chunks, forks through kv_copy, decode steps, kv_remove, over two layers.
Every layer's attention is checked against the oracle's restatement of
model.rs:431-475 over its own allocator, for each way of handing the step's
tables to the device; "tables" and "resident" must agree bit for bit.
"""

from __future__ import annotations

import numpy as np
import pytest

from helpers import BLOCK, attention_close

pytestmark = pytest.mark.gpu

N_LAYERS, N_HEADS, N_KV, HD = 2, 8, 2, 64
KVD = N_KV * HD


def _script():
    """(kind, args) steps: batches are lists of (seq, pos)."""
    steps = [("batch", [(0, p) for p in range(40)] + [(1, p) for p in range(20)])]
    steps += [("copy", (0, 2, 33)), ("copy", (0, 3, 40))]
    lens = {0: 40, 1: 20, 2: 33, 3: 40}
    for _ in range(5):
        steps.append(("batch", [(s, lens[s]) for s in (0, 1, 2, 3)]))
        for s in lens:
            lens[s] += 1
    steps.append(("remove", (1, 10)))
    lens[1] = 10
    steps.append(("batch", [(1, 10), (1, 11), (0, lens[0]), (2, lens[2])]))
    lens[1], lens[0], lens[2] = 12, lens[0] + 1, lens[2] + 1
    steps.append(("remove", (3, 0)))
    steps.append(("batch", [(s, lens[s]) for s in (0, 1, 2)] + [(7, p) for p in range(18)]))
    return steps


def _run(gpu, descriptor):
    import torch

    from langtrain_studio_amd import BatchToken, PagedKvBackend
    from oracle import OracleKv

    n_tokens = 64 * BLOCK
    be = PagedKvBackend(N_LAYERS, N_HEADS, N_KV, HD, n_tokens, n_seq_max=8, descriptor=descriptor)
    o = OracleKv(N_LAYERS, KVD, n_tokens)
    rng = np.random.default_rng(77)
    outs = []
    for kind, arg in _script():
        if kind == "copy":
            be.kv_copy(*arg)
            o.share(*arg)
            continue
        if kind == "remove":
            be.kv_remove(*arg)
            o.truncate(*arg)
            continue
        seqs = np.array([s for s, _ in arg], dtype=np.uint32)
        pos = np.array([p for _, p in arg], dtype=np.uint64)
        plan = be.begin_step([BatchToken(token=0, pos=int(p), seq=int(s)) for s, p in arg])
        sm = o.append_batch(seqs, pos)
        np.testing.assert_array_equal(plan.slot_mapping_host, sm)
        for layer in range(N_LAYERS):
            k = rng.standard_normal((len(arg), KVD), dtype=np.float32)
            v = rng.standard_normal((len(arg), KVD), dtype=np.float32)
            q = rng.standard_normal((len(arg), N_HEADS * HD), dtype=np.float32)
            out = be.layer(plan, layer, torch.from_numpy(q).to(gpu), torch.from_numpy(k).to(gpu),
                           torch.from_numpy(v).to(gpu)).cpu().numpy()
            o.write_batch(layer, sm, k, v)
            want = o.attention(layer, seqs, pos, q, N_HEADS, HD, threads=4)
            attention_close(out, want, "f16")
            outs.append(out)
    return outs


@pytest.mark.parametrize("descriptor", ["tables", "resident", "planned"])
def test_engine_loop_matches_oracle(gpu, descriptor):
    _run(gpu, descriptor)


def test_resident_descriptor_is_bit_identical_to_tables(gpu):
    for a, b in zip(_run(gpu, "tables"), _run(gpu, "resident")):
        np.testing.assert_array_equal(a.view(np.uint32), b.view(np.uint32))


def test_begin_step_errors_like_the_reference(gpu):
    from langtrain_studio_amd import BatchToken, KvCacheFull, NonContiguous, PagedKvBackend

    be = PagedKvBackend(1, 8, 2, 64, 2 * BLOCK)
    with pytest.raises(NonContiguous):
        be.begin_step([BatchToken(token=0, pos=3, seq=0)])  # kv.rs:88-91
    be.begin_step([BatchToken(token=0, pos=p, seq=0) for p in range(2 * BLOCK)])
    with pytest.raises(KvCacheFull):
        be.begin_step([BatchToken(token=0, pos=0, seq=1)])  # kv.rs:71
