"""The committed fixtures of tests/golden/ (written by make_golden.py) against
the oracle, the product's host logic (CPU) and the HIP kernels (GPU)."""

from __future__ import annotations

import json
import os

import numpy as np
import pytest

import oracle
from oracle import OracleError, OracleKv

HERE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def _load(name):
    return np.load(os.path.join(HERE, name), allow_pickle=False)


def test_oracle_f16_vectors():
    f = _load("f16_vectors.npz")
    np.testing.assert_array_equal(oracle.f32_to_f16(f["f32"]), f["f16_bits"])


def _replay(kv, trace, err_types):
    for i, op in enumerate(trace["ops"]):
        if op["op"] == "append":
            try:
                res = list(kv.append(op["seq"], op["pos"]))
            except err_types as e:
                res = ["err", e.code, str(e)]
            assert res == op["result"], (i, op, res)
        elif op["op"] == "truncate":
            kv.truncate(op["seq"], op["from"])
        else:
            kv.share(op["src"], op["dst"], op["len"])
        assert kv.free_blocks() == op["free"], i
        assert kv.cow_copies() == op["cow"], i
        assert [kv.len(q) for q in range(5)] == op["lens"], i
        for q, t in op["tables"].items():
            assert kv.block_table(int(q)).tolist() == t, (i, q)


def test_oracle_replays_kv_trace():
    trace = json.load(open(os.path.join(HERE, "kv_trace.json")))
    kv = OracleKv(trace["n_layers"], trace["kv_dim"], trace["n_tokens"])
    kv.init_free_order(trace["free_order"])
    _replay(kv, trace, OracleError)


def test_product_host_logic_replays_kv_trace():
    from langtrain_studio_amd import KvCache, KvError

    trace = json.load(open(os.path.join(HERE, "kv_trace.json")))
    kv = KvCache(trace["n_layers"], trace["kv_dim"], trace["n_tokens"], device=None)
    kv.init_free_order(trace["free_order"])
    _replay(kv, trace, KvError)


def test_oracle_attention_small():
    f = _load("attention_small.npz")
    kv = OracleKv(1, int(f["kv_dim"]), 10 * 16)
    kv.init_free_order(f["free_order"])
    np.testing.assert_array_equal(kv.append_batch(f["seqs"], f["pos"]), f["slot_mapping"])
    kv.write_batch(0, f["slot_mapping"], f["k"], f["v"])
    lens = f["lens"]
    rows_k = np.concatenate([kv.rows(0, s, int(n))[0] for s, n in enumerate(lens)])
    np.testing.assert_array_equal(rows_k, f["rows_k"])
    out = kv.attention(0, np.arange(3), lens - 1, f["q"], int(f["n_heads"]), int(f["head_dim"]))
    np.testing.assert_array_equal(out, f["out_oracle"])
    np.testing.assert_allclose(out, f["out_f64"], atol=2e-6, rtol=1e-5)


@pytest.mark.gpu
def test_gpu_write_f16_vectors(gpu):
    import torch

    from langtrain_studio_amd import KvCache

    f = _load("f16_vectors.npz")
    x, want = f["f32"], f["f16_bits"]
    kvd = 64
    rows = x.reshape(-1, kvd)
    kv = KvCache(1, kvd, 16 * (-(-rows.shape[0] // 16)), device=0)
    sm = kv.append_batch(np.zeros(rows.shape[0], np.uint32), np.arange(rows.shape[0]))
    d = torch.from_numpy(rows).to(gpu)
    kv.write_batch(0, torch.from_numpy(sm).to(gpu), d, d)
    k, v = kv.rows(0, 0, rows.shape[0])
    np.testing.assert_array_equal(k.reshape(-1), want)
    np.testing.assert_array_equal(v.reshape(-1), want)


@pytest.mark.gpu
def test_gpu_replays_kv_trace(gpu):
    from langtrain_studio_amd import KvCache, KvError

    trace = json.load(open(os.path.join(HERE, "kv_trace.json")))
    kv = KvCache(trace["n_layers"], trace["kv_dim"], trace["n_tokens"], device=0)
    kv.init_free_order(trace["free_order"])
    _replay(kv, trace, KvError)


@pytest.mark.gpu
def test_gpu_attention_small(gpu):
    import torch

    from helpers import attention_close
    from langtrain_studio_amd import KvCache

    f = _load("attention_small.npz")
    kv = KvCache(1, int(f["kv_dim"]), 10 * 16, device=0)
    kv.init_free_order(f["free_order"])
    sm = kv.append_batch(f["seqs"], f["pos"])
    np.testing.assert_array_equal(sm, f["slot_mapping"])
    kv.write_batch(0, torch.from_numpy(sm).to(gpu), torch.from_numpy(f["k"]).to(gpu),
                   torch.from_numpy(f["v"]).to(gpu))
    lens = f["lens"]
    rows_k = np.concatenate([kv.rows(0, s, int(n))[0] for s, n in enumerate(lens)])
    rows_v = np.concatenate([kv.rows(0, s, int(n))[1] for s, n in enumerate(lens)])
    np.testing.assert_array_equal(rows_k, f["rows_k"])
    np.testing.assert_array_equal(rows_v, f["rows_v"])
    out = kv.decode_attention(0, torch.from_numpy(f["q"]).to(gpu), torch.from_numpy(f["tables"]).to(gpu),
                              torch.from_numpy(lens).to(gpu), int(f["n_heads"]), int(f["head_dim"]))
    out = out.cpu().numpy()
    attention_close(out, f["out_oracle"], "f16")
    np.testing.assert_allclose(out, f["out_f64"], atol=1e-5, rtol=1e-4)
