#!/usr/bin/env python3
"""Writes the small committed fixtures under tests/golden/.

The reference holds no golden vectors for this path (its only known-answer
tests are kv.rs:202-229, restated in the tests directly). These fixtures are
produced here from seeded inputs by numpy (IEEE f16 rounding) and the CPU
oracle (whose functions are pinned in tests/test_oracle.py), and then serve
as fixed regression vectors for both the oracle and the HIP product:

  f16_vectors.npz      f32 inputs -> f16 bits (numpy RNE; NaN rule of f16::from_f32)
  kv_trace.json        a seeded op trace on a 12-block cache with every result
  attention_small.npz  a 3-sequence GQA case: K/V/Q inputs, stored f16 rows,
                       oracle output and float64 reference output

Run from the repository root: python tests/golden/make_golden.py
"""

from __future__ import annotations

import json
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))

from oracle import OracleError, OracleKv  # noqa: E402

BLOCK = 16


def f16_vectors():
    rng = np.random.default_rng(1234)
    edge = np.array([0.0, -0.0, 1.0, -2.5, 65504.0, 65519.99, 65520.0, -65520.0, 1e9, np.inf, -np.inf,
                     2 ** -24, 2 ** -25, 1.5 * 2 ** -25, 2 ** -26, 2 ** -14, 2 ** -14 - 2 ** -25,
                     1 + 2 ** -11, 1 + 3 * 2 ** -11, 1 + 2 ** -12, 6.1e-5, 1e-8, 3.14159265],
                    dtype=np.float32)
    rand = np.concatenate([rng.standard_normal(2000).astype(np.float32),
                           (rng.standard_normal(1000) * 1e-5).astype(np.float32),
                           (rng.integers(0, 2 ** 32, 2000, dtype=np.uint64).astype(np.uint32)).view(np.float32)])
    x = np.concatenate([edge, rand])
    nan = np.isnan(x)
    with np.errstate(over="ignore", invalid="ignore"):
        bits = x.astype(np.float16).view(np.uint16)
    u = x.view(np.uint32)
    nan_bits = (((u >> 16) & 0x8000) | 0x7C00 | 0x0200 | ((u >> 13) & 0x3FF)).astype(np.uint16)
    bits = np.where(nan, nan_bits, bits)
    # pad to a multiple of 8 (the product writes rows of kv_dim % 8 == 0)
    pad = (-x.size) % 64
    x = np.concatenate([x, np.zeros(pad, np.float32)])
    bits = np.concatenate([bits, np.zeros(pad, np.uint16)])
    np.savez_compressed(os.path.join(HERE, "f16_vectors.npz"), f32=x, f16_bits=bits)


def kv_trace():
    rng = np.random.default_rng(99)
    kv = OracleKv(1, 8, 12 * BLOCK)
    order = [int(b) for b in rng.permutation(12)]
    kv.init_free_order(order)
    ops = []
    for _ in range(400):
        r = rng.random()
        s = int(rng.integers(0, 5))
        if r < 0.55:
            pos = kv.len(s) if rng.random() < 0.93 else kv.len(s) + int(rng.integers(1, 3))
            try:
                res = list(kv.append(s, pos))
            except OracleError as e:
                res = ["err", e.code, str(e)]
            ops.append({"op": "append", "seq": s, "pos": pos, "result": res})
        elif r < 0.8:
            frm = int(rng.integers(0, 50))
            kv.truncate(s, frm)
            ops.append({"op": "truncate", "seq": s, "from": frm})
        else:
            d, n = int(rng.integers(0, 5)), int(rng.integers(0, 60))
            kv.share(s, d, n)
            ops.append({"op": "share", "src": s, "dst": d, "len": n})
        ops[-1]["free"] = kv.free_blocks()
        ops[-1]["cow"] = kv.cow_copies()
        ops[-1]["tables"] = {str(q): [int(b) for b in kv.block_table(q)] for q in range(5)}
        ops[-1]["lens"] = [kv.len(q) for q in range(5)]
    with open(os.path.join(HERE, "kv_trace.json"), "w") as f:
        json.dump({"n_layers": 1, "kv_dim": 8, "n_tokens": 12 * BLOCK, "free_order": order, "ops": ops}, f)


def attention_small():
    rng = np.random.default_rng(4321)
    n_heads, n_kv, hd = 8, 2, 64
    kvd = n_kv * hd
    lens = [1, 17, 40]
    kv = OracleKv(1, kvd, 10 * BLOCK)
    order = rng.permutation(10)
    kv.init_free_order(order)
    seqs = np.repeat(np.arange(3, dtype=np.uint32), lens)
    pos = np.concatenate([np.arange(n, dtype=np.uint64) for n in lens])
    sm = kv.append_batch(seqs, pos)
    k = rng.standard_normal((sm.size, kvd), dtype=np.float32)
    v = rng.standard_normal((sm.size, kvd), dtype=np.float32)
    kv.write_batch(0, sm, k, v)
    q = rng.standard_normal((3, n_heads * hd), dtype=np.float32)
    tables = np.stack([np.pad(kv.block_table(s), (0, 3 - len(kv.block_table(s))), constant_values=-1)
                       for s in range(3)]).astype(np.int32)
    out = kv.attention(0, np.arange(3), np.array(lens) - 1, q, n_heads, hd)
    rows_k = np.concatenate([kv.rows(0, s, n)[0] for s, n in enumerate(lens)])
    rows_v = np.concatenate([kv.rows(0, s, n)[1] for s, n in enumerate(lens)])
    ref64 = np.zeros((3, n_heads * hd))
    scale = float(np.float32(1.0 / np.sqrt(hd)))
    off = 0
    for s, n in enumerate(lens):
        kk = rows_k[off:off + n].view(np.float16).astype(np.float64)
        vv = rows_v[off:off + n].view(np.float16).astype(np.float64)
        off += n
        for h in range(n_heads):
            kh = h // (n_heads // n_kv)
            sc = kk[:, kh * hd:(kh + 1) * hd] @ q[s, h * hd:(h + 1) * hd].astype(np.float64) * scale
            w = np.exp(sc - sc.max())
            w /= w.sum()
            ref64[s, h * hd:(h + 1) * hd] = w @ vv[:, kh * hd:(kh + 1) * hd]
    np.savez_compressed(os.path.join(HERE, "attention_small.npz"), n_heads=n_heads, head_dim=hd,
                        kv_dim=kvd, lens=np.array(lens, np.int32), free_order=order.astype(np.uint32),
                        seqs=seqs, pos=pos, slot_mapping=sm, k=k, v=v, q=q, tables=tables,
                        rows_k=rows_k, rows_v=rows_v, out_oracle=out, out_f64=ref64)


if __name__ == "__main__":
    f16_vectors()
    kv_trace()
    attention_small()
    print("fixtures written to", HERE)
