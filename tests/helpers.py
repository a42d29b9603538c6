"""Shared builders for the parity tests: identical cache states on the HIP
product and on the CPU oracle, from the same seeded inputs."""

from __future__ import annotations

import numpy as np

BLOCK = 16


def special_f32(rng: np.random.Generator, n: int) -> np.ndarray:
    """Values that stress f32->f16 rounding: ties, subnormals, overflow, inf, NaN."""
    vals = [0.0, -0.0, 1.0, -1.0, 65504.0, 65519.99, 65520.0, -65520.0, 1e6, -1e6, np.inf, -np.inf,
            np.nan, 2.0 ** -24, 2.0 ** -25, 1.5 * 2.0 ** -25, 2.0 ** -26, 2.0 ** -14, 2.0 ** -15,
            1.0 + 2.0 ** -11, 1.0 + 3 * 2.0 ** -11, 1.0 + 2.0 ** -12, 6.1e-5, 1e-8, -1e-8, 3.14159]
    base = np.array(vals, dtype=np.float32)
    ties = (rng.integers(0, 1 << 23, n // 4).astype(np.uint32) & ~np.uint32(0x1fff)) | np.uint32(0x1000)
    ties = (ties | (rng.integers(100, 150, ties.size).astype(np.uint32) << 23)).view(np.float32)
    small = (rng.standard_normal(n // 4) * 1e-5).astype(np.float32)
    normal = rng.standard_normal(n - base.size - ties.size - small.size).astype(np.float32) * 100
    out = np.concatenate([base, ties, small, normal]).astype(np.float32)
    rng.shuffle(out)
    return out


def fill_sequences(caches, seq_lens, rng, kv_dim, layers=(0,), special=False):
    """Append positions 0..len-1 of every sequence (seq-major) and write the
    same K/V rows into every cache. `caches` holds (kind, cache) pairs with
    kind "gpu" (langtrain_studio_amd.KvCache) or "oracle" (oracle.OracleKv).
    Returns the f32 K and V rows written, per layer."""
    seqs = np.concatenate([np.full(n, s, dtype=np.uint32) for s, n in seq_lens.items()])
    pos = np.concatenate([np.arange(n, dtype=np.uint64) for n in seq_lens.values()])
    return append_rows(caches, seqs, pos, rng, kv_dim, layers, special)


def append_rows(caches, seqs, pos, rng, kv_dim, layers=(0,), special=False):
    """Claim cells for tokens (seqs[i], pos[i]) in every cache (in order, so
    copy-on-write happens as the reference's claim loop does) and write the
    same random K/V rows into them. Returns the slot mapping and the rows."""
    import torch

    seqs = np.asarray(seqs, dtype=np.uint32)
    pos = np.asarray(pos, dtype=np.uint64)
    sms = [c.append_batch(seqs, pos) for _, c in caches]
    for sm in sms[1:]:
        np.testing.assert_array_equal(sm, sms[0])
    rows = {}
    for layer in layers:
        if special:
            k = special_f32(rng, seqs.size * kv_dim).reshape(seqs.size, kv_dim)
            v = special_f32(rng, seqs.size * kv_dim).reshape(seqs.size, kv_dim)
        else:
            k = rng.standard_normal((seqs.size, kv_dim), dtype=np.float32)
            v = rng.standard_normal((seqs.size, kv_dim), dtype=np.float32)
        for kind, c in caches:
            if kind == "gpu":
                dev = torch.device("cuda", c.device)
                c.write_batch(layer, torch.from_numpy(sms[0]).to(dev), torch.from_numpy(k).to(dev),
                              torch.from_numpy(v).to(dev))
            else:
                c.write_batch(layer, sms[0], k, v)
        rows[layer] = (k, v)
    return sms[0], rows


def tables_and_lens(cache, seqs, lens, stride=None):
    seqs = np.asarray(seqs, dtype=np.uint32)
    lens = np.asarray(lens, dtype=np.int32)
    need = int(np.ceil(lens.max() / BLOCK)) if lens.size else 1
    stride = max(1, need) if stride is None else stride
    return cache.block_tables(seqs, stride), lens


def attention_close(got: np.ndarray, want: np.ndarray, dtype: str):
    """The tolerance stated for this path: max abs <= 1e-3 (f32 KV) or 2e-2
    (f16 KV), and relative L2 <= 1e-3. A q8_0 cache is held to the f32 bar
    against the oracle's attention over the same dequantised rows d * q."""
    atol = 1e-3 if dtype in ("f32", "q8_0") else 2e-2
    err = np.abs(got.astype(np.float64) - want.astype(np.float64))
    rel = np.linalg.norm(got.astype(np.float64) - want) / max(np.linalg.norm(want.astype(np.float64)), 1e-30)
    assert np.isfinite(got).all(), "non-finite attention output"
    assert err.max() <= atol, f"max abs error {err.max():.3e} > {atol}"
    assert rel <= 1e-3, f"relative L2 error {rel:.3e} > 1e-3"
    return float(err.max()), float(rel)
