"""Pins the CPU oracle before it is trusted as the checker.

* f32<->f16: numpy's IEEE-754 binary16 conversion (a library routine) and the
  host's F16C instructions, over every f16 bit pattern and ~3M f32 values.
* KvCache (kv.rs): the reference's two known-answer tests (kv.rs:202-229),
  hand-derived allocation orders, allocator invariants, and a content-level
  model (sequences as token lists, as MockBackend keeps them, mock.rs:127-136).
* Attention (model.rs:431-475): float64 numpy brute force on small inputs and
  the closed forms len==1 -> V row, equal keys -> mean of V, q == 0 -> mean of V.
* Pool (pool.rs:217-257): every task runs exactly once, concurrent callers.
"""

from __future__ import annotations

import threading

import numpy as np
import pytest

import oracle
from oracle import OracleError, OracleKv

BLOCK = 16


# ---------------------------------------------------------------------------- f16
def test_f16_to_f32_all_bit_patterns():
    bits = np.arange(1 << 16, dtype=np.uint32).astype(np.uint16)
    want = bits.view(np.float16).astype(np.float32)
    nan = np.isnan(want)
    for simd in (False, True):
        got = oracle.f16_to_f32(bits, simd=simd)
        np.testing.assert_array_equal(got[~nan].view(np.uint32), want[~nan].view(np.uint32))
        assert np.isnan(got[nan]).all()


def test_f32_to_f16_matches_numpy_rne():
    rng = np.random.default_rng(0)
    x = np.concatenate([
        (rng.integers(0, 2 ** 32, 1 << 21, dtype=np.uint64).astype(np.uint32)).view(np.float32),
        rng.standard_normal(1 << 19).astype(np.float32) * np.float32(1e-5),   # subnormal range
        rng.standard_normal(1 << 19).astype(np.float32) * np.float32(3e4),    # overflow edge
        np.array([65504, 65519.996, 65520, -65520, 2 ** -24, 2 ** -25, 1.5 * 2 ** -25, 2 ** -26,
                  1 + 2 ** -11, 1 + 3 * 2 ** -11, np.inf, -np.inf, 0.0, -0.0], dtype=np.float32),
    ])
    x = x[~np.isnan(x)]
    with np.errstate(over="ignore"):
        want = x.astype(np.float16).view(np.uint16)
    np.testing.assert_array_equal(oracle.f32_to_f16(x), want)
    np.testing.assert_array_equal(oracle.f32_to_f16(x, simd=True), want)


def test_f32_to_f16_ties_round_to_even():
    # 1 + 2^-11 is exactly halfway between 1 and 1 + 2^-10: ties go to the even mantissa.
    assert oracle.f32_to_f16(np.float32(1 + 2 ** -11))[()] == 0x3C00
    assert oracle.f32_to_f16(np.float32(1 + 3 * 2 ** -11))[()] == 0x3C02
    assert oracle.f32_to_f16(np.float32(65520.0))[()] == 0x7C00      # rounds up to inf
    assert oracle.f32_to_f16(np.float32(65519.99))[()] == 0x7BFF
    assert oracle.f32_to_f16(np.float32(2 ** -25))[()] == 0x0000      # tie to even: zero
    assert oracle.f32_to_f16(np.float32(1.5 * 2 ** -25))[()] == 0x0001


def test_f32_to_f16_nan_rule():
    """NaN keeps its top 10 payload bits and is made quiet (half's from_f32)."""
    payloads = np.array([0x7FC00000, 0x7F800001, 0xFFA00000, 0x7FFFFFFF, 0x7F802000], dtype=np.uint32)
    got = oracle.f32_to_f16(payloads.view(np.float32))
    want = ((payloads >> 16) & 0x8000) | 0x7C00 | 0x0200 | ((payloads >> 13) & 0x3FF)
    np.testing.assert_array_equal(got, want.astype(np.uint16))
    if oracle.has_f16c():
        np.testing.assert_array_equal(oracle.f32_to_f16(payloads.view(np.float32), simd=True), got)


# ---------------------------------------------------------------------------- KvCache
def _fill(kv, seq, n, base):
    for p in range(kv.len(seq), n):
        b, s = kv.append(seq, p)
        x = np.full(kv.kv_dim, base + p, dtype=np.float32)
        kv.write(0, b, s, x, x)


def test_share_then_diverge_copies_on_write():
    """kv.rs:202-217."""
    kv = OracleKv(1, 4, 256)
    _fill(kv, 0, 20, 0.0)
    kv.share(0, 1, 20)
    free_before = kv.free_blocks()
    b, s = kv.append(1, 20)
    kv.write(0, b, s, np.full(4, 1000.0, np.float32), np.full(4, 1000.0, np.float32))
    assert kv.free_blocks() == free_before - 1
    a = oracle.f16_to_f32(kv.rows(0, 0, 20)[0][:, 0])
    c = oracle.f16_to_f32(kv.rows(0, 1, 21)[0][:, 0])
    np.testing.assert_array_equal(a, c[:20])
    assert c[20] == 1000.0
    assert kv.len(0) == 20


@pytest.mark.parametrize("dtype", ["f16", "f32", "q8_0"])
def test_copy_blocks_is_the_cow_body(dtype):
    """ora_copy_blocks (the copy-on-write body of kv.rs:99-110, in bulk) against
    numpy copies of the pools: every layer's K and V rows (and Q8_0 scales) of
    each source block land in its destination, in pair order (a chain a->b,
    b->c moves a's rows to c), nothing else changes, out-of-range pairs are
    skipped."""
    rng = np.random.default_rng(5)
    L, kvd, nb = 3, 64, 12
    kv = OracleKv(L, kvd, nb * BLOCK, dtype=dtype)
    for layer in range(L):
        cells = np.arange(nb * BLOCK, dtype=np.int32)
        k = rng.standard_normal((cells.size, kvd), dtype=np.float32)
        kv.write_batch(layer, cells, k, -k)
    before = [kv.pool(layer) for layer in range(L)]
    sc_before = [kv.scales(layer) for layer in range(L)] if dtype == "q8_0" else None
    pairs = np.array([[1, 4], [4, 7], [9, 2], [-1, 3], [0, nb], [11, 0]], np.int32)
    assert kv.copy_blocks(pairs) == 4
    for layer in range(L):
        k, v = kv.pool(layer)
        want_k, want_v = before[layer][0].copy(), before[layer][1].copy()
        for a, b in pairs[:3].tolist() + [[11, 0]]:
            want_k[b], want_v[b] = want_k[a], want_v[a]
        np.testing.assert_array_equal(k, want_k)
        np.testing.assert_array_equal(v, want_v)
        np.testing.assert_array_equal(k[7], before[layer][0][1])  # the chain carried block 1's rows
        if dtype == "q8_0":
            ks, vs = kv.scales(layer)
            wk, wv = sc_before[layer][0].copy(), sc_before[layer][1].copy()
            for a, b in pairs[:3].tolist() + [[11, 0]]:
                wk[b], wv[b] = wk[a], wv[a]
            np.testing.assert_array_equal(ks, wk)
            np.testing.assert_array_equal(vs, wv)


def test_truncate_frees_blocks():
    """kv.rs:219-229."""
    kv = OracleKv(1, 4, 64)
    _fill(kv, 3, 40, 0.0)
    assert kv.free_blocks() == 1
    kv.truncate(3, 10)
    assert kv.free_blocks() == 3
    kv.truncate(3, 0)
    assert kv.free_blocks() == 4
    with pytest.raises(OracleError, match="not contiguous"):
        kv.append(3, 5)


def test_allocation_order_is_lifo_from_zero():
    """(0..n).rev() free stack: a fresh cache hands out 0,1,2,...; released
    blocks are pushed in table order, so the last released is reused first."""
    kv = OracleKv(1, 8, 10 * BLOCK)
    for p in range(48):
        kv.append(0, p)
    np.testing.assert_array_equal(kv.block_table(0), [0, 1, 2])
    for p in range(20):
        kv.append(1, p)
    np.testing.assert_array_equal(kv.block_table(1), [3, 4])
    kv.truncate(0, 5)  # releases blocks 1 then 2: stack top is 2
    for p in range(33):
        kv.append(2, p)
    np.testing.assert_array_equal(kv.block_table(2), [2, 1, 5])


def test_error_messages_match_reference():
    kv = OracleKv(1, 8, 2 * BLOCK)
    with pytest.raises(OracleError, match=r"^seq 7: position 3 is not contiguous \(length 0\)$"):
        kv.append(7, 3)
    for p in range(32):
        kv.append(0, p)
    with pytest.raises(OracleError, match=r"^KV cache full$"):
        kv.append(1, 0)
    with pytest.raises(OracleError, match=r"^KV cache full$"):
        kv.append(0, 32)


def test_cow_count_is_holders_minus_one():
    """n holders of a partially filled shared block: the first n-1 appenders
    copy, the last holder (refcount 1 by then) writes in place."""
    kv = OracleKv(1, 8, 64 * BLOCK)
    for p in range(40):
        kv.append(0, p)
    for d in range(1, 6):
        kv.share(0, d, 40)
    assert kv.refcount(kv.block_table(0)[-1]) == 6
    for s in range(6):
        kv.append(s, 40)
    assert kv.cow_copies() == 5
    # an aligned share (len % 16 == 0) needs no copy: a fresh block is allocated
    for d in range(10, 13):
        kv.share(0, d, 32)
    for d in range(10, 13):
        kv.append(d, 32)
    assert kv.cow_copies() == 5


def _invariants(kv, model):
    """free + distinct blocks in use == n_blocks; refcount == number of holders;
    each table has ceil(len/16) blocks; lengths agree with the model."""
    holders = {}
    for s, toks in model.items():
        assert kv.len(s) == len(toks)
        t = kv.block_table(s)
        assert len(t) == -(-len(toks) // BLOCK)
        for b in t:
            holders[int(b)] = holders.get(int(b), 0) + 1
    assert kv.free_blocks() + len(holders) == kv.n_blocks
    for b in range(kv.n_blocks):
        assert kv.refcount(b) == holders.get(b, 0)


def test_random_ops_against_content_model():
    """Random append / truncate / share against a model that keeps each
    sequence as a list of values (MockBackend's view, mock.rs:127-136): the
    paged rows must always read back as the model's contents."""
    rng = np.random.default_rng(7)
    kv = OracleKv(1, 8, 40 * BLOCK, dtype="f32")  # f32 storage keeps every counter value exact
    model: dict[int, list[float]] = {}
    counter = 0.0
    for step in range(1500):
        op = rng.choice(["append", "append", "append", "truncate", "share"])
        s = int(rng.integers(0, 6))
        if op == "append":
            n = int(rng.integers(1, 20))
            for _ in range(n):
                pos = len(model.get(s, []))
                try:
                    b, sl = kv.append(s, pos)
                except OracleError as e:
                    assert "KV cache full" in str(e)
                    break
                counter += 1.0
                x = np.full(8, counter, dtype=np.float32)
                kv.write(0, b, sl, x, x)
                model.setdefault(s, []).append(counter)
        elif op == "truncate":
            frm = int(rng.integers(0, 60))
            kv.truncate(s, frm)
            if s in model and frm < len(model[s]):
                model[s] = model[s][:frm]
                if frm == 0:
                    del model[s]
        else:
            d = int(rng.integers(0, 6))
            n = int(rng.integers(0, 80))
            kv.share(s, d, n)
            # share truncates dst first, so share(s, s, n) empties s (kv.rs:173-174)
            src = model.get(s)
            model.pop(d, None)
            if s != d and src is not None and min(n, len(src)) > 0:
                model[d] = list(src[:min(n, len(src))])
        model = {k: v for k, v in model.items() if v}
        _invariants(kv, model)
        for t, toks in model.items():
            k, _ = kv.rows(0, t, len(toks))
            np.testing.assert_array_equal(k[:, 0], np.array(toks, dtype=np.float32))


def test_init_free_order_seeds_allocation():
    kv = OracleKv(1, 8, 8 * BLOCK)
    order = [5, 2, 7, 0, 1, 3, 6, 4]
    kv.init_free_order(order)
    for p in range(8 * BLOCK):
        kv.append(0, p)
    np.testing.assert_array_equal(kv.block_table(0), order)


# ---------------------------------------------------------------------------- attention
def _brute_force(kv_rows_k, kv_rows_v, q, n_heads, head_dim, scale):
    """float64 softmax(q k^T * scale) v for one token, GQA contiguous groups."""
    kvd = kv_rows_k.shape[1]
    n_kv = kvd // head_dim
    g = n_heads // n_kv
    out = np.zeros(n_heads * head_dim)
    for h in range(n_heads):
        kh = h // g
        k = kv_rows_k[:, kh * head_dim:(kh + 1) * head_dim].astype(np.float64)
        v = kv_rows_v[:, kh * head_dim:(kh + 1) * head_dim].astype(np.float64)
        s = k @ q[h * head_dim:(h + 1) * head_dim].astype(np.float64) * scale
        w = np.exp(s - s.max())
        w /= w.sum()
        out[h * head_dim:(h + 1) * head_dim] = w @ v
    return out


@pytest.mark.parametrize("dtype", ["f16", "f32"])
@pytest.mark.parametrize("n_heads,n_kv,hd", [(8, 2, 64), (7, 1, 128), (4, 4, 16), (6, 2, 20)])
def test_attention_matches_float64_brute_force(dtype, n_heads, n_kv, hd):
    rng = np.random.default_rng(n_heads * 100 + hd)
    kvd = n_kv * hd
    kv = OracleKv(1, kvd, 30 * BLOCK, dtype=dtype)
    lens = [1, 9, 16, 17, 120]
    rows = {}
    for s, n in enumerate(lens):
        k = rng.standard_normal((n, kvd), dtype=np.float32)
        v = rng.standard_normal((n, kvd), dtype=np.float32)
        for p in range(n):
            b, sl = kv.append(s, p)
            kv.write(0, b, sl, k[p], v[p])
        rows[s] = kv.rows(0, s, n)
    q = rng.standard_normal((len(lens), n_heads * hd), dtype=np.float32)
    scale = 1.0 / np.sqrt(hd)
    got = kv.attention(0, np.arange(len(lens)), np.array(lens) - 1, q, n_heads, hd, scale=float(scale), threads=3)
    for s, n in enumerate(lens):
        k, v = rows[s]
        if dtype == "f16":
            k, v = oracle.f16_to_f32(k), oracle.f16_to_f32(v)
        want = _brute_force(k, v, q[s], n_heads, hd, float(np.float32(scale)))
        np.testing.assert_allclose(got[s], want, atol=2e-6, rtol=1e-5)


def test_attention_closed_forms():
    rng = np.random.default_rng(3)
    kv = OracleKv(1, 64, 20 * BLOCK, dtype="f32")
    # seq 0: one position -> output is its V row exactly
    b, s = kv.append(0, 0)
    k0, v0 = rng.standard_normal(64, dtype=np.float32), rng.standard_normal(64, dtype=np.float32)
    kv.write(0, b, s, k0, v0)
    # seq 1: all K rows equal -> output is the mean of V
    kc = rng.standard_normal(64, dtype=np.float32)
    vs = rng.standard_normal((50, 64), dtype=np.float32)
    for p in range(50):
        b, s = kv.append(1, p)
        kv.write(0, b, s, kc, vs[p])
    q = rng.standard_normal((3, 4 * 64), dtype=np.float32)
    q[2] = 0.0  # seq 1 again with q = 0: also the mean of V
    out = kv.attention(0, [0, 1, 1], [0, 49, 49], q, 4, 64)
    np.testing.assert_array_equal(out[0], np.tile(v0, 4))
    mean = vs.astype(np.float64).mean(0)
    np.testing.assert_allclose(out[1], np.tile(mean, 4), atol=1e-6)
    np.testing.assert_allclose(out[2], np.tile(mean, 4), atol=1e-6)


def test_attention_thread_count_does_not_change_bits():
    """Tasks are independent, so results are deterministic (pool.rs / README:102)."""
    rng = np.random.default_rng(9)
    kv = OracleKv(1, 256, 64 * BLOCK)
    for s, n in enumerate([300, 5, 170]):
        k = rng.standard_normal((n, 256), dtype=np.float32)
        for p in range(n):
            b, sl = kv.append(s, p)
            kv.write(0, b, sl, k[p], -k[p])
    q = rng.standard_normal((3, 16 * 64), dtype=np.float32)
    a = kv.attention(0, [0, 1, 2], [299, 4, 169], q, 16, 64, threads=1)
    b = kv.attention(0, [0, 1, 2], [299, 4, 169], q, 16, 64, threads=5)
    np.testing.assert_array_equal(a, b)


@pytest.mark.parametrize("dtype", ["f16", "f32", "q8_0"])
def test_attention_tables_front_end_equals_attention_by_sequence(dtype):
    """ora_attention_tables, the checker of the GPU parity tests, is the
    by-sequence attention (model.rs:431-475 over the kv.rs tables) with the
    block tables handed in: the same bits on a permuted pool with forks that
    share blocks, queries at earlier positions than a sequence's end, rows
    padded with -1 past each length and a stride wider than any table. A -1
    or out-of-pool entry inside a length, or a stride too short for a length,
    is refused (kv.rs:147 panics there)."""
    rng = np.random.default_rng(21 + len(dtype))
    kvd, hd, n_heads = 256, 64, 12  # four kv heads, group 3
    n_blocks = 96
    kv = OracleKv(1, kvd, n_blocks * BLOCK, dtype=dtype)
    kv.init_free_order(rng.permutation(n_blocks))
    lens = {0: 200, 1: 17, 2: 1, 3: 64, 4: 0}
    for s, n in lens.items():
        if n:
            k = rng.standard_normal((n, kvd), dtype=np.float32) * 3
            v = rng.standard_normal((n, kvd), dtype=np.float32)
            kv.write_batch(0, kv.append_batch(np.full(n, s, np.uint32), np.arange(n, dtype=np.uint64)), k, v)
    kv.share(0, 5, 150)  # a fork; its next token copies the shared partial block
    sm = kv.append_batch(np.full(11, 5, np.uint32), np.arange(150, 161, dtype=np.uint64))
    kv.write_batch(0, sm, rng.standard_normal((11, kvd), dtype=np.float32),
                   rng.standard_normal((11, kvd), dtype=np.float32))
    assert kv.cow_copies() == 1
    seqs = np.array([0, 1, 2, 3, 5, 0, 5, 3], dtype=np.uint32)
    pos = np.array([199, 16, 0, 63, 160, 100, 15, 31], dtype=np.uint64)
    q = rng.standard_normal((seqs.size, n_heads * hd), dtype=np.float32)
    want = kv.attention(0, seqs, pos, q, n_heads, hd, threads=2)

    stride = 20  # wider than any table (13 blocks)
    tables = np.full((seqs.size, stride), -1, dtype=np.int32)
    for i, (s, p) in enumerate(zip(seqs, pos)):
        nb = -(-(int(p) + 1) // BLOCK)
        tables[i, :nb] = kv.block_table(int(s))[:nb]
    lens_a = (pos + 1).astype(np.int32)
    got = kv.attention_tables(0, tables, lens_a, q, n_heads, hd, threads=3)
    np.testing.assert_array_equal(got.view(np.uint32), want.view(np.uint32))
    # the same with the real table entries past each length left in place
    full = np.full((seqs.size, stride), -1, dtype=np.int32)
    for i, s in enumerate(seqs):
        t = kv.block_table(int(s))
        full[i, :t.size] = t
    got = kv.attention_tables(0, full, lens_a, q, n_heads, hd)
    np.testing.assert_array_equal(got.view(np.uint32), want.view(np.uint32))

    for bad in (-1, n_blocks):
        t = tables.copy()
        t[0, 12] = bad  # the last block of seq 0 at position 199
        with pytest.raises(OracleError):
            kv.attention_tables(0, t, lens_a, q, n_heads, hd)
    with pytest.raises(OracleError):
        kv.attention_tables(0, tables[:, :12].copy(), lens_a, q, n_heads, hd)


# ---------------------------------------------------------------------------- pool
def test_pool_runs_every_task_exactly_once():
    """pool.rs:217-227."""
    for n in (1, 3, 64, 1000):
        hits = oracle.pool_selftest(4, n)
        assert (hits == 1).all(), n


def test_pool_concurrent_callers():
    """pool.rs:229-250: several callers share one pool."""
    errors = []

    def caller():
        try:
            for _ in range(50):
                if not (oracle.pool_selftest(3, 17) == 1).all():
                    errors.append("miss")
        except Exception as e:  # pragma: no cover
            errors.append(repr(e))

    threads = [threading.Thread(target=caller) for _ in range(4)]
    for t in threads:
        t.start()
    for t in threads:
        t.join()
    assert not errors


# ---------------------------------------------------------------------------- RoPE (model.rs:291-308)
def _rope64(x, n_heads, head_dim, rope_dim, neox, base, pos):
    """float64 rotation on the same f32 angles (pos * inv_freq, both f32)."""
    x = x.astype(np.float64).copy()
    half = rope_dim // 2
    inv = np.array([np.float32(base) ** np.float32(-2.0 * i / rope_dim) for i in range(half)], dtype=np.float64)
    ang = (np.float32(pos) * inv.astype(np.float32)).astype(np.float64)
    for h in range(n_heads):
        v = x[h * head_dim:(h + 1) * head_dim]
        a = np.arange(half) if neox else 2 * np.arange(half)
        b = a + half if neox else a + 1
        x0, x1 = v[a].copy(), v[b].copy()
        v[a] = x0 * np.cos(ang) - x1 * np.sin(ang)
        v[b] = x0 * np.sin(ang) + x1 * np.cos(ang)
    return x


@pytest.mark.parametrize("neox,rope_dim,head_dim", [(False, 128, 128), (True, 128, 128), (True, 64, 128),
                                                    (False, 64, 64)])
def test_oracle_rope_against_float64(neox, rope_dim, head_dim):
    """The oracle's rotation (applied to q in place) against float64 numpy on
    the same f32 angles: pairing, signs and frequencies; position 0 is the
    identity and dimensions past rope_dim are untouched, bit for bit."""
    rng = np.random.default_rng(rope_dim + head_dim + neox)
    n_kv, n_heads = 2, 4
    kv_dim = n_kv * head_dim
    o = OracleKv(1, kv_dim, 64 * 16, dtype="f32")
    pos = np.array([0, 1, 7, 100, 4095, 32767], dtype=np.int32)
    sm = o.append_batch(np.zeros(pos.size, np.uint32), np.arange(pos.size, dtype=np.uint64))
    k = rng.standard_normal((pos.size, kv_dim), dtype=np.float32)
    q = rng.standard_normal((pos.size, n_heads * head_dim), dtype=np.float32)
    q0 = q.copy()
    o.write_rope_batch(0, sm, pos, k, k, 500000.0, rope_dim, head_dim, neox, q=q, n_heads=n_heads)
    np.testing.assert_array_equal(q[0], q0[0])
    for i, p in enumerate(pos):
        want = _rope64(q0[i], n_heads, head_dim, rope_dim, neox, 500000.0, int(p))
        np.testing.assert_allclose(q[i], want, rtol=0, atol=2e-6 * (1 + np.abs(want)).max())
        for h in range(n_heads):
            tail = slice(h * head_dim + rope_dim, (h + 1) * head_dim)
            np.testing.assert_array_equal(q[i, tail], q0[i, tail])
    kr, _ = o.rows(0, 0, pos.size)
    for i, p in enumerate(pos):  # f32 pools hold the rotated k exactly as the oracle computed it
        want = _rope64(k[i], n_kv, head_dim, rope_dim, neox, 500000.0, int(p))
        np.testing.assert_allclose(kr[i], want, rtol=0, atol=2e-6 * (1 + np.abs(want)).max())


# ---------------------------------------------------------------------------- Q8_0 (quant.rs:785-791)
def test_quantize_block_known_answers():
    """Hand-derived blocks: amax 127 gives d = 1 exactly, so q = round(x)
    with ties away from zero (RNE would give 2 for 2.5 and 0 for 0.5)."""
    x = np.zeros(32, np.float32)
    x[:10] = [127, 2.5, -2.5, 0.5, -0.5, 1.5, -1.5, 63.5, -126.5, 1.4999999]
    d, q = oracle.quantize_block(x)
    assert d == 1.0
    assert q[:10].tolist() == [127, 3, -3, 1, -1, 2, -2, 64, -127, 1]
    assert (q[10:] == 0).all()
    # amax 254: d = 2, id = 0.5; 5 -> 2.5 -> 3, -7 -> -3.5 -> -4, 1 -> 0.5 -> 1
    x = np.zeros(32, np.float32)
    x[:4] = [-254, 5, -7, 1]
    d, q = oracle.quantize_block(x)
    assert d == 2.0 and q[:4].tolist() == [-127, 3, -4, 1]


def test_quantize_block_special_values():
    # all zeros: d = 0, id = 0
    d, q = oracle.quantize_block(np.zeros(32, np.float32))
    assert d == 0.0 and (q == 0).all()
    # NaN is skipped by f32::max and quantises to 0 (NaN as i8 == 0)
    x = np.zeros(32, np.float32)
    x[0], x[1], x[2] = np.nan, 127.0, -3.0
    d, q = oracle.quantize_block(x)
    assert d == 1.0 and q[0] == 0 and q[1] == 127 and q[2] == -3
    x[:] = np.nan
    d, q = oracle.quantize_block(x)
    assert d == 0.0 and (q == 0).all()
    # inf: d = inf, id = 1 / inf = 0; inf * 0 = NaN -> 0, finite * 0 = 0
    x = np.ones(32, np.float32)
    x[3] = -np.inf
    d, q = oracle.quantize_block(x)
    assert d == np.inf and (q == 0).all()
    # subnormal amax: 1 / d overflows to inf, so quants saturate (as i8 of +-inf)
    x = np.zeros(32, np.float32)
    x[:3] = [1e-40, -1e-40, 0.0]
    d, q = oracle.quantize_block(x)
    assert d == np.float32(np.float32(1e-40) / np.float32(127))
    with np.errstate(over="ignore"):
        assert np.isinf(np.float32(1.0) / np.float32(d))
    assert q[:3].tolist() == [127, -128, 0]


def test_quantize_block_round_trip_bound():
    """Random blocks over many magnitudes: q = round(x / d) within
    [-127, 127], the element of largest magnitude maps to +-127, and
    |x - d q| <= d / 2 (up to the rounding of x * id)."""
    rng = np.random.default_rng(7)
    for i in range(2000):
        x = (rng.standard_normal(32) * 10.0 ** rng.integers(-30, 30)).astype(np.float32)
        d, q = oracle.quantize_block(x)
        assert d == np.float32(np.abs(x).max()) / np.float32(127)
        assert np.abs(q.astype(int)).max() == 127
        j = np.argmax(np.abs(x))
        assert q[j] == np.sign(x[j]) * 127
        err = np.abs(x.astype(np.float64) - np.float64(d) * q)
        assert (err <= 0.5 * d * (1 + 1e-5)).all(), i


def test_q8_pool_layout_and_attention():
    """Q8_0 storage: row quants and per-32 f16 scales equal quantize_block of
    each 32-element run; attention equals the float64 brute force over the
    dequantised rows d * q, which stay within d / 2 (+ the f16 rounding of d)
    of the rows written; copy-on-write copies scales with quants."""
    rng = np.random.default_rng(11)
    n_heads, n_kv, hd = 8, 2, 64
    kvd = n_kv * hd
    kv = OracleKv(1, kvd, 40 * BLOCK, dtype="q8_0")
    lens = [1, 17, 120]
    written = {}
    for s, n in enumerate(lens):
        k = rng.standard_normal((n, kvd), dtype=np.float32)
        v = rng.standard_normal((n, kvd), dtype=np.float32)
        for p in range(n):
            b, sl = kv.append(s, p)
            kv.write(0, b, sl, k[p], v[p])
        written[s] = (k, v)
    kv.share(2, 5, 100)
    b, sl = kv.append(5, 100)  # copy-on-write of block 6 of seq 2
    kv.write(0, b, sl, *[rng.standard_normal(kvd, dtype=np.float32)] * 2)
    written[5] = tuple(np.concatenate([w[:100], np.zeros((1, kvd), np.float32)]) for w in written[2])
    qk, qv = kv.pool(0)
    sk, sv = kv.scales(0)

    def deq(quants, scales, seq, n):
        t = kv.block_table(seq)
        cells = [(t[p // BLOCK], p % BLOCK) for p in range(n)]
        qs = np.stack([quants[b, s] for b, s in cells]).astype(np.float64)
        ds = np.stack([oracle.f16_to_f32(scales[b, s]) for b, s in cells]).astype(np.float64)
        return qs * np.repeat(ds, 32, axis=1)

    for s, n in enumerate(lens):
        t = kv.block_table(s)
        for p in range(n):
            for blk in range(kvd // 32):
                d, q = oracle.quantize_block(written[s][0][p, blk * 32:(blk + 1) * 32])
                assert sk[t[p // BLOCK], p % BLOCK, blk] == oracle.f32_to_f16(np.float32(d))
                np.testing.assert_array_equal(qk[t[p // BLOCK], p % BLOCK, blk * 32:(blk + 1) * 32], q)
    q = rng.standard_normal((4, n_heads * hd), dtype=np.float32)
    seqs, n_ctx = [0, 1, 2, 5], lens + [100]
    got = kv.attention(0, np.array(seqs), np.array(n_ctx[:3] + [100]) - 1, q, n_heads, hd, threads=2)
    for i, (s, n) in enumerate(zip(seqs, n_ctx)):
        k = deq(qk, sk, s, n)
        v = deq(qv, sv, s, n)
        bound = np.repeat(np.abs(written[s][0][:n]).reshape(n, -1, 32).max(axis=2) / 127, 32, axis=1)
        assert (np.abs(k - written[s][0][:n]) <= bound * (0.5 + 2 ** -10 * 128)).all()
        want = _brute_force(k, v, q[i], n_heads, hd, float(np.float32(1.0 / np.sqrt(hd))))
        np.testing.assert_allclose(got[i], want, atol=2e-6, rtol=1e-5)
