"""Parity at the full sizes of the benchmarked workloads (Llama-3-8B layer:
32 q heads / 8 kv heads / head_dim 128, f16, 16-token blocks over permuted
pools), through the oracle where it finishes in seconds and through exact
properties where it would not.

* decode step, 64 sequences, contexts U[2048, 4096]: attention against the
  oracle on the read-back pool (tolerance), batch invariance and attention by
  resident rows (bit-exact);
* the same step as one fused append + attention launch (the timed entry
  point): bit-equal to write + attention on a twin cache, within tolerance
  of the oracle on both attention engines;
* the same step on a q8_0 cache: attention against the oracle over the
  read-back quants and scales, batch invariance (bit-exact);
* long context, 32 x 32 768 tokens, fully permuted pool (4.3 GB): the gather
  of every sequence equals the f16 rounding of the rows written, in order
  (bit-exact), and attention matches the oracle;
* prefix sharing, 256 forks of a 4088-token prefix with 64-token suffixes:
  255 copy-on-write copies each equal to the shared block's prefix rows
  (bit-exact), and planned (grouped) attention matches the oracle.
"""

from __future__ import annotations

import numpy as np
import pytest

from helpers import BLOCK, attention_close

pytestmark = pytest.mark.gpu

N_HEADS, N_KV, HD = 32, 8, 128
KVD = N_KV * HD


def _cache(n_blocks, seed, dtype="f16"):
    import torch

    from langtrain_studio_amd import KvCache

    kv = KvCache(1, KVD, n_blocks * BLOCK, dtype=dtype, device=0, stream=torch.cuda.current_stream())
    kv.init_free_order(np.random.default_rng(seed).permutation(n_blocks))
    return kv


def _write_random(kv, sm, seed, chunk=1 << 15):
    """Write N(0,1) K/V rows for slot mapping sm, chunk by chunk, from a
    seeded generator (regenerable with _random_rows)."""
    import torch

    for i, (k, v) in enumerate(_random_rows(sm.size, seed, chunk)):
        kv.write_batch(0, torch.from_numpy(sm[i * chunk:i * chunk + k.shape[0]]).cuda(), k, v)


def _random_rows(n, seed, chunk):
    import torch

    gen = torch.Generator(device="cuda")
    gen.manual_seed(seed)
    for i in range(0, n, chunk):
        m = min(chunk, n - i)
        yield (torch.randn((m, KVD), generator=gen, device="cuda"),
               torch.randn((m, KVD), generator=gen, device="cuda"))


def _oracle_with_pool(kv, n_blocks):
    from oracle import OracleKv

    o = OracleKv(1, KVD, n_blocks * BLOCK, dtype="f16")
    o.load_pool(0, *kv.read_pool(0))
    return o


def test_llama3_decode_step_full_size(gpu):
    import torch

    rng = np.random.default_rng(2024)
    B = 64
    ctx = rng.integers(2048, 4097, B)
    n_blocks = int(np.ceil(sum(-(-(int(c) + 1) // BLOCK) for c in ctx) * 1.1))
    kv = _cache(n_blocks, 1)
    seqs = np.repeat(np.arange(B, dtype=np.uint32), ctx)
    pos = np.concatenate([np.arange(int(c), dtype=np.uint64) for c in ctx])
    _write_random(kv, kv.append_batch(seqs, pos), 3)
    # the step: one appended token per sequence, then attention over len = ctx + 1
    step_sm = kv.append_batch(np.arange(B, dtype=np.uint32), ctx.astype(np.uint64))
    _write_random(kv, step_sm, 4)
    lens = (ctx + 1).astype(np.int32)
    tables = kv.block_tables(np.arange(B, dtype=np.uint32))
    q = torch.randn((B, N_HEADS * HD), generator=torch.Generator(device="cuda").manual_seed(5), device="cuda")
    d_tables, d_lens = torch.from_numpy(tables).cuda(), torch.from_numpy(lens).cuda()
    out = kv.decode_attention(0, q, d_tables, d_lens, N_HEADS, HD).cpu().numpy()

    o = _oracle_with_pool(kv, n_blocks)
    want = o.attention_tables(0, tables, lens, q.cpu().numpy(), N_HEADS, HD, threads=16)
    attention_close(out, want, "f16")

    # a query's bits do not depend on the rest of the batch
    sub = np.array([5, 17, 40, 63])
    alone = kv.decode_attention(0, q[sub].contiguous(), d_tables[sub].contiguous(), d_lens[sub].contiguous(),
                                N_HEADS, HD).cpu().numpy()
    np.testing.assert_array_equal(alone.view(np.uint32), out[sub].view(np.uint32))
    # the resident tables give the same bits
    rows = torch.from_numpy(kv.seq_rows(np.arange(B, dtype=np.uint32))).cuda()
    by_rows = kv.decode_attention_rows(0, q, rows, d_lens, N_HEADS, HD).cpu().numpy()
    np.testing.assert_array_equal(by_rows.view(np.uint32), out.view(np.uint32))


def test_llama3_fused_step_full_size(gpu):
    """The decode step as the headline times it: ltkv_append_decode_attention
    (model.rs:414-475 for one layer in one launch: the new K/V rows written
    by the waves of each query's last partition, attention over len = ctx + 1)
    at 64 sequences x U[2048, 4096] over a permuted pool, 64 queries x 4
    partitions taken longest first.
    * outputs and pools bit-equal to write + decode_attention on a twin cache;
    * outputs within the f16 tolerance of the oracle on the read-back pool;
    * the same step on the vector-ALU engine within the same tolerance."""
    import torch

    rng = np.random.default_rng(2026)
    B = 64
    ctx = rng.integers(2048, 4097, B)
    n_blocks = int(np.ceil(sum(-(-(int(c) + 1) // BLOCK) for c in ctx) * 1.1))
    fused, twin = _cache(n_blocks, 21), _cache(n_blocks, 21)
    seqs = np.repeat(np.arange(B, dtype=np.uint32), ctx)
    pos = np.concatenate([np.arange(int(c), dtype=np.uint64) for c in ctx])
    sm = fused.append_batch(seqs, pos)
    np.testing.assert_array_equal(twin.append_batch(seqs, pos), sm)
    _write_random(fused, sm, 22)
    _write_random(twin, sm, 22)
    step_seqs, step_pos = np.arange(B, dtype=np.uint32), ctx.astype(np.uint64)
    step_sm = fused.append_batch(step_seqs, step_pos)
    np.testing.assert_array_equal(twin.append_batch(step_seqs, step_pos), step_sm)
    assert (step_sm % BLOCK == 0).any() and (step_sm % BLOCK != 0).any()
    gen = torch.Generator(device="cuda").manual_seed(23)
    k = torch.randn((B, KVD), generator=gen, device="cuda")
    v = torch.randn((B, KVD), generator=gen, device="cuda")
    q = torch.randn((B, N_HEADS * HD), generator=gen, device="cuda")
    lens = (ctx + 1).astype(np.int32)
    tables = fused.block_tables(step_seqs)
    d_sm, d_tables, d_lens = (torch.from_numpy(x).cuda() for x in (step_sm, tables, lens))

    one = fused.append_decode_attention(0, d_sm, k, v, q, d_tables, d_lens, N_HEADS, HD).cpu().numpy()
    twin.write_batch(0, d_sm, k, v)
    two = twin.decode_attention(0, q, d_tables, d_lens, N_HEADS, HD).cpu().numpy()
    np.testing.assert_array_equal(one.view(np.uint32), two.view(np.uint32))
    fk, fv = fused.read_pool(0)
    tk, tv = twin.read_pool(0)
    np.testing.assert_array_equal(fk, tk)
    np.testing.assert_array_equal(fv, tv)
    del fk, fv, tk, tv, twin

    o = _oracle_with_pool(fused, n_blocks)
    want = o.attention_tables(0, tables, lens, q.cpu().numpy(), N_HEADS, HD, threads=16)
    attention_close(one, want, "f16")

    # the vector-ALU engine runs the same entry point as write + attention
    fused.set_attention_engine("valu")
    valu = fused.append_decode_attention(0, d_sm, k, v, q, d_tables, d_lens, N_HEADS, HD).cpu().numpy()
    fused.set_attention_engine("auto")
    attention_close(valu, want, "f16")
    assert not np.array_equal(valu.view(np.uint32), one.view(np.uint32))


def test_llama3_decode_step_full_size_q8(gpu):
    """The headline step on a q8_0 cache (the decode-q8 workload): attention
    against the oracle over the same quants and scales read back from the
    pool, and batch invariance bit for bit."""
    import torch

    from oracle import OracleKv

    rng = np.random.default_rng(2025)
    B = 64
    ctx = rng.integers(2048, 4097, B)
    n_blocks = int(np.ceil(sum(-(-(int(c) + 1) // BLOCK) for c in ctx) * 1.1))
    kv = _cache(n_blocks, 11, dtype="q8_0")
    seqs = np.repeat(np.arange(B, dtype=np.uint32), ctx + 1)
    pos = np.concatenate([np.arange(int(c) + 1, dtype=np.uint64) for c in ctx])
    _write_random(kv, kv.append_batch(seqs, pos), 12)
    lens = (ctx + 1).astype(np.int32)
    tables = kv.block_tables(np.arange(B, dtype=np.uint32))
    q = torch.randn((B, N_HEADS * HD), generator=torch.Generator(device="cuda").manual_seed(13), device="cuda")
    d_tables, d_lens = torch.from_numpy(tables).cuda(), torch.from_numpy(lens).cuda()
    out = kv.decode_attention(0, q, d_tables, d_lens, N_HEADS, HD).cpu().numpy()

    o = OracleKv(1, KVD, n_blocks * BLOCK, dtype="q8_0")
    o.load_pool(0, *kv.read_pool(0))
    ks, vs = kv.read_scales(0)  # [block][group][slot] -> the oracle's [block][slot][group]
    o.load_scales(0, ks.transpose(0, 2, 1), vs.transpose(0, 2, 1))
    want = o.attention_tables(0, tables, lens, q.cpu().numpy(), N_HEADS, HD, threads=16)
    attention_close(out, want, "q8_0")

    sub = np.array([3, 31, 62])
    alone = kv.decode_attention(0, q[sub].contiguous(), d_tables[sub].contiguous(), d_lens[sub].contiguous(),
                                N_HEADS, HD).cpu().numpy()
    np.testing.assert_array_equal(alone.view(np.uint32), out[sub].view(np.uint32))


def test_long_context_full_size(gpu):
    import torch

    B, ctx = 32, 32768
    n_blocks = B * ctx // BLOCK + 64
    kv = _cache(n_blocks, 6)
    sm = kv.append_batch(np.repeat(np.arange(B, dtype=np.uint32), ctx), np.tile(np.arange(ctx, dtype=np.uint64), B))
    chunk = 1 << 16
    _write_random(kv, sm, 7, chunk)
    tables = kv.block_tables(np.arange(B, dtype=np.uint32), ctx // BLOCK)
    d_tables = torch.from_numpy(tables).cuda()
    lens = torch.full((B,), ctx, dtype=torch.int32, device="cuda")
    offs = torch.arange(B, dtype=torch.int64, device="cuda") * ctx
    k_out = torch.empty((B * ctx, KVD), dtype=torch.float16, device="cuda")
    v_out = torch.empty_like(k_out)
    kv.gather(0, d_tables, lens, offs, k_out, v_out)
    # rows were written sequence-major, so the gather must return the
    # written rows in order, rounded to f16 (RNE), bit for bit
    for i, (k, v) in enumerate(_random_rows(sm.size, 7, chunk)):
        r = slice(i * chunk, i * chunk + k.shape[0])
        assert torch.equal(k_out[r].view(torch.int16), k.half().view(torch.int16)), f"K rows {r}"
        assert torch.equal(v_out[r].view(torch.int16), v.half().view(torch.int16)), f"V rows {r}"
    del k_out, v_out

    q = torch.randn((B, N_HEADS * HD), generator=torch.Generator(device="cuda").manual_seed(8), device="cuda")
    # 32 partitions of 1024 tokens per query, 4096 items x head pairs on the
    # chip's wave slots: each wave streams a run of four partitions
    out = kv.decode_attention(0, q, d_tables, lens, N_HEADS, HD).cpu().numpy()
    o = _oracle_with_pool(kv, n_blocks)
    want = o.attention_tables(0, tables, lens.cpu().numpy(), q.cpu().numpy(), N_HEADS, HD, threads=16)
    attention_close(out, want, "f16")
    # a query alone (a wave per partition) gives the bits it gets in the batch
    for i in (0, 17):
        one = kv.decode_attention(0, q[i:i + 1].contiguous(), d_tables[i:i + 1].contiguous(),
                                  lens[i:i + 1].contiguous(), N_HEADS, HD).cpu().numpy()
        np.testing.assert_array_equal(one[0].view(np.uint32), out[i].view(np.uint32))
    # the same step with 4096-token partitions fixed (8 a query instead of 32)
    kv.set_attention_partition(4096)
    out4 = kv.decode_attention(0, q, d_tables, lens, N_HEADS, HD).cpu().numpy()
    kv.set_attention_partition(0)
    attention_close(out4, want, "f16")


def test_prefix_sharing_full_size(gpu):
    import torch

    S, prefix, suffix = 256, 4088, 64
    n_blocks = (prefix + 15) // BLOCK + S * ((suffix + 8) // BLOCK + 2) + 64
    kv = _cache(n_blocks, 9)
    root = S  # the prefix's own sequence, forked S times
    _write_random(kv, kv.append_batch(np.full(prefix, root, np.uint32), np.arange(prefix, dtype=np.uint64)), 10)
    for s in range(S):
        kv.share(root, s, prefix)
    kv.truncate(root, 0)  # the forks hold the prefix alone now
    shared_last = int(kv.block_table(0)[prefix // BLOCK])
    before = kv.read_pool(0)[0][shared_last].copy()
    seqs = np.repeat(np.arange(S, dtype=np.uint32), suffix)
    pos = np.tile(np.arange(prefix, prefix + suffix, dtype=np.uint64), S)
    sm = kv.append_batch(seqs, pos)  # each fork's first append copies the partial block
    assert kv.cow_copies() == S - 1
    _write_random(kv, sm, 11)
    pool_k, pool_v = kv.read_pool(0)
    for s in range(S):
        b = int(kv.block_table(s)[prefix // BLOCK])
        # the prefix rows of the copied (or, for the last holder, original) block are the shared ones
        np.testing.assert_array_equal(pool_k[b][:prefix % BLOCK], before[:prefix % BLOCK])
    lens = np.full(S, prefix + suffix, dtype=np.int32)
    q = torch.randn((S, N_HEADS * HD), generator=torch.Generator(device="cuda").manual_seed(12), device="cuda")
    stats = kv.plan_attention(np.arange(S, dtype=np.uint32), lens, N_HEADS, HD)
    assert stats["groups"] == 1 and stats["grouped"] == S
    out = kv.planned_attention(0, q).cpu().numpy()
    tables = kv.block_tables(np.arange(S, dtype=np.uint32))
    o = _oracle_with_pool(kv, n_blocks)
    want = o.attention_tables(0, tables, lens, q.cpu().numpy(), N_HEADS, HD, threads=16)
    attention_close(out, want, "f16")


def test_qwen_mixed_step_full_size(gpu):
    """The continuous-batching mixed step at its own size (Qwen2.5-7B layer:
    28 q heads / 4 kv heads / head_dim 128, f16): 120 decode sequences with
    contexts U[512, 8192] and 8 prefill streams over a permuted pool; one churn
    round (finished sequences release their blocks, kv.rs:76-81, and arrivals
    allocate from the fragmented pool); then the step model.rs:380-475 runs on
    8 chunks of 512 tokens plus one token per decode sequence (4216 tokens),
    driven as scheduler.rs:389-407 batches them:
    * the claim gives the oracle's slot mapping and tables, and the fused RoPE
      append gives the oracle's pool and rotated Q, bit for bit;
    * decode attention of the 120 decode queries (the per-query kernel: G = 7,
      up to 9 partitions of 1024 tokens), per-query attention over all 4216
      tokens, and the planned step (each chunk a causal group) all match the
      oracle within the f16 tolerance;
    * the planned step's decode rows equal the per-query kernel's bit for bit."""
    import torch

    from langtrain_studio_amd import KvCache
    from oracle import OracleKv

    n_heads, n_kv, hd = 28, 4, 128
    kvd = n_kv * hd
    n_dec, n_pre, chunk = 120, 8, 512
    rng = np.random.default_rng(4004)
    n_blocks = int((n_dec + n_pre) * 8192 // BLOCK * 1.1)
    g = KvCache(1, kvd, n_blocks * BLOCK, dtype="f16", device=0, stream=torch.cuda.current_stream())
    o = OracleKv(1, kvd, n_blocks * BLOCK, dtype="f16")
    order = rng.permutation(n_blocks)
    g.init_free_order(order)
    o.init_free_order(order)
    history = []  # (slot mapping) of every claim, written with random rows below

    def claim(seqs, pos):
        seqs, pos = np.asarray(seqs, np.uint32), np.asarray(pos, np.uint64)
        sm = g.append_batch(seqs, pos)
        np.testing.assert_array_equal(sm, o.append_batch(seqs, pos))
        return sm

    def new_seq(sid, ctx):
        if ctx:
            history.append(claim(np.full(ctx, sid), np.arange(ctx)))

    dec = list(range(n_dec))
    for sid in dec:
        new_seq(sid, int(rng.integers(512, 8193)))
    # prefill streams: a prompt of U[512, 8192] tokens, some 512-token chunks done
    pre = []
    for i in range(n_pre):
        sid, target = 1000 + i, int(rng.integers(512, 8193))
        new_seq(sid, chunk * int(rng.integers(0, (target - chunk) // chunk + 1)))
        pre.append(sid)
    # churn: finished decode sequences free their blocks, arrivals take them
    finished = np.flatnonzero(rng.random(n_dec) < 0.05)
    assert finished.size >= 3
    for j, i in enumerate(finished):
        g.truncate(dec[i], 0)
        o.truncate(dec[i], 0)
        dec[i] = 2000 + j
        new_seq(dec[i], int(rng.integers(512, 8193)))
    assert g.free_blocks() == o.free_blocks()
    for sid in dec + pre:
        np.testing.assert_array_equal(g.block_table(sid), o.block_table(sid))
    for i, sm in enumerate(history):
        _write_random(g, sm, 100 + i)
    o.load_pool(0, *g.read_pool(0))

    # the mixed step: 8 chunks of 512 tokens, then one token per decode sequence
    seqs, pos = [], []
    for sid in pre:
        start = g.len(sid)
        seqs += [sid] * chunk
        pos += list(range(start, start + chunk))
    for sid in dec:
        seqs.append(sid)
        pos.append(g.len(sid))
    n = len(seqs)
    assert n == n_pre * chunk + n_dec
    sm = claim(seqs, pos)
    g.rope_init(1e6, hd, hd, True, 8192 + chunk + 1)
    k = rng.standard_normal((n, kvd), dtype=np.float32)
    v = rng.standard_normal((n, kvd), dtype=np.float32)
    q = rng.standard_normal((n, n_heads * hd), dtype=np.float32)
    pos32 = np.array(pos, np.int32)
    dq = torch.from_numpy(q.copy()).cuda()
    g.write_rope(0, torch.from_numpy(sm).cuda(), torch.from_numpy(pos32).cuda(), torch.from_numpy(k).cuda(),
                 torch.from_numpy(v).cuda(), q=dq, n_heads=n_heads)
    o.write_rope_batch(0, sm, pos32, k, v, 1e6, hd, hd, True, q=q, n_heads=n_heads)
    np.testing.assert_array_equal(dq.cpu().numpy().view(np.uint32), q.view(np.uint32))
    gk, gv = g.read_pool(0)
    ok, ov = o.pool(0)
    np.testing.assert_array_equal(gk, ok)
    np.testing.assert_array_equal(gv, ov)
    del gk, gv, ok, ov

    lens = pos32 + 1
    tables, la = g.block_tables(np.array(seqs, np.uint32)), lens.astype(np.int32)
    want = o.attention_tables(0, tables, la, q, n_heads, hd, threads=16)
    d_tables, d_lens = torch.from_numpy(tables).cuda(), torch.from_numpy(la).cuda()
    dsel = slice(n_pre * chunk, n)
    dec_out = g.decode_attention(0, dq[dsel].contiguous(), d_tables[dsel].contiguous(), d_lens[dsel].contiguous(),
                                 n_heads, hd).cpu().numpy()
    assert int(la[dsel].max()) > 7168  # the longest decode queries span 8+ partitions
    attention_close(dec_out, want[dsel], "f16")
    attention_close(g.decode_attention(0, dq, d_tables, d_lens, n_heads, hd).cpu().numpy(), want, "f16")
    stats = g.plan_attention(np.array(seqs, np.uint32), la, n_heads, hd)
    assert stats["groups"] == n_pre and stats["grouped"] == n_pre * chunk
    planned = g.planned_attention(0, dq).cpu().numpy()
    attention_close(planned, want, "f16")
    np.testing.assert_array_equal(planned[dsel].view(np.uint32), dec_out.view(np.uint32))
