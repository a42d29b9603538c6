#!/usr/bin/env python3
"""Benchmark of the MI355X paged KV-cache path (one GPU).

Default workload: a Llama-3-8B-shaped layer (32 query heads, 8 KV heads,
head_dim 128, f16 KV, 16-token blocks), 64 sequences with contexts drawn
uniformly from [2048, 4096], block tables over a permuted pool sized to the
sequences plus 10% free. One step = append one token per sequence + one GQA
paged decode-attention pass over the contexts including it; contexts grow by
one per step. `value` times the step as one launch (ltkv_append_decode_attention:
the attention kernel writes and uses each new row); the same steps as two
launches (write kernel, then attention) give `unfused_step_us` and the
per-kernel `append_us` / `attention_us`; `attention_valu_us` times the same
attention launches on the vector-ALU kernels (LTKV_ENGINE_VALU, no matrix
cores). Inputs are synthetic (seeded N(0,1)) and resident in HBM before the
timed region.

Prints one JSON line: the metric, µs per step, the attention kernel's roofline
(algorithmic bytes / HIP-event time of the unfused attention launch vs 8 TB/s),
and the CPU baseline (the oracle's restatement of the reference CPU path,
timed on this host's cores on the same state).
"""

from __future__ import annotations

import argparse
import json
import math
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

METRIC = "paged decode attn µs/step + KV append GB/s (% of HBM roofline), 1 GPU"
PEAK_HBM_GBPS = 8000.0
PEAK_F16_MFMA_TFLOPS = 2500.0  # dense
BLOCK = 16


def _args():
    p = argparse.ArgumentParser(description=__doc__.split("\n\n")[0])
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=100)
    p.add_argument("--warmup", type=int, default=5)
    p.add_argument("--seed", type=int, default=0)
    p.add_argument("--partition", type=int, default=0, help="attention partition tokens (0 = default)")
    p.add_argument("--kv-dtype", default="f16", choices=["f16", "q8_0"],
                   help="cache element type of the prefill and prefix-cow workloads")
    p.add_argument("--cpu-seconds", type=float, default=10.0, help="budget of the CPU baseline sample")
    p.add_argument("--cpu-threads", type=int, default=0,
                   help="CPU baseline threads (0 = every CPU of this process's share)")
    p.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    p.add_argument("--workload", default="decode",
                   choices=["decode", "copy", "copy-bulk", "append-sweep", "long-context", "tinyllama", "prefix-cow",
                            "mixed", "prefill", "rope-append", "decode-q8", "descriptor", "descriptor-long",
                            "decode-timeline", "decode-shapes"],
                   help="decode = the headline line; the others print measurement lines of their own")
    return p.parse_args()


TRAFFIC_PROFILE = "profiles/attn_mfma_llama3_decode.md"


def _profiled_traffic():
    """HBM bytes per attention launch (FETCH_SIZE x 2 + WRITE_SIZE, calibrated
    against a plain copy) from the committed rocprofv3 summary of this workload."""
    import re

    try:
        text = open(os.path.join(ROOT, TRAFFIC_PROFILE)).read()
    except OSError:
        return None
    m = re.search(r"traffic_bytes_per_launch = (\d+)", text)
    return int(m.group(1)) if m else None


def _host_cpus() -> str:
    """Logical CPUs this process may use and the host's CPU model and sockets."""
    try:
        usable = len(os.sched_getaffinity(0))
    except AttributeError:
        usable = os.cpu_count() or 1
    model, sockets, logical = "unknown", set(), 0
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                key, _, val = line.partition(":")
                key = key.strip()
                if key == "model name":
                    model = val.strip()
                elif key == "physical id":
                    sockets.add(val.strip())
                elif key == "processor":
                    logical += 1
    except OSError:
        pass
    return f"{usable} of {logical or '?'} logical CPUs usable, {len(sockets) or '?'} socket(s), {model}"


def _cpu_share() -> tuple[int, str]:
    """CPUs this process may run on: the affinity mask, bounded by the
    cgroup's CPU quota when one is set (the lease's real share of the host)."""
    try:
        aff = len(os.sched_getaffinity(0))
    except AttributeError:
        aff = os.cpu_count() or 1
    quota = None
    try:
        q, period = open("/sys/fs/cgroup/cpu.max").read().split()[:2]
        if q != "max":
            quota = max(1, int(q) // int(period))
    except (OSError, ValueError):
        try:
            q = int(open("/sys/fs/cgroup/cpu/cpu.cfs_quota_us").read())
            period = int(open("/sys/fs/cgroup/cpu/cpu.cfs_period_us").read())
            if q > 0:
                quota = max(1, q // period)
        except (OSError, ValueError):
            pass
    n = min(aff, quota) if quota else aff
    return n, f"{aff} CPUs in the affinity mask, cgroup CPU quota {quota if quota else 'none'}"


_CPU = None


def _oracle_calibration_ms(path: str) -> float:
    """One-thread time of a fixed attention job (4 queries x 2048 tokens,
    Llama-3-8B heads) on the oracle library at `path`: best of three."""
    from oracle import oracle as ora

    ora.use_library(path)
    rng = np.random.default_rng(0)
    kvd, n = 1024, 4 * 2048
    o = ora.OracleKv(1, kvd, n)
    sm = o.append_batch(np.repeat(np.arange(4, dtype=np.uint32), 2048), np.tile(np.arange(2048, dtype=np.uint64), 4))
    k = rng.standard_normal((n, kvd), dtype=np.float32)
    o.write_batch(0, sm, k, k)
    q = rng.standard_normal((4, 32 * 128), dtype=np.float32)
    best = float("inf")
    for _ in range(3):
        t0 = time.perf_counter()
        o.attention(0, np.arange(4, dtype=np.uint32), np.full(4, 2047, np.uint64), q, 32, 128, threads=1)
        best = min(best, time.perf_counter() - t0)
    return best * 1e3


def _cpu_setup(args) -> dict:
    """Once per run: the oracle built twice for this host's CPU (the prebuilt
    x86-64-v3 library, AVX2 + F16C, and a -march=native build made here), the
    faster of the two on a calibration job kept for the baseline; the thread
    count (every CPU of this process's share unless --cpu-threads) and a host
    description."""
    global _CPU
    if _CPU is None:
        import tempfile

        from oracle import oracle as ora

        builds = {"x86-64-v3 (prebuilt)": ora._LIB_PATH}
        note = ""
        try:
            builds["native (built on this host)"] = ora.build_native(tempfile.mkdtemp(prefix="ltkv_oracle_"))
        except Exception as e:  # noqa: BLE001 - the baseline still runs on the prebuilt library
            note = f"; -march=native build failed: {str(e)[:100]}"
        cal = {name: _oracle_calibration_ms(path) for name, path in builds.items()}
        best = min(cal, key=cal.get)
        ora.use_library(builds[best])
        build = (f"g++ -O3 -ffp-contract=off -march={best}, the faster on a one-thread calibration job ("
                 + ", ".join(f"{k}: {v:.1f} ms" for k, v in cal.items()) + ")" + note)
        threads, share = _cpu_share()
        if args.cpu_threads > 0:
            threads = args.cpu_threads
        _CPU = {"threads": threads, "host": f"{_host_cpus()}; {share}", "build": build}
    return _CPU


def _cpu_record(args, value: float, unit: str, sample: str, threads: int, **extra) -> dict:
    """The cpu_baseline object of a JSON line: the oracle (the C++ restatement
    of the reference CPU path) timed on this host."""
    cpu = _cpu_setup(args)
    rec = {"value": round(value, 1), "unit": unit, "cores": threads, "kind": "port", "sample": sample,
           "build": cpu["build"], "host": cpu["host"]}
    rec.update(extra)
    return rec


def _cpu_time(fn, n_max: int, budget_s: float, at_least: int = 1) -> tuple[float, int]:
    """Mean seconds of fn(i) for i = 0, 1, ... until n_max calls or the budget
    is spent (at least `at_least` calls)."""
    times = []
    t_end = time.perf_counter() + budget_s
    i = 0
    while i < n_max and (i < at_least or time.perf_counter() < t_end):
        t0 = time.perf_counter()
        fn(i)
        times.append(time.perf_counter() - t0)
        i += 1
    return float(np.mean(times)), i


class Llama3Decode:
    """The Llama-3-8B decode workload, built through the product's own API."""

    n_heads, n_kv, head_dim, batch = 32, 8, 128, 64

    def __init__(self, steps: int, seed: int, partition: int, dtype: str = "f16", ctx=None):
        import torch

        from langtrain_studio_amd import KvCache

        self.torch = torch
        self.dtype = dtype
        dev = torch.device("cuda", 0)
        self.dev = dev
        rng = np.random.default_rng(seed)
        B, kvd = self.batch, self.n_kv * self.head_dim
        self.kvd = kvd
        self.steps = steps
        self.ctx = rng.integers(2048, 4097, B)
        if ctx is not None:  # the same seeded pool order and data, other lengths
            self.ctx = np.asarray(ctx, dtype=np.int64)
        need = sum(math.ceil((int(c) + steps) / BLOCK) for c in self.ctx)
        self.n_blocks = int(math.ceil(need * 1.1))
        stream = torch.cuda.current_stream(dev)
        self.kv = KvCache(1, kvd, self.n_blocks * BLOCK, dtype=dtype, device=0, stream=stream)
        if partition:
            self.kv.set_attention_partition(partition)
        self.order = rng.permutation(self.n_blocks)
        self.kv.init_free_order(self.order)

        # Prefill: every sequence's positions, claimed through the allocator.
        self.pre_seqs = np.repeat(np.arange(B, dtype=np.uint32), self.ctx)
        self.pre_pos = np.concatenate([np.arange(int(c), dtype=np.uint64) for c in self.ctx])
        sm = self.kv.append_batch(self.pre_seqs, self.pre_pos)
        gen = torch.Generator(device=dev)
        gen.manual_seed(seed)
        chunk = 1 << 15
        for i in range(0, sm.size, chunk):
            n = min(chunk, sm.size - i)
            k = torch.randn((n, kvd), generator=gen, device=dev)
            v = torch.randn((n, kvd), generator=gen, device=dev)
            self.kv.write_batch(0, torch.from_numpy(sm[i:i + n]).to(dev), k, v)
        torch.cuda.synchronize()

        # Decode steps: claim every step's cell up front (host bookkeeping is
        # not part of the device timed region), tables cover the final length.
        seqs = np.arange(B, dtype=np.uint32)
        self.step_sm = np.stack([self.kv.append_batch(seqs, (self.ctx + s).astype(np.uint64))
                                 for s in range(steps)])
        self.stride = int(math.ceil((int(self.ctx.max()) + steps) / BLOCK))
        self.tables = self.kv.block_tables(seqs, self.stride)
        self.lens = np.stack([(self.ctx + s + 1).astype(np.int32) for s in range(steps)])
        self.d_sm = torch.from_numpy(self.step_sm).to(dev)
        self.d_tables = torch.from_numpy(self.tables).to(dev)
        self.d_lens = torch.from_numpy(self.lens).to(dev)
        rs = np.random.default_rng(seed + 1)
        self.q = rs.standard_normal((steps, B, self.n_heads * self.head_dim), dtype=np.float32)
        self.k_new = rs.standard_normal((steps, B, kvd), dtype=np.float32)
        self.v_new = rs.standard_normal((steps, B, kvd), dtype=np.float32)
        self.d_q = torch.from_numpy(self.q).to(dev)
        self.d_k = torch.from_numpy(self.k_new).to(dev)
        self.d_v = torch.from_numpy(self.v_new).to(dev)
        self.d_out = torch.empty((B, self.n_heads * self.head_dim), device=dev)
        torch.cuda.synchronize()

    def append(self, s: int):
        self.kv.write_batch(0, self.d_sm[s], self.d_k[s], self.d_v[s])

    def attend(self, s: int):
        self.kv.decode_attention(0, self.d_q[s], self.d_tables, self.d_lens[s], self.n_heads, self.head_dim,
                                 out=self.d_out)

    # Bytes one cached token row (K or V) occupies: f16 elements, or q8_0
    # quants plus one f16 scale per 32 elements.
    def row_bytes(self) -> int:
        return self.kvd * 2 if self.dtype == "f16" else self.kvd + self.kvd // 32 * 2

    # Algorithmic bytes of one launch at step s.
    def attention_bytes(self, s: int) -> float:
        lens = self.lens[s].astype(np.int64)
        kv = lens.sum() * 2 * self.row_bytes()
        qo = 2 * self.batch * self.n_heads * self.head_dim * 4
        tables = (-(-lens // BLOCK)).sum() * 4 + self.batch * 4
        return float(kv + qo + tables)

    def append_bytes(self) -> float:
        return float(self.batch * (self.kvd * (4 + 4) + 2 * self.row_bytes()) + self.batch * 4)


def cpu_baseline(w: Llama3Decode, threads: int, budget_s: float):
    """The oracle (C++ restatement of kv.rs + model.rs attention + pool.rs)
    running the same decode steps on the same cache state: (µs per step, steps)."""
    from oracle import OracleKv

    o = OracleKv(1, w.kvd, w.n_blocks * BLOCK, dtype=w.dtype)
    o.init_free_order(w.order)
    o.append_batch(w.pre_seqs, w.pre_pos)
    k, v = w.kv.read_pool(0)  # device state after the GPU run (same cells; the
    o.load_pool(0, k, v)      # timed steps rewrite the decode cells identically)
    if w.dtype == "q8_0":  # device layout [block][group][slot] -> the oracle's [block][slot][group]
        o.load_scales(0, *(x.transpose(0, 2, 1) for x in w.kv.read_scales(0)))
    seqs = np.arange(w.batch, dtype=np.uint32)

    def step(s):
        sm = o.append_batch(seqs, (w.ctx + s).astype(np.uint64))
        o.write_batch(0, sm, w.k_new[s], w.v_new[s])
        o.attention(0, seqs, (w.ctx + s).astype(np.uint64), w.q[s], w.n_heads, w.head_dim, threads=threads)

    sec, n = _cpu_time(step, w.steps, budget_s, at_least=2)
    return sec * 1e6, n


def _time_op(fn, reps: int, warmup: int = 2) -> float:
    """Mean µs of fn() over reps, HIP events on the current stream."""
    import torch

    for _ in range(warmup):
        fn()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    start.record()
    for _ in range(reps):
        fn()
    end.record()
    torch.cuda.synchronize()
    return start.elapsed_time(end) * 1e3 / reps


def bench_copy(args):
    """A plain device-to-device copy of known size: the calibration for the
    FETCH_SIZE / WRITE_SIZE counters (bytes the counters report per byte moved)."""
    import torch

    nbytes = 1 << 30
    src = torch.empty(nbytes // 4, dtype=torch.float32, device="cuda")
    src.fill_(1.0)
    dst = torch.empty_like(src)
    us = _time_op(lambda: dst.copy_(src), reps=max(args.steps, 1))
    print(json.dumps({"workload": "copy", "bytes_read": nbytes, "bytes_written": nbytes, "us": round(us, 2),
                      "GBps": round(2 * nbytes / (us * 1e-6) / 1e9, 1)}), flush=True)


def bench_copy_bulk(args):
    """Kernel 2, the copy-on-write body (kv.rs:99-110), on distinct blocks:
    131 072 (src, dst) pairs drawn from a permutation of a 262 144-block pool at
    the Llama-3-8B layer shape (K and V, 32 KiB each per block), so every
    source block is read once from HBM and every destination written once:
    8.6 GB read + 8.6 GB written per launch."""
    import torch

    from langtrain_studio_amd import KvCache

    n_pairs, kvd = 131072, 1024
    n_blocks = 2 * n_pairs
    rng = np.random.default_rng(args.seed)
    kv = KvCache(1, kvd, n_blocks * BLOCK, dtype="f16", device=0, stream=torch.cuda.current_stream())
    _fill_pool_random(kv, kvd, n_blocks, args.seed)
    pairs = rng.permutation(n_blocks).astype(np.int32).reshape(n_pairs, 2)
    d_pairs = torch.from_numpy(pairs).cuda()
    us = _time_op(lambda: kv.copy_blocks(d_pairs), reps=max(min(args.steps, 20), 5))
    nbytes = n_pairs * 2 * 2 * BLOCK * kvd * 2  # K and V, read and written
    line = {"workload": "copy-bulk llama3-8b f16: 131072 distinct (src, dst) block pairs, 1 layer",
            "copy_us": round(us, 1), "bytes": nbytes, "GBps": round(nbytes / (us * 1e-6) / 1e9, 1),
            "frac": round(nbytes / (us * 1e-6) / 1e9 / PEAK_HBM_GBPS, 4)}
    if not args.no_cpu:
        # the oracle's copy (memmove per block, one thread as the reference's
        # copy_within) over a sample of the same pairs, scaled to all of them
        from oracle import OracleKv

        n_s = 8192
        o = OracleKv(1, kvd, 2 * n_s * BLOCK, dtype="f16")
        sample = np.arange(2 * n_s, dtype=np.int32).reshape(n_s, 2)
        sec, n = _cpu_time(lambda _: o.copy_blocks(sample), 1 << 20, min(args.cpu_seconds, 5.0), at_least=2)
        per_pair = sec / n_s
        line["cpu_baseline"] = _cpu_record(
            args, per_pair * n_pairs * 1e6, "µs/launch", f"{n} passes over {n_s} block pairs, scaled to "
            f"{n_pairs}", 1, GBps=round(nbytes / (per_pair * n_pairs) / 1e9, 2))
    print(json.dumps(line), flush=True)


def bench_append_sweep(args):
    """Bulk slot-mapped append at the Llama-3-8B layer shape (kv_dim 1024, f16):
    512 sequences x 512 tokens claimed through the allocator over a permuted
    pool; the first n slots of that mapping are written for each size, in
    batch order (ltkv_write) and in ascending cell order (ltkv_cell_order +
    ltkv_write_ordered)."""
    import torch

    from langtrain_studio_amd import KvCache

    kvd, n_seqs, per_seq = 1024, 512, 512
    total = n_seqs * per_seq
    rng = np.random.default_rng(args.seed)
    n_blocks = total // BLOCK + 64
    kv = KvCache(1, kvd, n_blocks * BLOCK, dtype="f16", device=0, stream=torch.cuda.current_stream())
    kv.init_free_order(rng.permutation(n_blocks))
    sm = kv.append_batch(np.repeat(np.arange(n_seqs, dtype=np.uint32), per_seq),
                         np.tile(np.arange(per_seq, dtype=np.uint64), n_seqs))
    d_sm = torch.from_numpy(sm).cuda()
    gen = torch.Generator(device="cuda")
    gen.manual_seed(args.seed)
    k = torch.randn((total, kvd), generator=gen, device="cuda")
    v = torch.randn((total, kvd), generator=gen, device="cuda")
    rows = []
    for n in (64, 256, 1024, 4096, 16384, 65536, 262144):
        us = _time_op(lambda: kv.write_batch(0, d_sm[:n], k[:n], v[:n]), reps=20)
        nbytes = n * kvd * (4 + 4 + 2 + 2) + n * 4
        # the same rows in ascending cell order (ltkv_cell_order on the host,
        # once per claim; the order array is 4 more bytes per token)
        d_order = torch.from_numpy(kv.cell_order(sm[:n])).cuda()
        us_o = _time_op(lambda: kv.write_batch_ordered(0, d_sm[:n], k[:n], v[:n], d_order), reps=20)
        obytes = nbytes + n * 4
        rows.append({"tokens": n, "us": round(us, 2), "GBps": round(nbytes / (us * 1e-6) / 1e9, 1),
                     "frac": round(nbytes / (us * 1e-6) / 1e9 / PEAK_HBM_GBPS, 4),
                     "ordered_us": round(us_o, 2), "ordered_GBps": round(obytes / (us_o * 1e-6) / 1e9, 1),
                     "ordered_frac": round(obytes / (us_o * 1e-6) / 1e9 / PEAK_HBM_GBPS, 4)})
    print(json.dumps({"workload": "append-sweep", "shape": "kv_dim 1024 f32->f16", "rows": rows}), flush=True)


def bench_long_context(args):
    """Long-context stress at the Llama-3-8B layer shape: 32 sequences x 32768
    tokens over a fully permuted pool (worst-case scatter). Times the gather
    of every sequence to contiguous K/V and one decode-attention pass."""
    import torch

    from langtrain_studio_amd import KvCache

    B, ctx, n_heads, n_kv, hd = 32, 32768, 32, 8, 128
    kvd = n_kv * hd
    rng = np.random.default_rng(args.seed)
    n_blocks = B * ctx // BLOCK + 64
    kv = KvCache(1, kvd, n_blocks * BLOCK, dtype="f16", device=0, stream=torch.cuda.current_stream())
    if args.partition:
        kv.set_attention_partition(args.partition)
    order = rng.permutation(n_blocks)
    kv.init_free_order(order)
    seqs_all = np.repeat(np.arange(B, dtype=np.uint32), ctx)
    pos_all = np.tile(np.arange(ctx, dtype=np.uint64), B)
    sm = kv.append_batch(seqs_all, pos_all)
    gen = torch.Generator(device="cuda")
    gen.manual_seed(args.seed)
    chunk = 1 << 16
    for i in range(0, sm.size, chunk):
        kk = torch.randn((chunk, kvd), generator=gen, device="cuda")
        vv = torch.randn((chunk, kvd), generator=gen, device="cuda")
        kv.write_batch(0, torch.from_numpy(sm[i:i + chunk]).cuda(), kk, vv)
    del kk, vv
    tables = torch.from_numpy(kv.block_tables(np.arange(B, dtype=np.uint32), ctx // BLOCK)).cuda()
    lens = torch.full((B,), ctx, dtype=torch.int32, device="cuda")
    offs = torch.arange(B, dtype=torch.int64, device="cuda") * ctx
    k_out = torch.empty((B * ctx, kvd), dtype=torch.float16, device="cuda")
    v_out = torch.empty_like(k_out)
    g_us = _time_op(lambda: kv.gather(0, tables, lens, offs, k_out, v_out), reps=10)
    g_bytes = 2 * 2 * B * ctx * kvd * 2 + tables.numel() * 4
    q = torch.randn((B, n_heads * hd), generator=gen, device="cuda")
    out = torch.empty_like(q)
    a_us = _time_op(lambda: kv.decode_attention(0, q, tables, lens, n_heads, hd, out=out), reps=10)
    a_bytes = B * ctx * 2 * kvd * 2 + 2 * q.numel() * 4 + tables.numel() * 4 + B * 4
    line = {
        "workload": "long-context 32x32768 llama3-8b f16, random tables",
        "gather_us": round(g_us, 1), "gather_GBps": round(g_bytes / (g_us * 1e-6) / 1e9, 1),
        "gather_frac": round(g_bytes / (g_us * 1e-6) / 1e9 / PEAK_HBM_GBPS, 4), "gather_bytes": g_bytes,
        "attention_us": round(a_us, 1), "attention_GBps": round(a_bytes / (a_us * 1e-6) / 1e9, 1),
        "attention_frac": round(a_bytes / (a_us * 1e-6) / 1e9 / PEAK_HBM_GBPS, 4), "attention_bytes": a_bytes,
        "tokens_per_s": round(B / (a_us * 1e-6), 1),
    }
    if not args.partition:
        # The default partitions (a function of each query's own length, so
        # a query's bits do not depend on its batch) favour small batches of
        # long queries; an engine that knows it runs 32 of them can fix
        # 4096-token partitions (ltkv_set_attention_partition): 1024 items,
        # one per SIMD.
        kv.set_attention_partition(4096)
        p_us = _time_op(lambda: kv.decode_attention(0, q, tables, lens, n_heads, hd, out=out), reps=10)
        kv.set_attention_partition(0)
        line["attention_partition_4096_us"] = round(p_us, 1)
        line["attention_partition_4096_frac"] = round(a_bytes / (p_us * 1e-6) / 1e9 / PEAK_HBM_GBPS, 4)
    del k_out, v_out
    if not args.no_cpu:
        # the oracle on the same state: same allocator order and claims, pool read back
        from oracle import OracleKv

        threads = _cpu_setup(args)["threads"]
        o = OracleKv(1, kvd, n_blocks * BLOCK, dtype="f16")
        o.init_free_order(order)
        o.append_batch(seqs_all, pos_all)
        o.load_pool(0, *kv.read_pool(0))
        # gather: KvCache::rows collected (kv.rs:133-150), one sequence at a
        # time on one thread as the reference's iterator runs
        g_sec, g_n = _cpu_time(lambda i: o.rows(0, i % B, ctx), B, min(args.cpu_seconds, 10.0), at_least=2)
        q_h, tables_h, lens_h = q.cpu().numpy(), tables.cpu().numpy(), lens.cpu().numpy()
        a_sec, a_n = _cpu_time(lambda _: o.attention_tables(0, tables_h, lens_h, q_h, n_heads, hd, threads=threads),
                               3, min(args.cpu_seconds, 10.0))
        line["cpu_baseline"] = _cpu_record(
            args, a_sec * 1e6, "µs/step", f"{a_n} decode-attention passes over all 32 x 32768 tokens; gather: "
            f"{g_n} sequences' rows collected on one thread, scaled to 32", threads,
            tokens_per_s=round(B / a_sec, 1), gather_us=round(g_sec * B * 1e6, 1), gather_cores=1,
            gather_GBps=round(g_bytes / (g_sec * B) / 1e9, 2))
    print(json.dumps(line), flush=True)


def _fill_pool_random(kv, kvd, n_blocks, seed, layer=0):
    """Write N(0,1) rows into every cell of a layer's pool (device-only,
    outside timing), so blocks that arrivals inherit hold finite data."""
    import torch

    gen = torch.Generator(device="cuda")
    gen.manual_seed(seed)
    cells = np.arange(n_blocks * BLOCK, dtype=np.int32)
    chunk = 1 << 16
    for i in range(0, cells.size, chunk):
        sm = torch.from_numpy(cells[i:i + chunk]).cuda()
        k = torch.randn((sm.numel(), kvd), generator=gen, device="cuda")
        v = torch.randn((sm.numel(), kvd), generator=gen, device="cuda")
        kv.write_batch(layer, sm, k, v)
    torch.cuda.synchronize()


def bench_tinyllama(args):
    """TinyLlama-shaped layer, f32 KV (32 q heads, 4 kv heads, head_dim 64): 4
    sequences with contexts U[128,512] over a permuted 1024-block pool; one
    append of one token per sequence, then one decode step (scale 1/8)."""
    import torch

    from langtrain_studio_amd import KvCache

    rng = np.random.default_rng(args.seed)
    n_heads, n_kv, hd, B = 32, 4, 64, 4
    kvd = n_kv * hd
    kv = KvCache(1, kvd, 1024 * BLOCK, dtype="f32", device=0, stream=torch.cuda.current_stream())
    order = rng.permutation(1024)
    kv.init_free_order(order)
    ctx = rng.integers(128, 513, B)
    pre_seqs = np.repeat(np.arange(B, dtype=np.uint32), ctx)
    pre_pos = np.concatenate([np.arange(int(c), dtype=np.uint64) for c in ctx])
    sm = kv.append_batch(pre_seqs, pre_pos)
    k = torch.randn((sm.size, kvd), device="cuda")
    kv.write_batch(0, torch.from_numpy(sm).cuda(), k, k)
    seqs = np.arange(B, dtype=np.uint32)
    d_sm = torch.from_numpy(kv.append_batch(seqs, ctx.astype(np.uint64))).cuda()
    tables = torch.from_numpy(kv.block_tables(seqs)).cuda()
    lens = torch.from_numpy((ctx + 1).astype(np.int32)).cuda()
    kn = torch.randn((B, kvd), device="cuda")
    q = torch.randn((B, n_heads * hd), device="cuda")
    out = torch.empty_like(q)

    def step():
        kv.write_batch(0, d_sm, kn, kn)
        kv.decode_attention(0, q, tables, lens, n_heads, hd, scale=0.125, out=out)

    us = _time_op(step, reps=max(args.steps, 10))
    a_us = _time_op(lambda: kv.decode_attention(0, q, tables, lens, n_heads, hd, scale=0.125, out=out),
                    reps=max(args.steps, 10))
    a_bytes = int((ctx + 1).sum()) * 2 * kvd * 4 + 2 * q.numel() * 4
    line = {"workload": "tinyllama f32, 4 seqs ctx U[128,512]", "step_us": round(us, 2),
            "tokens_per_s": round(B / (us * 1e-6), 1),
            "attention_us": round(a_us, 2), "attention_bytes": a_bytes,
            "attention_frac": round(a_bytes / (a_us * 1e-6) / 1e9 / PEAK_HBM_GBPS, 4)}
    if not args.no_cpu:
        # the oracle on the same state: same allocator order and claims, pool read back
        from oracle import OracleKv

        threads = _cpu_setup(args)["threads"]
        o = OracleKv(1, kvd, 1024 * BLOCK, dtype="f32")
        o.init_free_order(order)
        o.append_batch(pre_seqs, pre_pos)
        o.load_pool(0, *kv.read_pool(0))
        sm_h, kn_h, q_h = o.append_batch(seqs, ctx.astype(np.uint64)), kn.cpu().numpy(), q.cpu().numpy()
        tables_h, lens_h = tables.cpu().numpy(), lens.cpu().numpy()

        def cpu_step(_):
            o.write_batch(0, sm_h, kn_h, kn_h)
            o.attention_tables(0, tables_h, lens_h, q_h, n_heads, hd, scale=0.125, threads=threads)

        sec, n = _cpu_time(cpu_step, 1 << 20, min(args.cpu_seconds, 5.0), at_least=10)
        line["cpu_baseline"] = _cpu_record(args, sec * 1e6, "µs/step",
                                           f"{n} steps of the same work (append of 4 rows + decode attention)",
                                           threads, tokens_per_s=round(B / sec, 1))
    print(json.dumps(line), flush=True)


def bench_prefill(args):
    """Chunked-prefill attention at the Qwen2.5-7B layer shape (28 q heads, 4
    kv heads, head_dim 128, f16): 8 sequences with contexts U[512, 8192]
    each append a 512-token chunk, and every chunk token attends to its own
    prefix (causal within the chunk). Planned attention makes each chunk one
    causal group on the matrix cores; the per-query decode kernel on the same
    4096 queries is timed beside it. Flops count 4 * q_heads * head_dim per
    (query token, visible token) pair, QK and PV, once."""
    import torch

    from langtrain_studio_amd import KvCache

    n_heads, n_kv, hd, n_seq, chunk = 28, 4, 128, 8, 512
    kvd = n_kv * hd
    rng = np.random.default_rng(args.seed)
    ctx = rng.integers(512, 8193, n_seq)
    n_blocks = int(sum(-(-int(c + chunk) // BLOCK) for c in ctx) * 1.1) + 16
    kv = KvCache(1, kvd, n_blocks * BLOCK, dtype=args.kv_dtype, device=0, stream=torch.cuda.current_stream())
    kv.init_free_order(rng.permutation(n_blocks))
    _fill_pool_random(kv, kvd, n_blocks, args.seed)
    kv.append_batch(np.repeat(np.arange(n_seq, dtype=np.uint32), ctx),
                    np.concatenate([np.arange(int(c), dtype=np.uint64) for c in ctx]))
    seqs = np.repeat(np.arange(n_seq, dtype=np.uint32), chunk)
    pos = np.concatenate([np.arange(int(c), int(c) + chunk, dtype=np.uint64) for c in ctx])
    sm = torch.from_numpy(kv.append_batch(seqs, pos)).cuda()
    kn = torch.randn((seqs.size, kvd), device="cuda")
    kv.write_batch(0, sm, kn, kn)
    lens = (pos + 1).astype(np.int64)
    q = torch.randn((seqs.size, n_heads * hd), device="cuda")
    out = torch.empty_like(q)
    stats = kv.plan_attention(seqs, lens, n_heads, hd, shared_prefix=True)
    plan_t = []
    for _ in range(5):  # host planning time of a warm plan, the device idle
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        stats = kv.plan_attention(seqs, lens, n_heads, hd, shared_prefix=True)
        plan_t.append(time.perf_counter() - t0)
    plan_us = float(np.median(plan_t)) * 1e6
    reps = max(args.steps, 10)
    p_us = _time_op(lambda: kv.planned_attention(0, q, out=out), reps=reps)
    kv.plan_attention(seqs, lens, n_heads, hd, shared_prefix=True, f16_products=True)
    p16_us = _time_op(lambda: kv.planned_attention(0, q, out=out), reps=reps)
    tables = torch.from_numpy(kv.block_tables(seqs)).cuda()
    d_lens = torch.from_numpy(lens.astype(np.int32)).cuda()
    d_us = _time_op(lambda: kv.decode_attention(0, q, tables, d_lens, n_heads, hd, out=out), reps=reps)
    flops = 4.0 * n_heads * hd * float(lens.sum())
    eb = 2 if args.kv_dtype == "f16" else 1 + 2 / 32  # bytes per cached element (q8_0: quant + scale share)
    kv_bytes = int(sum(int(c) + chunk for c in ctx) * 2 * kvd * eb)  # K and V of each context once
    print(json.dumps({
        "workload": f"prefill qwen2.5-7b {args.kv_dtype}: 8 chunks x 512 tokens, contexts U[512,8192]",
        "attention_us": round(p_us, 2), "TFLOPs": round(flops / (p_us * 1e-6) / 1e12, 1),
        "mfma_frac": round(flops / (p_us * 1e-6) / 1e12 / PEAK_F16_MFMA_TFLOPS, 4),
        "kv_bytes": kv_bytes, "flops": flops,
        "f16_products_us": round(p16_us, 2), "f16_products_TFLOPs": round(flops / (p16_us * 1e-6) / 1e12, 1),
        "plan": {k: stats[k] for k in ("groups", "grouped", "shared_blocks", "prefix_workgroups")},
        "plan_host_us": round(plan_us, 1),
        "attention_per_query_us": round(d_us, 2),
        "per_query_TFLOPs": round(flops / (d_us * 1e-6) / 1e12, 1)}), flush=True)


def bench_rope_append(args):
    """Fused RoPE + append (model.rs:414-429 in one launch) at the Qwen2.5-7B
    continuous-batching step: 4216 tokens (8 prefill chunks x 512 + 120 decode
    tokens) at positions U[0, 8704), 28 q heads / 4 kv heads / 128, NeoX pairs;
    and at the Llama-3-8B shape with 4096 tokens (interleaved pairs), into f16
    and into q8_0 cells. Bytes per token: K and V f32 read + f16 (or q8_0
    quants and scales) written, Q f32 read and written, slot and position;
    the cos/sin table reads are not counted (cache-resident)."""
    import torch

    from langtrain_studio_amd import KvCache

    rng = np.random.default_rng(args.seed)
    rows = []
    for dtype, name, n_heads, n_kv, hd, n, neox, base in (
            ("f16", "qwen2.5-7b", 28, 4, 128, 4216, True, 1e6), ("f16", "llama3-8b", 32, 8, 128, 4096, False, 5e5),
            ("q8_0", "qwen2.5-7b", 28, 4, 128, 4216, True, 1e6), ("q8_0", "llama3-8b", 32, 8, 128, 4096, False, 5e5)):
        kvd = n_kv * hd
        n_blocks = n // BLOCK + 64
        kv = KvCache(1, kvd, n_blocks * BLOCK, dtype=dtype, device=0, stream=torch.cuda.current_stream())
        kv.init_free_order(rng.permutation(n_blocks))
        kv.rope_init(base, hd, hd, neox, 8704)
        sm = torch.from_numpy(kv.append_batch(np.zeros(n, np.uint32), np.arange(n, dtype=np.uint64))).cuda()
        pos = torch.from_numpy(rng.integers(0, 8704, n).astype(np.int32)).cuda()
        k = torch.randn((n, kvd), device="cuda")
        v = torch.randn((n, kvd), device="cuda")
        q = torch.randn((n, n_heads * hd), device="cuda")
        fused = _time_op(lambda: kv.write_rope(0, sm, pos, k, v, q=q, n_heads=n_heads), reps=20)
        plain = _time_op(lambda: kv.write_batch(0, sm, k, v), reps=20)
        cell = 2 if dtype == "f16" else 1 + 2 / 32  # bytes written per K/V element (q8_0: quant + scale share)
        nbytes = int(n * (kvd * (4 + cell) * 2 + n_heads * hd * 8 + 8))
        rows.append({"shape": f"{name}: {n} tokens, {n_heads}q/{n_kv}kv x {hd}, {'neox' if neox else 'interleaved'}",
                     "dtype": dtype,
                     "fused_us": round(fused, 2), "bytes": nbytes,
                     "GBps": round(nbytes / (fused * 1e-6) / 1e9, 1),
                     "frac": round(nbytes / (fused * 1e-6) / 1e9 / PEAK_HBM_GBPS, 4),
                     "append_only_us": round(plain, 2)})
    print(json.dumps({"workload": "rope-append", "rows": rows}), flush=True)


def _unique_tokens(tables: np.ndarray, lens: np.ndarray) -> int:
    """Tokens of the distinct physical blocks a batch reads: every block once,
    with the most tokens any query reads from it (shared prefix blocks count
    once, as the unique-byte roofline of a prefix-sharing step does)."""
    lens = lens.astype(np.int64)
    nb = -(-lens // BLOCK)
    qi = np.repeat(np.arange(lens.size), nb)
    j = np.concatenate([np.arange(n) for n in nb])
    blocks = tables[qi, j]
    toks = np.minimum(BLOCK, lens[qi] - j * BLOCK)
    best = np.zeros(int(blocks.max()) + 1, np.int64)
    np.maximum.at(best, blocks, toks)
    return int(best.sum())


def bench_prefix_cow(args, timeline=None):
    """Prefix sharing at the Llama-3-8B layer shape: 256 sequences hold a
    4088-token prefix (256 blocks, the last holding 8 tokens, refcount 256);
    step 0 appends a 64-token private suffix to every sequence, which copies
    the shared partial block 255 times in every layer (the last holder writes
    in place); then 32 decode steps. The cache has 8 layers (1.2 GB of pools,
    more than the 256 MB last-level cache) and each step's attention runs on
    layers 0..7 back to back, as a decode step's layers do, so every layer's
    K/V comes from HBM. Attention bytes per step count each physical block
    once with the tokens read from it (unique bytes), from that step's lengths."""
    import torch

    from langtrain_studio_amd import KvCache

    n_heads, n_kv, hd, S, prefix, suffix, steps, L = 32, 8, 128, 256, 4088, 64, 32, 8
    kvd = n_kv * hd
    rng = np.random.default_rng(args.seed)
    per_seq = -(-(prefix + suffix + steps) // BLOCK) - prefix // BLOCK + 1
    n_blocks = int((prefix // BLOCK + 1 + S * per_seq) * 1.1)
    kv = KvCache(L, kvd, n_blocks * BLOCK, dtype=args.kv_dtype, device=0, stream=torch.cuda.current_stream())
    eb = 2 if args.kv_dtype == "f16" else 1 + 2 / 32  # bytes per cached element (q8_0: quant + scale share)
    order = rng.permutation(n_blocks)
    kv.init_free_order(order)
    for layer in range(L):
        _fill_pool_random(kv, kvd, n_blocks, args.seed + layer, layer)
    kv.append_batch(np.zeros(prefix, np.uint32), np.arange(prefix, dtype=np.uint64))
    for d in range(1, S):
        kv.share(0, d, prefix)
    # step 0: the suffix append (copy-on-write launched by the claim itself)
    seqs0 = np.repeat(np.arange(S, dtype=np.uint32), suffix)
    pos0 = np.tile(np.arange(prefix, prefix + suffix, dtype=np.uint64), S)
    shared_last = int(kv.block_table(0)[-1])
    kn = torch.randn((seqs0.size, kvd), device="cuda")
    sm0 = kv.append_batch(seqs0, pos0)  # launches the 255 copies (every layer) itself
    d_sm0 = torch.from_numpy(sm0).cuda()
    torch.cuda.synchronize()
    assert kv.cow_copies() == S - 1, kv.cow_copies()
    app_us = _time_op(lambda: kv.write_batch(0, d_sm0, kn, kn), reps=10)
    for layer in range(1, L):
        kv.write_batch(layer, d_sm0, kn, kn)
    cow_bytes = int((S - 1) * 2 * 2 * BLOCK * kvd * eb * L)
    seqs = np.arange(S, dtype=np.uint32)
    sms, lens = [], []
    for s in range(steps):
        pos = np.full(S, prefix + suffix + s, dtype=np.uint64)
        sms.append(kv.append_batch(seqs, pos))
        lens.append((pos + 1).astype(np.int32))
    tables_h = kv.block_tables(seqs)
    tables = torch.from_numpy(tables_h).cuda()
    d_sm = torch.from_numpy(np.stack(sms)).cuda()
    d_lens = torch.from_numpy(np.stack(lens)).cuda()
    q = torch.randn((steps, S, n_heads * hd), device="cuda")
    kd = torch.randn((steps, S, kvd), device="cuda")
    out = torch.empty((S, n_heads * hd), device="cuda")
    ev = [[torch.cuda.Event(enable_timing=True) for _ in range(2)] for _ in range(steps)]

    def write_step(s):
        for layer in range(L):
            kv.write_batch(layer, d_sm[s], kd[s], kd[s])

    if timeline is not None:
        # Profiling build: the stamps of step 0's planned per-query pass (the
        # decode kernel's launch after the grouped kernel), layer 0.
        kv.plan_attention(seqs, lens[0], n_heads, hd, shared_prefix=True)
        write_step(0)
        for _ in range(5):
            kv.planned_attention(0, q[0], out=out)
        timeline("prefix-cow planned step, per-query pass (256 forks of a 4088-token prefix, "
                 "llama3-8b layer, f16)")
        return

    # Per-query decode attention (every sequence reads its whole table). One
    # untimed call on the last layer first keeps the queue busy, so the timed
    # region holds device time; layer 0 was last read 8 layers (~1 GB) ago.
    for s in range(steps):
        write_step(s)
        kv.decode_attention(L - 1, q[s], tables, d_lens[s], n_heads, hd, out=out)
        ev[s][0].record()
        for layer in range(L):
            kv.decode_attention(layer, q[s], tables, d_lens[s], n_heads, hd, out=out)
        ev[s][1].record()
    torch.cuda.synchronize()
    flat_t = np.array([e[0].elapsed_time(e[1]) for e in ev]) * 1e3 / L
    # Planned attention: the step's tables are planned once on the host (the
    # shared prefix becomes one group) and uploaded before the timed region.
    plan_s = []
    for s in range(steps):
        # host planning time alone: the device idle, so the plan's upload does
        # not wait for the previous step's launches
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        stats = kv.plan_attention(seqs, lens[s], n_heads, hd, shared_prefix=True)
        plan_s.append(time.perf_counter() - t0)
        write_step(s)
        kv.planned_attention(L - 1, q[s], out=out)
        ev[s][0].record()
        for layer in range(L):
            kv.planned_attention(layer, q[s], out=out)
        ev[s][1].record()
    torch.cuda.synchronize()
    att_t = np.array([e[0].elapsed_time(e[1]) for e in ev]) * 1e3 / L
    # The same plans with the grouped products on f16-rounded Q and weights
    # (LTKV_PLAN_F16_PRODUCTS: ~3e-4 relative error instead of f32 accuracy).
    for s in range(steps):
        kv.plan_attention(seqs, lens[s], n_heads, hd, shared_prefix=True, f16_products=True)
        write_step(s)
        kv.planned_attention(L - 1, q[s], out=out)
        ev[s][0].record()
        for layer in range(L):
            kv.planned_attention(layer, q[s], out=out)
        ev[s][1].record()
    torch.cuda.synchronize()
    att16_t = np.array([e[0].elapsed_time(e[1]) for e in ev]) * 1e3 / L
    # The copy-on-write copies of step 0 again, timed alone (same pairs, all layers).
    dst = tables_h[:, prefix // BLOCK]
    pairs = np.stack([np.full(S, shared_last), dst], 1)[dst != shared_last].astype(np.int32)
    assert len(pairs) == S - 1
    d_pairs = torch.from_numpy(pairs).cuda()
    cow_us = _time_op(lambda: kv.copy_blocks(d_pairs), reps=100, warmup=10)
    row = 2 * kvd * eb  # K and V bytes of one token row
    qo = 2 * S * n_heads * hd * 4
    uniq = np.array([_unique_tokens(tables_h, l) * row + qo + (-(-l.astype(np.int64) // BLOCK)).sum() * 4 + S * 4
                     for l in lens])
    logical = np.array([l.astype(np.int64).sum() * row for l in lens])
    att_us, flat_us = float(att_t.mean()), float(flat_t.mean())
    frac = float(np.mean(uniq / (att_t * 1e-6) / 1e9 / PEAK_HBM_GBPS))
    line = {
        "workload": f"prefix-cow llama3-8b {args.kv_dtype}: 256 seqs x 4088 shared + 64 private, 32 decode steps, "
                    f"{L} layers",
        "cow_copies": S - 1, "cow_layers": L, "cow_us": round(cow_us, 2), "cow_bytes": cow_bytes,
        "cow_GBps": round(cow_bytes / (cow_us * 1e-6) / 1e9, 1),
        "cow_frac": round(cow_bytes / (cow_us * 1e-6) / 1e9 / PEAK_HBM_GBPS, 4),
        "suffix_append_us": round(app_us, 2), "attention_us": round(att_us, 2),
        "attention_unique_bytes": round(float(uniq.mean())),
        "attention_logical_bytes": round(float(logical.mean())),
        "attention_frac_unique": round(frac, 4),
        "attention_logical_GBps": round(float(logical.mean()) / (att_us * 1e-6) / 1e9, 1),
        "tokens_per_s": round(S / (att_us * 1e-6), 1),
        "plan": {k: stats[k] for k in ("groups", "grouped", "shared_blocks", "prefix_workgroups")},
        "plan_host_us": round(float(np.mean(plan_s)) * 1e6, 1),
        "attention_f16_products_us": round(float(att16_t.mean()), 2),
        "attention_f16_products_frac_unique": round(float(np.mean(uniq / (att16_t * 1e-6) / 1e9 / PEAK_HBM_GBPS)), 4),
        "attention_per_query_us": round(flat_us, 2),
        "attention_per_query_frac_unique": round(float(np.mean(uniq / (flat_t * 1e-6) / 1e9 / PEAK_HBM_GBPS)), 4)}
    if not args.no_cpu:
        # the oracle on the same history: copy-on-write as the reference does
        # it (a memmove per layer inside append, kv.rs:99-110), then each
        # step's attention per (query, kv head) over the whole table
        from oracle import OracleKv

        threads = _cpu_setup(args)["threads"]
        o = OracleKv(L, kvd, n_blocks * BLOCK, dtype=args.kv_dtype)
        o.init_free_order(order)
        o.append_batch(np.zeros(prefix, np.uint32), np.arange(prefix, dtype=np.uint64))
        for d in range(1, S):
            o.share(0, d, prefix)
        o.load_pool(0, *kv.read_pool(0))
        if args.kv_dtype == "q8_0":
            o.load_scales(0, *(x.transpose(0, 2, 1) for x in kv.read_scales(0)))
        t0 = time.perf_counter()
        o.append_batch(seqs, np.full(S, prefix, np.uint64))  # 255 copies x 8 layers
        cow_cpu = (time.perf_counter() - t0) * 1e6
        assert o.cow_copies() == S - 1
        q_h = q.cpu().numpy()
        sec, n = _cpu_time(lambda s: o.attention_tables(0, tables_h, lens[s], q_h[s], n_heads, hd, threads=threads),
                           steps, min(args.cpu_seconds, 10.0), at_least=1)
        line["cpu_baseline"] = _cpu_record(
            args, sec * 1e6, "µs/step", f"{n} decode steps' attention (256 queries, one layer) on the same pool "
            "and tables; copy-on-write: the 256 first suffix appends (255 copies x 8 layers)", threads,
            tokens_per_s=round(S / sec, 1), cow_us=round(cow_cpu, 1), cow_cores=1)
    print(json.dumps(line), flush=True)


def bench_mixed(args):
    """Continuous batching at the Qwen2.5-7B layer shape (28 q heads, 4 kv
    heads, head_dim 128, f16): every step appends 8 prefill chunks of 512
    tokens and one token for each of 120 decode sequences (contexts U[512,
    8192]), then runs decode attention for the 120. Decode sequences finish
    with probability 2% per step (their blocks are freed, LIFO) and arrivals
    take their slot from the fragmented pool; prefill streams restart when
    their prompt is done. The allocator runs ahead of the timed device loop."""
    import torch

    from langtrain_studio_amd import KvCache

    n_heads, n_kv, hd, n_dec, n_pre, chunk, steps = 28, 4, 128, 120, 8, 512, max(args.steps, 1)
    kvd = n_kv * hd
    rng = np.random.default_rng(args.seed)
    n_blocks = int((n_dec + n_pre) * 8192 // BLOCK * 1.1) + (n_dec + n_pre) * (steps // BLOCK + 2)
    kv = KvCache(1, kvd, n_blocks * BLOCK, dtype="f16", device=0, stream=torch.cuda.current_stream())
    if args.partition:
        kv.set_attention_partition(args.partition)
    kv.init_free_order(rng.permutation(n_blocks))
    _fill_pool_random(kv, kvd, n_blocks, args.seed)
    next_id = [0]

    def new_seq(ctx):
        sid = next_id[0]
        next_id[0] += 1
        if ctx:
            kv.append_batch(np.full(ctx, sid, np.uint32), np.arange(ctx, dtype=np.uint64))
        return sid

    dec = [new_seq(int(rng.integers(512, 8193))) for _ in range(n_dec)]
    pre = [(new_seq(0), int(rng.integers(512, 8193))) for _ in range(n_pre)]
    plan_sm, plan_tables, plan_lens = [], [], []
    stride = (8192 + steps + chunk) // BLOCK + 2
    for s in range(steps):
        seqs, pos = [], []
        for i, (sid, target) in enumerate(pre):
            start = kv.len(sid)
            n = min(chunk, target - start)
            seqs += [sid] * n
            pos += list(range(start, start + n))
        for sid in dec:
            seqs.append(sid)
            pos.append(kv.len(sid))
        sm = kv.append_batch(np.array(seqs, np.uint32), np.array(pos, np.uint64))
        plan_sm.append(np.pad(sm, (0, n_pre * chunk + n_dec - sm.size), constant_values=-1))
        plan_tables.append(kv.block_tables(np.array(dec, np.uint32), stride))
        plan_lens.append(np.array([kv.len(sid) for sid in dec], np.int32))
        for i, (sid, target) in enumerate(pre):  # prompt done: the stream restarts
            if kv.len(sid) >= target:
                kv.truncate(sid, 0)
                pre[i] = (new_seq(0), int(rng.integers(512, 8193)))
        for i, sid in enumerate(dec):  # 2% finish per step; an arrival takes the slot
            if rng.random() < 0.02:
                kv.truncate(sid, 0)
                dec[i] = new_seq(int(rng.integers(512, 8193)))
    d_sm = torch.from_numpy(np.stack(plan_sm)).cuda()
    d_tables = torch.from_numpy(np.stack(plan_tables)).cuda()
    d_lens = torch.from_numpy(np.stack(plan_lens)).cuda()
    rows = n_pre * chunk + n_dec
    kn = torch.randn((rows, kvd), device="cuda")
    q = torch.randn((n_dec, n_heads * hd), device="cuda")
    out = torch.empty_like(q)
    ev = [[torch.cuda.Event(enable_timing=True) for _ in range(3)] for _ in range(steps)]
    torch.cuda.synchronize()
    for s in range(steps):
        ev[s][0].record()
        kv.write_batch(0, d_sm[s], kn, kn)
        ev[s][1].record()
        kv.decode_attention(0, q, d_tables[s], d_lens[s], n_heads, hd, out=out)
        ev[s][2].record()
    torch.cuda.synchronize()
    app_us = float(np.mean([e[0].elapsed_time(e[1]) for e in ev]) * 1e3)
    att_us = float(np.mean([e[1].elapsed_time(e[2]) for e in ev]) * 1e3)
    app_bytes = float(np.mean([(p >= 0).sum() for p in plan_sm])) * (kvd * 12 + 4)
    att_bytes = float(np.mean([l.astype(np.int64).sum() for l in plan_lens])) * 2 * kvd * 2 + 2 * q.numel() * 4

    # One more step at the final state with every token of the batch: the
    # fused RoPE append of all 4216 tokens, then one planned attention over
    # all of them (each prefill chunk a causal group on the matrix cores, the
    # decode tokens per query), timed 4 times back to back after a warm call.
    seqs, pos = [], []
    for sid, target in pre:
        start = kv.len(sid)
        seqs += [sid] * chunk
        pos += list(range(start, start + chunk))
    for sid in dec:
        seqs.append(sid)
        pos.append(kv.len(sid))
    kv.rope_init(1e6, hd, hd, True, 8192 + chunk + steps + 1)
    sm = torch.from_numpy(kv.append_batch(np.array(seqs, np.uint32), np.array(pos, np.uint64))).cuda()
    d_pos = torch.from_numpy(np.array(pos, np.int32)).cuda()
    qa = torch.randn((len(seqs), n_heads * hd), device="cuda")
    out_all = torch.empty_like(qa)
    rope_us = _time_op(lambda: kv.write_rope(0, sm, d_pos, kn, kn, q=qa, n_heads=n_heads), reps=10)
    stats = kv.plan_attention(np.array(seqs, np.uint32), np.array(pos, np.int64) + 1, n_heads, hd)
    kv.planned_attention(0, qa, out=out_all)
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(4):
        kv.planned_attention(0, qa, out=out_all)
    e1.record()
    torch.cuda.synchronize()
    all_us = e0.elapsed_time(e1) * 1e3 / 4
    line = {
        "workload": "mixed qwen2.5-7b f16: 8x512 prefill append + 120 decode, 2% churn, "
                    f"{steps} steps", "append_us": round(app_us, 2),
        "append_GBps": round(app_bytes / (app_us * 1e-6) / 1e9, 1),
        "attention_us": round(att_us, 2), "attention_bytes": round(att_bytes),
        "attention_frac": round(att_bytes / (att_us * 1e-6) / 1e9 / PEAK_HBM_GBPS, 4),
        "step_us": round(app_us + att_us, 2),
        "decode_tokens_per_s": round(n_dec / ((app_us + att_us) * 1e-6), 1),
        "full_step": {"rope_append_us": round(rope_us, 2),
                      "attention_all_tokens_us": round(all_us, 2),
                      "plan": {k: stats[k] for k in ("groups", "grouped", "prefix_workgroups")}}}
    if not args.no_cpu:
        # the oracle doing each timed step's work: the append of every batch
        # row (f32 -> f16 writes) and the 120 decode queries' attention, on
        # the pool read back from the device
        from oracle import OracleKv

        threads = _cpu_setup(args)["threads"]
        o = OracleKv(1, kvd, n_blocks * BLOCK, dtype="f16")
        o.load_pool(0, *kv.read_pool(0))
        kn_h, q_h = kn.cpu().numpy(), q.cpu().numpy()
        sm_h, tables_h, lens_h = np.stack(plan_sm), np.stack(plan_tables), np.stack(plan_lens)

        def cpu_step(s):
            o.write_batch(0, sm_h[s], kn_h, kn_h)
            o.attention_tables(0, tables_h[s], lens_h[s], q_h, n_heads, hd, threads=threads)

        sec, n = _cpu_time(cpu_step, steps, min(args.cpu_seconds, 10.0), at_least=2)
        line["cpu_baseline"] = _cpu_record(
            args, sec * 1e6, "µs/step", f"{n} steps of the same work (append of the step's "
            f"{rows} rows + decode attention of the 120 decode queries)", threads,
            decode_tokens_per_s=round(n_dec / sec, 1))
    print(json.dumps(line), flush=True)


def bench_descriptor(args, n_dec=120, ctx=(512, 8193), n_pre=8):
    """The step descriptor two ways, on the continuous-batching step of the
    Qwen2.5-7B layer (120 decode sequences, contexts U[512, 8192], 2% finish
    per step and arrivals take their slot, plus 8 prefill streams of 512-token
    chunks). Per step the host claims the cells, then either
      tables: builds every decode query's full block table and the slot
              mapping on the host and uploads both (the engine-side path of
              ltkv_decode_attention), or
      resident: uploads the table entries that changed (ltkv_sync_tables),
              the tokens' rows and positions, derives the slot mapping on
              the device (ltkv_slot_mapping) and attends by row
              (ltkv_decode_attention_rows).
    A third mode, resident-slots, also derives the slot mapping on the
    device from the tokens' rows and positions (what an engine that keeps
    positions on the device for RoPE would upload) instead of uploading the
    host's. All run the same appends and attention; timed per step on the
    host clock (claim + descriptor + launches + stream synchronisation), and
    the block tables' host-to-device bytes are counted. descriptor-long runs
    the decode part alone at 256 sequences x U[8192, 16384] tokens, where a
    step's full tables are 1 MB."""
    import torch

    from langtrain_studio_amd import KvCache

    n_heads, n_kv, hd, chunk = 28, 4, 128, 512
    steps = max(args.steps, 1)
    kvd = n_kv * hd
    dev = torch.device("cuda", 0)
    stride = (ctx[1] + steps + chunk) // BLOCK + 2
    n_blocks = int((n_dec + n_pre) * ctx[1] // BLOCK * 1.1) + (n_dec + n_pre) * (steps // BLOCK + 2)
    results = {}
    for mode in ("tables", "resident", "resident-slots"):
        rng = np.random.default_rng(args.seed)
        kv = KvCache(1, kvd, n_blocks * BLOCK, dtype="f16", device=0, stream=torch.cuda.current_stream())
        kv.init_free_order(rng.permutation(n_blocks))
        _fill_pool_random(kv, kvd, n_blocks, args.seed)
        next_id = [0]

        def new_seq(ctx):
            sid = next_id[0]
            next_id[0] += 1
            if ctx:
                kv.append_batch(np.full(ctx, sid, np.uint32), np.arange(ctx, dtype=np.uint64))
            return sid

        dec = [new_seq(int(rng.integers(*ctx))) for _ in range(n_dec)]
        pre = [(new_seq(0), int(rng.integers(*ctx))) for _ in range(n_pre)]
        kn = torch.randn((n_pre * chunk + n_dec, kvd), device=dev)
        q = torch.randn((n_dec, n_heads * hd), device=dev)
        out = torch.empty_like(q)
        h_tab = torch.empty((n_dec, stride), dtype=torch.int32).pin_memory()
        d_tab = torch.empty((n_dec, stride), dtype=torch.int32, device=dev)
        if mode != "tables":
            kv.sync_tables()
        torch.cuda.synchronize()
        up0 = 0
        wall, table_bytes = [], 0
        d_dec_rows = torch.empty((n_dec,), dtype=torch.int32, device=dev)
        h_dec_rows = torch.empty((n_dec,), dtype=torch.int32).pin_memory()
        rows_stale = True
        for s in range(steps + 3):
            t0 = time.perf_counter()
            seqs, pos, pre_counts = [], [], []
            for sid, target in pre:
                start = kv.len(sid)
                n = min(chunk, target - start)
                seqs += [sid] * n
                pos += list(range(start, start + n))
                pre_counts.append(n)
            for sid in dec:
                seqs.append(sid)
                pos.append(kv.len(sid))
            seqs_a = np.array(seqs, np.uint32)
            pos_a = np.array(pos, np.uint64)
            sm = kv.append_batch(seqs_a, pos_a)
            lens = torch.from_numpy(np.array([kv.len(sid) for sid in dec], np.int32)).to(dev, non_blocking=True)
            n_tok = len(seqs)
            if mode == "tables":
                d_sm = torch.from_numpy(sm).to(dev, non_blocking=True)
                h_tab.numpy()[:] = kv.block_tables(np.array(dec, np.uint32), stride)
                d_tab.copy_(h_tab, non_blocking=True)
                kv.write_batch(0, d_sm, kn[:n_tok], kn[:n_tok])
                kv.decode_attention(0, q, d_tab, lens, n_heads, hd, out=out)
                if s >= 3:
                    table_bytes += d_tab.numel() * 4
            elif mode == "resident":
                d_sm = torch.from_numpy(sm).to(dev, non_blocking=True)
                if rows_stale:  # a decode sequence arrived: refresh the rows the step reads
                    h_dec_rows.numpy()[:] = kv.seq_rows(np.array(dec, np.uint32))
                    d_dec_rows.copy_(h_dec_rows, non_blocking=True)  # pinned, as the tables' upload
                    rows_stale = False
                kv.write_batch(0, d_sm, kn[:n_tok], kn[:n_tok])
                kv.decode_attention_rows(0, q, d_dec_rows, lens, n_heads, hd, out=out)
            else:
                # one row lookup per sequence, expanded to its tokens
                srows = kv.seq_rows(np.array([sid for sid, _ in pre] + dec, np.uint32))
                tok_rows = np.concatenate([np.repeat(srows[:n_pre], pre_counts), srows[n_pre:]])
                d_rows = torch.from_numpy(tok_rows).to(dev, non_blocking=True)
                d_pos = torch.from_numpy(pos_a.astype(np.int64)).to(dev, non_blocking=True)
                d_sm = kv.slot_mapping(d_rows, d_pos)
                kv.write_batch(0, d_sm, kn[:n_tok], kn[:n_tok])
                kv.decode_attention_rows(0, q, d_rows[n_tok - n_dec:], lens, n_heads, hd, out=out)
            if mode != "tables" and s == 2:
                torch.cuda.synchronize()
                up0 = kv.table_uploads()
            torch.cuda.synchronize()
            if s >= 3:
                wall.append(time.perf_counter() - t0)
            for i, (sid, target) in enumerate(pre):
                if kv.len(sid) >= target:
                    kv.truncate(sid, 0)
                    pre[i] = (new_seq(0), int(rng.integers(*ctx)))
            for i, sid in enumerate(dec):
                if rng.random() < 0.02:
                    kv.truncate(sid, 0)
                    dec[i] = new_seq(int(rng.integers(*ctx)))
                    rows_stale = True
        if mode != "tables":
            kv.sync_tables()
            torch.cuda.synchronize()
            table_bytes = (kv.table_uploads() - up0) * 12
        results[mode] = {"step_wall_us": round(float(np.mean(wall)) * 1e6, 1),
                         "step_wall_us_p50": round(float(np.median(wall)) * 1e6, 1),
                         "table_h2d_bytes_per_step": round(table_bytes / steps)}
        del kv
    what = (f"{n_pre}x512 prefill append + {n_dec} decode ctx U[{ctx[0]},{ctx[1] - 1}]" if n_pre
            else f"{n_dec} decode ctx U[{ctx[0]},{ctx[1] - 1}]")
    print(json.dumps({
        "workload": f"descriptor qwen2.5-7b f16: {what}, 2% churn, {steps} steps",
        "tables": results["tables"], "resident": results["resident"],
        "resident_slots": results["resident-slots"],
        "h2d_ratio": round(results["tables"]["table_h2d_bytes_per_step"]
                           / max(results["resident"]["table_h2d_bytes_per_step"], 1), 1)}), flush=True)


def _time_decode(w: Llama3Decode, steps: int, warmup: int):
    """Times `steps` decode steps (append then attention) with HIP events on
    the stream both run on: (µs per step, attention µs, append µs, wall s)."""
    import torch

    for s in range(warmup):  # rewrites the same cells with the same data: state unchanged
        w.append(s)
        w.attend(s)
    torch.cuda.synchronize()

    ev = [[torch.cuda.Event(enable_timing=True) for _ in range(3)] for _ in range(steps)]
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for s in range(steps):
        ev[s][0].record()
        w.append(s)
        ev[s][1].record()
        w.attend(s)
        ev[s][2].record()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    total_ms = ev[0][0].elapsed_time(ev[-1][2])
    app_ms = np.array([e[0].elapsed_time(e[1]) for e in ev])
    att_ms = np.array([e[1].elapsed_time(e[2]) for e in ev])
    return total_ms * 1e3 / steps, float(att_ms.mean() * 1e3), float(app_ms.mean() * 1e3), wall


def _time_decode_fused(w: Llama3Decode, steps: int, warmup: int) -> float:
    """The same steps with the append fused into the attention launch
    (ltkv_append_decode_attention): µs per step, HIP events."""
    import torch

    def step(s):
        w.kv.append_decode_attention(0, w.d_sm[s], w.d_k[s], w.d_v[s], w.d_q[s], w.d_tables, w.d_lens[s],
                                     w.n_heads, w.head_dim, out=w.d_out)

    for s in range(warmup):
        step(s)
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for s in range(steps):
        step(s)
    e1.record()
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) * 1e3 / steps


def _time_decode_graph(w: Llama3Decode, steps: int) -> float:
    """The same steps, each captured once as a HIP graph (append + attention
    with its merge) and replayed back to back: µs per step, HIP events around
    the replays. Graph launches drop the per-kernel launch gaps an engine
    that captures its decode loop would not pay."""
    import torch

    graphs = []
    for s in range(steps):
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            w.kv.set_stream(torch.cuda.current_stream())  # the capture stream
            w.append(s)
            w.attend(s)
        graphs.append(g)
    w.kv.set_stream(torch.cuda.current_stream())
    for g in graphs[:3]:
        g.replay()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for g in graphs:
        g.replay()
    e1.record()
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) * 1e3 / steps


def _use_timeline_library():
    """Points the binding at the profiling build (libltkv_timeline.so: the
    same kernels with per-wave phase stamps) before anything loads the
    product library; returns the stamp reader."""
    import ctypes

    from langtrain_studio_amd import _lib
    from langtrain_studio_amd.build import TIMELINE_LIB

    if _lib._lib is not None:
        raise RuntimeError("the product library is already loaded")
    if not os.path.exists(TIMELINE_LIB):
        print(json.dumps({"error": f"{TIMELINE_LIB} is missing: python -m langtrain_studio_amd.build"}))
        sys.exit(1)
    _lib.LIB_PATH = TIMELINE_LIB
    lib = _lib.load()
    lib.ltkv_timeline_read.argtypes = [ctypes.c_void_p, ctypes.c_size_t]
    lib.ltkv_timeline_read.restype = ctypes.c_int

    def read() -> np.ndarray:
        buf = np.zeros(65536 * 8, dtype=np.uint64)
        if lib.ltkv_timeline_read(buf.ctypes.data, buf.size) != 0:
            raise RuntimeError("ltkv_timeline_read failed")
        return buf.reshape(-1, 8)

    return read


def _timeline_stats(t: np.ndarray) -> dict:
    """Per-wave phase times of one decode-kernel launch, in µs from the first
    wave's entry (s_memrealtime runs at 100 MHz)."""
    t = t[t[:, 0] > 0].astype(np.int64)
    t0 = int(t[:, 0].min())
    names = ["entry", "item_found", "first_loads_issued", "first_tile_computed", "tile_loop_done",
             "result_written"]
    phases = {}
    for i, name in enumerate(names):
        v = (t[:, i][t[:, i] > 0] - t0) / 100.0
        phases[name] = {q: round(float(np.percentile(v, p)), 2) for q, p in
                        (("p10", 10), ("p50", 50), ("p90", 90), ("max", 100))}
    streaming = (t[:, 2] > 0) & (t[:, 6] > 0)
    s0, s1 = (t[streaming, 3] - t0) / 100.0, (t[streaming, 4] - t0) / 100.0
    span = float((t[:, 5].max() - t0) / 100.0)
    live = {f"{x:.0f}": int(((s0 <= x) & (s1 > x)).sum()) for x in np.arange(0.0, span + 10.0, 10.0)}
    tiles = t[streaming, 6]
    rate = tiles / np.maximum((t[streaming, 4] - t[streaming, 2]) / 100.0, 1e-3)
    return {"waves": int(len(t)), "span_us": round(span, 2), "phases_us": phases,
            "streaming_waves_at_us": live, "tiles_per_wave": {"min": int(tiles.min()),
                                                                "mean": round(float(tiles.mean()), 1),
                                                                "max": int(tiles.max())},
            "tiles_per_us_per_wave": round(float(rate.mean()), 3)}


def bench_decode_timeline(args):
    """Per-wave timeline of the headline decode launch (unfused attention,
    64 queries x U[2048, 4096]) from the profiling build: when each wave found
    its item, issued its first loads, computed its first tile and finished,
    and how many waves stream at each 10 µs. One line per launch of the last
    `--steps` steps (at most 5), then the same launch on a q8_0 pool, one at
    the Qwen2.5-7B shape and the prefix-cow planned step's per-query pass."""
    import torch

    read = _use_timeline_library()
    steps = max(1, min(args.steps, 5))
    w = Llama3Decode(steps, args.seed, args.partition)
    for s in range(steps):
        w.append(s)
        w.attend(s)
    torch.cuda.synchronize()
    read()
    # Each reading takes the last of five back-to-back launches (the stamps
    # of a launch overwrite the previous one's), so the GPU is in its running
    # state rather than just out of the synchronisation of the reading.
    for s in range(steps):
        for _ in range(5):
            w.attend(s)
        print(json.dumps({"workload": "decode-timeline llama3-8b-layer decode, 64 seqs ctx U[2048,4096], f16, "
                                      "unfused attention launch", "step": s, **_timeline_stats(read())}),
              flush=True)
    del w
    torch.cuda.synchronize()
    # the same launch on a q8_0 pool (half partitions: two waves per SIMD)
    w = Llama3Decode(1, args.seed, args.partition, dtype="q8_0")
    w.append(0)
    w.attend(0)
    torch.cuda.synchronize()
    read()
    for _ in range(5):
        w.attend(0)
    print(json.dumps({"workload": "decode-timeline llama3-8b-layer decode, 64 seqs ctx U[2048,4096], q8_0, "
                                  "unfused attention launch", **_timeline_stats(read())}), flush=True)
    del w
    torch.cuda.synchronize()
    _timeline_qwen_decode(read, args.seed)

    def emit(what):
        print(json.dumps({"workload": "decode-timeline " + what, **_timeline_stats(read())}), flush=True)

    bench_prefix_cow(args, timeline=emit)


def _timeline_qwen_decode(read, seed):
    """Per-wave timeline of one decode launch at the Qwen2.5-7B shape (28 q
    heads, 4 kv heads, head_dim 128, f16: one kv head a wave, two waves per
    SIMD), 120 queries of contexts U[512, 8192] over a permuted pool: about
    2500 items on 2048 wave slots, so waves share SIMDs and some start when
    others end. Also reports the waves started in the launch's first 50 us
    (two per SIMD) by half: the first 1024 of the grid against the rest."""
    import torch

    from langtrain_studio_amd import KvCache

    n_heads, n_kv, hd, n_q = 28, 4, 128, 120
    kvd = n_kv * hd
    rng = np.random.default_rng(seed)
    n_blocks = n_q * 8192 // BLOCK + 64
    kv = KvCache(1, kvd, n_blocks * BLOCK, dtype="f16", device=0, stream=torch.cuda.current_stream())
    kv.init_free_order(rng.permutation(n_blocks))
    _fill_pool_random(kv, kvd, n_blocks, seed)
    lens = rng.integers(512, 8193, size=n_q)
    for i, n in enumerate(lens):
        kv.append_batch(np.full(int(n), i, np.uint32), np.arange(int(n), dtype=np.uint64))
    tables = torch.from_numpy(kv.block_tables(np.arange(n_q, dtype=np.uint32), 8192 // BLOCK)).cuda()
    d_lens = torch.from_numpy(lens.astype(np.int32)).cuda()
    q = torch.randn((n_q, n_heads * hd), device="cuda")
    out = torch.empty_like(q)
    for _ in range(3):
        kv.decode_attention(0, q, tables, d_lens, n_heads, hd, out=out)
    torch.cuda.synchronize()
    read()
    for _ in range(5):
        kv.decode_attention(0, q, tables, d_lens, n_heads, hd, out=out)
    t = read()
    stats = _timeline_stats(t)
    t = t[t[:, 0] > 0].astype(np.int64)
    t0 = int(t[:, 0].min())
    early = (t[:, 0] - t0) < 5000  # entered in the first 50 us
    halves = {}
    for name, sel in (("grid_waves_0_1023", early & (np.arange(len(t)) < 1024)),
                      ("grid_waves_1024_up", early & (np.arange(len(t)) >= 1024))):
        if sel.any():
            halves[name] = {"waves": int(sel.sum()),
                            "first_loads_issued_p50_us": round(float(np.median(t[sel, 2] - t0)) / 100.0, 2),
                            "result_written_p50_us": round(float(np.median(t[sel, 5] - t0)) / 100.0, 2)}
    print(json.dumps({"workload": "decode-timeline qwen2.5-7b-layer decode, 120 seqs ctx U[512,8192], f16, "
                                  "unfused attention launch", **stats, "first_round_by_grid_half": halves}),
          flush=True)
    del kv
    torch.cuda.synchronize()


def bench_decode_shapes(args):
    """How much the headline launch's uneven items cost: the same 64-query
    decode attention (unfused, HIP events over `--steps` launches) with every
    context equal (2048 / 3072 / 4096 tokens; 3072 is the mean of the
    headline's U[2048, 4096]) and, on the headline's contexts, with fixed
    partitions of 256-1024 tokens (ltkv_set_attention_partition) against the
    per-query default."""
    import torch

    reps = max(10, args.steps)
    out = {"workload": "decode-shapes llama3-8b-layer decode attention, 64 seqs, f16"}

    def timed(w):
        for _ in range(5):
            w.attend(0)
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(reps):
            w.attend(0)
        e1.record()
        torch.cuda.synchronize()
        us = e0.elapsed_time(e1) * 1e3 / reps
        return {"us": round(us, 2), "frac": round(w.attention_bytes(0) / (us * 1e-6) / 1e9 / PEAK_HBM_GBPS, 4)}

    w = Llama3Decode(1, args.seed, 0)
    out["random_U2048_4096"] = {"default": timed(w)}
    for p in (256, 512, 768, 1024):
        w.kv.set_attention_partition(p)
        out["random_U2048_4096"][f"partition_{p}"] = timed(w)
    del w
    for n in (2048, 3072, 4096):
        w = Llama3Decode(1, args.seed, 0, ctx=np.full(64, n))
        out[f"equal_{n}"] = timed(w)
        del w
    print(json.dumps(out), flush=True)


def bench_decode_q8(args):
    """The Llama-3-8B decode step on a q8_0 KV cache (int8 quants plus one f16
    scale per 32 elements: 1.06 bytes per element instead of 2)."""
    steps, warmup = args.steps, args.warmup
    w = Llama3Decode(max(steps, warmup, 1), args.seed, args.partition, dtype="q8_0")
    us_step, att_us, app_us, wall = _time_decode(w, steps, warmup)
    att_bytes = float(np.mean([w.attention_bytes(s) for s in range(steps)]))
    att_gbps = att_bytes / (att_us * 1e-6) / 1e9
    app_gbps = w.append_bytes() / (app_us * 1e-6) / 1e9
    line = {
        "workload": "decode-q8 llama3-8b-layer: 32q/8kv heads, head_dim 128, q8_0 KV, 64 seqs ctx "
                    "U[2048,4096], 1 append + 1 decode attention per step",
        "steps": steps, "step_us": round(us_step, 2),
        "attention_us": round(att_us, 2), "attention_bytes": round(att_bytes),
        "attention_GBps": round(att_gbps, 1), "attention_frac": round(att_gbps / PEAK_HBM_GBPS, 4),
        "append_us": round(app_us, 2), "append_GBps": round(app_gbps, 1),
        "append_frac": round(app_gbps / PEAK_HBM_GBPS, 4), "wall_s": round(wall, 3),
    }
    if not args.no_cpu:
        threads = _cpu_setup(args)["threads"]
        cpu_us, n = cpu_baseline(w, threads, min(args.cpu_seconds, 10.0))
        line["cpu_baseline"] = _cpu_record(
            args, cpu_us, "µs/step", f"{n} decode steps of the same workload on the oracle's q8_0 mode", threads,
            tokens_per_s=round(w.batch / (cpu_us * 1e-6), 1))
    print(json.dumps(line), flush=True)


def main():
    args = _args()
    if args.gpus != 1:
        print(json.dumps({"error": "ltkv's bench runs on exactly one GPU; --gpus must be 1 "
                          "(the path shards by sequence across GPUs with no exchange)"}))
        sys.exit(2)
    import torch

    if not torch.cuda.is_available():
        print(json.dumps({"error": "no HIP device visible"}))
        sys.exit(1)
    extra = {"copy": bench_copy, "copy-bulk": bench_copy_bulk, "append-sweep": bench_append_sweep, "long-context": bench_long_context,
             "tinyllama": bench_tinyllama, "prefix-cow": bench_prefix_cow, "mixed": bench_mixed,
             "prefill": bench_prefill, "rope-append": bench_rope_append, "decode-q8": bench_decode_q8,
             "descriptor": bench_descriptor, "decode-timeline": bench_decode_timeline,
             "decode-shapes": bench_decode_shapes,
             "descriptor-long": lambda a: bench_descriptor(a, n_dec=256, ctx=(8192, 16385), n_pre=0)}
    if args.workload in extra:
        extra[args.workload](args)
        return
    steps, warmup = args.steps, args.warmup
    w = Llama3Decode(max(steps, warmup, 1), args.seed, args.partition)
    us_step, att_us, app_us, wall = _time_decode(w, steps, warmup)
    graph_us = _time_decode_graph(w, steps)
    fused_us = _time_decode_fused(w, steps, warmup)
    # The same steps on the vector-ALU kernels (LTKV_ENGINE_VALU: no matrix
    # cores), the design the matrix-core kernel is measured against.
    w.kv.set_attention_engine("valu")
    _, valu_att_us, _, _ = _time_decode(w, steps, warmup)
    w.kv.set_attention_engine("auto")
    att_bytes = float(np.mean([w.attention_bytes(s) for s in range(steps)]))
    att_gbps = att_bytes / (att_us * 1e-6) / 1e9
    app_gbps = w.append_bytes() / (app_us * 1e-6) / 1e9
    roofline_us = att_bytes / (PEAK_HBM_GBPS * 1e9) * 1e6

    cpu = cpu1 = None
    if not args.no_cpu:
        threads = _cpu_setup(args)["threads"]
        cpu_us, n = cpu_baseline(w, threads, args.cpu_seconds)
        cpu = _cpu_record(args, cpu_us, "µs/step",
                          f"{n} decode steps of the same workload (64 seqs, append+write+attention, same cache "
                          f"state), oracle C++ restatement, {threads} threads", threads,
                          tokens_per_s=round(w.batch / (cpu_us * 1e-6), 1))
        cpu1_us, n1 = cpu_baseline(w, 1, min(args.cpu_seconds, 5.0))
        cpu1 = {"value": round(cpu1_us, 1), "unit": "µs/step", "cores": 1, "kind": "port",
                "sample": f"{n1} decode steps, same work, one thread",
                "tokens_per_s": round(w.batch / (cpu1_us * 1e-6), 1)}

    out = {
        "metric": METRIC,
        "value": round(fused_us, 2),
        "unit": "µs/step",
        "n_gpus": 1,
        "steps": steps,
        "warmup": warmup,
        "ms_per_step": round(fused_us / 1e3, 5),
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f16",
        "data": "synthetic (seeded N(0,1) Q/K/V, permuted block pool)",
        "config": {"workload": "llama3-8b-layer decode: 32q/8kv heads, head_dim 128, f16 KV, block 16, "
                               "64 seqs ctx U[2048,4096], 1 append + 1 decode attention per step, "
                               "fused into one launch (ltkv_append_decode_attention)",
                   "global_batch": 64, "seq_len": "2048-4096", "parallelism": "none (1 GPU)"},
        "tokens_per_s": round(w.batch / (fused_us * 1e-6), 1),
        "attention_us": round(att_us, 2),
        "attention_roofline_us": round(roofline_us, 2),
        "append_us": round(app_us, 2),
        "append_GBps": round(app_gbps, 1),
        "append_frac": round(app_gbps / PEAK_HBM_GBPS, 4),
        "unfused_step_us": round(us_step, 2),
        "graph_step_us": round(graph_us, 2),
        "attention_valu_us": round(valu_att_us, 2),
        "attention_valu_frac": round(att_bytes / (valu_att_us * 1e-6) / 1e9 / PEAK_HBM_GBPS, 4),
        "roofline": {"bound": "hbm", "achieved": round(att_gbps, 1), "peak": PEAK_HBM_GBPS, "unit": "GB/s",
                     "frac": round(att_gbps / PEAK_HBM_GBPS, 4), "traffic": _profiled_traffic(),
                     "traffic_source": TRAFFIC_PROFILE,
                     "kernel": "attn_mfma_kernel + attn_merge_kernel (one decode-attention launch)",
                     "bytes_per_launch": round(att_bytes)},
        "wall_s": round(wall, 3),
        "cpu_baseline": cpu,
        "cpu_baseline_1thread": cpu1,
    }
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
