"""CPU checks of the product library: it loads, exports exactly the C ABI of
include/ltkv.h, and its host block manager (a metadata-only cache, no GPU)
makes the same decisions as the oracle's restatement of kv.rs."""

from __future__ import annotations

import os
import re
import subprocess

import numpy as np
import pytest

from conftest import ROOT

HEADER = os.path.join(ROOT, "include", "ltkv.h")


def _declared():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"LTKV_API[^;(]*?\b(ltkv_\w+)\s*\(", text)))


def test_header_declares_the_abi():
    names = _declared()
    assert "ltkv_decode_attention" in names and "ltkv_write" in names
    assert len(names) >= 25


def test_library_exports_every_declared_symbol():
    from langtrain_studio_amd import _lib

    lib = _lib.load()
    for name in _declared():
        assert hasattr(lib, name), name
    assert set(_declared()) == set(_lib.SIGNATURES), "ctypes table out of sync with ltkv.h"
    out = subprocess.run(["nm", "-D", "--defined-only", _lib.LIB_PATH], capture_output=True, text=True).stdout
    exported = {l.split()[-1] for l in out.splitlines() if l.strip()}
    exported = {e for e in exported if not e.startswith("__hip_cuid")}
    assert exported == set(_declared()), exported ^ set(_declared())


def test_profiling_build_adds_only_the_timeline_reader():
    """libltkv_timeline.so (-DLTKV_TIMELINE) is the product's ABI plus
    ltkv_timeline_read; the product library has no instrumentation symbol."""
    from langtrain_studio_amd.build import TIMELINE_LIB

    if not os.path.exists(TIMELINE_LIB):
        pytest.skip("profiling build not built (python -m langtrain_studio_amd.build)")
    out = subprocess.run(["nm", "-D", "--defined-only", TIMELINE_LIB], capture_output=True, text=True).stdout
    exported = {l.split()[-1] for l in out.splitlines() if l.strip()}
    exported = {e for e in exported if not e.startswith("__hip_cuid")}
    assert exported == set(_declared()) | {"ltkv_timeline_read"}, exported ^ set(_declared())


def test_header_compiles_as_c():
    src = f'#include "{HEADER}"\nint main(void) {{ return LTKV_BLOCK == 16 ? 0 : 1; }}\n'
    res = subprocess.run(["gcc", "-std=c99", "-Wall", "-Werror", "-x", "c", "-", "-o", "/dev/null"],
                         input=src, capture_output=True, text=True)
    assert res.returncode == 0, res.stderr


def test_metadata_only_cache_rejects_device_ops():
    from langtrain_studio_amd import KvCache, KvError

    kv = KvCache(1, 64, 256, device=None)
    with pytest.raises(KvError, match="metadata-only"):
        kv.synchronize()
    with pytest.raises(KvError, match="metadata-only"):
        kv.read_pool(0)


def test_create_argument_errors():
    from langtrain_studio_amd import KvCache, KvError

    with pytest.raises(KvError, match="must be > 0"):
        KvCache(1, 0, 256, device=None)
    with pytest.raises(KvError, match="must be > 0"):
        KvCache(0, 64, 256, device=None)
    with pytest.raises(KvError, match="multiple of 32"):
        KvCache(1, 48, 256, dtype="q8_0", device=None)
    KvCache(1, 4, 256, device=None)  # any kv_dim, as kv.rs:202-229 use 4


def test_reference_known_answers_on_product_host_logic():
    """kv.rs:202-229 bookkeeping through the product's C ABI (no data)."""
    from langtrain_studio_amd import KvCache, NonContiguous

    kv = KvCache(1, 4, 256, device=None)
    for p in range(20):
        kv.append(0, p)
    kv.share(0, 1, 20)
    before = kv.free_blocks()
    assert kv.append(1, 20) == (2, 4)
    assert kv.free_blocks() == before - 1 and kv.len(0) == 20 and kv.cow_copies() == 1
    kv = KvCache(1, 4, 64, device=None)
    for p in range(40):
        kv.append(3, p)
    assert kv.free_blocks() == 1
    kv.truncate(3, 10)
    assert kv.free_blocks() == 3
    kv.truncate(3, 0)
    assert kv.free_blocks() == 4
    with pytest.raises(NonContiguous, match=r"^seq 3: position 5 is not contiguous \(length 0\)$"):
        kv.append(3, 5)


def test_product_allocator_tracks_oracle_on_random_ops():
    from langtrain_studio_amd import KvCache, KvError
    from oracle import OracleError, OracleKv

    rng = np.random.default_rng(21)
    n_blocks = 48
    g = KvCache(2, 16, n_blocks * 16, device=None)
    o = OracleKv(2, 16, n_blocks * 16)
    order = rng.permutation(n_blocks)
    g.init_free_order(order)
    o.init_free_order(order)
    for step in range(3000):
        op = rng.choice(["append", "batch", "truncate", "share"], p=[0.45, 0.2, 0.2, 0.15])
        s = int(rng.integers(0, 8))
        if op == "append":
            pos = g.len(s) if rng.random() < 0.95 else g.len(s) + 1
            res = []
            for kv, err in ((g, KvError), (o, OracleError)):
                try:
                    res.append(kv.append(s, pos))
                except err as e:
                    res.append(("err", e.code, str(e)))
            assert res[0] == res[1], (step, res)
        elif op == "batch":
            seqs = rng.integers(0, 8, int(rng.integers(1, 12))).astype(np.uint32)
            lens = {}
            pos = []
            for q in seqs:
                lens.setdefault(int(q), g.len(int(q)))
                pos.append(lens[int(q)])
                lens[int(q)] += 1
            res = []
            for kv, err in ((g, KvError), (o, OracleError)):
                try:
                    res.append(("ok", kv.append_batch(seqs, pos).tolist()))
                except err as e:
                    res.append(("err", e.code, str(e), e.n_done, e.slot_mapping[:e.n_done].tolist()))
            assert res[0] == res[1], (step, res)
        elif op == "truncate":
            frm = int(rng.integers(0, 70))
            g.truncate(s, frm)
            o.truncate(s, frm)
        else:
            d, n = int(rng.integers(0, 8)), int(rng.integers(0, 90))
            g.share(s, d, n)
            o.share(s, d, n)
        assert g.free_blocks() == o.free_blocks()
        assert g.cow_copies() == o.cow_copies()
        for q in range(8):
            assert g.len(q) == o.len(q)
            np.testing.assert_array_equal(g.block_table(q), o.block_table(q))
        for b in range(n_blocks):
            assert g.refcount(b) == o.refcount(b)
    assert o.cow_copies() > 20


def test_block_tables_pad_with_minus_one():
    from langtrain_studio_amd import KvCache, KvError

    kv = KvCache(1, 8, 100 * 16, device=None)
    kv.append_batch([0] * 40 + [1] * 3, list(range(40)) + list(range(3)))
    t = kv.block_tables([0, 1, 5], 4)
    np.testing.assert_array_equal(t, [[0, 1, 2, -1], [3, -1, -1, -1], [-1, -1, -1, -1]])
    with pytest.raises(KvError):
        kv.block_tables([0], 2)


def test_init_free_order_validation():
    from langtrain_studio_amd import KvCache, KvError

    kv = KvCache(1, 8, 4 * 16, device=None)
    with pytest.raises(KvError, match="permutation"):
        kv.init_free_order([0, 1, 1, 2])
    kv.init_free_order([3, 1, 0, 2])
    kv.append(0, 0)
    with pytest.raises(KvError, match="no sequences"):
        kv.init_free_order([0, 1, 2, 3])


@pytest.mark.parametrize("n_seqs,per_seq,slack", [(64, 40, 1.1), (3, 5, 200.0)])
def test_cell_order_groups_rows_by_ascending_block(n_seqs, per_seq, slack):
    """ltkv_cell_order on a claimed batch over a permuted pool (both the
    counting sort and, with few rows against the pool, the sorting form):
    every written row once, skipped cells left out, cells ascending (a
    block's rows in a claim are one sequence's increasing positions)."""
    from langtrain_studio_amd import KvCache

    rng = np.random.default_rng(n_seqs)
    n_blocks = int(n_seqs * -(-per_seq // 16) * slack) + 4
    kv = KvCache(1, 64, n_blocks * 16, device=None)
    kv.init_free_order(rng.permutation(n_blocks))
    # interleave the sequences' tokens, as a mixed step claims them
    order_tok = rng.permutation(np.repeat(np.arange(n_seqs), per_seq))
    seqs, pos, nxt = [], [], np.zeros(n_seqs, dtype=np.int64)
    for s in order_tok:
        seqs.append(s)
        pos.append(nxt[s])
        nxt[s] += 1
    sm = kv.append_batch(np.array(seqs, np.uint32), np.array(pos, np.uint64)).copy()
    sm[::7] = -1  # skipped cells
    order = kv.cell_order(sm)
    assert order.dtype == np.int32
    np.testing.assert_array_equal(np.sort(order), np.flatnonzero(sm >= 0))
    cells = sm[order]
    assert (np.diff(cells) > 0).all()
    assert kv.cell_order(np.zeros(0, np.int32)).size == 0
