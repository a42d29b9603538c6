"""The Backend trait's KV methods of PagedKvBackend on a metadata-only cache
(no GPU): n_ctx is the cache capacity (native/src/lib.rs:140-142), kv_remove
is KvCache::truncate and kv_copy is KvCache::share (lib.rs:192-198)."""

import pytest

from langtrain_studio_amd import PagedKvBackend


def _meta(**kw):
    return PagedKvBackend(2, 8, 2, 64, 100, device=None, **kw)


def test_n_ctx_is_the_block_rounded_capacity():
    b = _meta()
    assert b.n_ctx() == 112  # 100 tokens -> 7 blocks of 16 (kv.rs:36)
    assert b.n_seq_max() == 1 and b.n_batch() == 512


def test_kv_copy_and_kv_remove_follow_share_and_truncate():
    import numpy as np

    b = _meta()
    b.kv.append_batch(np.zeros(40, dtype=np.uint32), np.arange(40, dtype=np.uint64))
    b.kv_copy(0, 5, 20)
    assert b.kv.len(5) == 20 and b.kv.block_table(5).tolist() == b.kv.block_table(0)[:2].tolist()
    b.kv_copy(0, 6, 100)  # len past the source: clamped to its length (kv.rs:177)
    assert b.kv.len(6) == 40
    b.kv_remove(0, 17)
    assert b.kv.len(0) == 17 and len(b.kv.block_table(0)) == 2
    b.kv_remove(9, 0)  # a missing sequence is a no-op
    b.kv_remove(6, 0)
    assert b.kv.len(6) == 0
    assert b.kv.free_blocks() == 7 - 2  # blocks 0 and 1 stay held by sequences 0 and 5


def test_descriptor_is_checked():
    with pytest.raises(ValueError):
        _meta(descriptor="bogus")
    with pytest.raises(ValueError):
        PagedKvBackend(1, 6, 4, 64, 64, device=None)  # 6 query heads over 4 kv heads
