"""Row bookkeeping of the resident block tables on a metadata-only cache (no
GPU): a sequence gets a row with its first block, keeps it while it lives,
and its row is reused after truncate(seq, 0) (kv.rs:153-169) removes it."""

import numpy as np
import pytest

from langtrain_studio_amd.kv import KvError


def _meta(n_tokens=1 << 14):
    from langtrain_studio_amd import KvCache

    return KvCache(1, 64, n_tokens, dtype="f16", device=None)


def _fill(c, seq, start, end):
    c.append_batch(np.full(end - start, seq, dtype=np.uint32), np.arange(start, end, dtype=np.uint64))


def test_rows_assigned_on_first_block_and_stable():
    c = _meta()
    assert c.seq_rows([3, 4]).tolist() == [-1, -1]
    _fill(c, 3, 0, 5)
    _fill(c, 4, 0, 40)
    _fill(c, 3, 5, 100)
    assert c.seq_rows([3, 4, 9]).tolist() == [0, 1, -1]


def test_failed_append_assigns_no_row():
    c = _meta()
    with pytest.raises(KvError):
        c.append(8, 3)  # not contiguous: the sequence stays empty
    assert c.seq_rows([8]).tolist() == [-1]


def test_removed_rows_are_reused_last_in_first_out():
    c = _meta()
    for s in range(4):
        _fill(c, s, 0, 10)
    c.truncate(1, 0)
    c.truncate(2, 0)
    assert c.seq_rows([1, 2]).tolist() == [-1, -1]
    _fill(c, 7, 0, 3)
    _fill(c, 8, 0, 3)
    assert c.seq_rows([7, 8, 0, 3]).tolist() == [2, 1, 0, 3]
    c.truncate(0, 4)  # a shorter table keeps its row
    assert c.seq_rows([0]).tolist() == [0]


def test_share_gives_the_destination_a_row():
    c = _meta()
    _fill(c, 1, 0, 50)
    c.share(1, 2, 20)
    c.share(1, 3, 0)  # len 0 leaves the destination empty (kv.rs:180)
    assert c.seq_rows([1, 2, 3]).tolist() == [0, 1, -1]
    c.share(2, 1, 5)  # the old destination row is released, then taken again
    assert c.seq_rows([1, 2]).tolist() == [0, 1]


def test_device_ops_need_a_device():
    c = _meta()
    _fill(c, 1, 0, 5)
    with pytest.raises(KvError):
        c.sync_tables()
