"""Host logic of ltkv_plan_attention on a metadata-only cache (no GPU):
prefix-group detection over tables forked with share (kv.rs:172-183) and
diverged by copy-on-write (kv.rs:95-110), argument checks and figures."""

import numpy as np
import pytest

BLOCK = 16


def _meta(kv_dim=1024, n_tokens=1 << 20):
    from langtrain_studio_amd import KvCache

    return KvCache(1, kv_dim, n_tokens, dtype="f16", device=None)


def _fill(c, seq, start, end):
    if end > start:
        c.append_batch(np.full(end - start, seq, dtype=np.uint32), np.arange(start, end, dtype=np.uint64))


def _fork(c, root, prefix, children, extra):
    """root holds `prefix` tokens; each child shares them and appends extra[i]."""
    _fill(c, root, 0, prefix)
    for s, e in zip(children, extra):
        c.share(root, s, prefix)
        _fill(c, s, prefix, prefix + e)


def test_prefix_group_of_forked_sequences():
    """256 sequences forked from a 4088-token prefix, each with a private
    suffix: one group whose shared part is the 255 full common blocks (the
    partial block diverged by copy-on-write in every child)."""
    c = _meta()
    kids = list(range(1, 257))
    _fork(c, 0, 4088, kids, [64] * 256)
    lens = [c.len(s) for s in kids]
    st = c.plan_attention(kids, lens, 32, 128, shared_prefix=True)
    assert st["groups"] == 1 and st["grouped"] == 256 and st["shared_blocks"] == 255
    assert st["queries"] == 256 and st["table_width"] == -(-4152 // BLOCK)
    # 8 member tiles (32 members x 4 heads = 128 rows) x 8 kv heads x the prefix partitions
    assert st["prefix_workgroups"] % 64 == 0 and st["prefix_workgroups"] > 0
    st = c.plan_attention(kids, lens, 32, 128, shared_prefix=False)
    assert st["groups"] == 0 and st["grouped"] == 0 and st["prefix_workgroups"] == 0


def test_root_and_children_share_only_common_blocks():
    """The root itself (still holding the original partial block) groups with
    its children over the full blocks they all hold."""
    c = _meta()
    _fork(c, 0, 100, [1, 2, 3], [5, 0, 30])
    seqs = [0, 1, 2, 3]
    lens = [c.len(s) for s in seqs]
    assert lens == [100, 105, 100, 130]
    st = c.plan_attention(seqs, lens, 32, 128)
    assert st["groups"] == 1 and st["grouped"] == 4 and st["shared_blocks"] == 100 // BLOCK


def test_best_member_set_in_a_bucket():
    """Sequences with the same first block but different shared lengths: the
    plan keeps the member set that saves the most block reads."""
    c = _meta()
    _fill(c, 0, 0, 640)                       # 40 blocks
    for s in (1, 2, 3):                       # long forks: share all 40 blocks
        c.share(0, s, 640)
        _fill(c, s, 640, 650)
    c.share(0, 4, 40)                         # a short fork: 2 full blocks + 8 tokens
    _fill(c, 4, 40, 300)
    seqs = [0, 1, 2, 3, 4]
    lens = [c.len(s) for s in seqs]
    st = c.plan_attention(seqs, lens, 32, 128)
    # (4 - 1) * 40 blocks beat (5 - 1) * 2 blocks
    assert st["groups"] == 1 and st["grouped"] == 4 and st["shared_blocks"] == 40


def test_disjoint_groups_and_singletons():
    c = _meta()
    _fork(c, 0, 320, [1, 2], [3, 3])
    _fork(c, 10, 200, [11, 12, 13], [0, 17, 40])
    _fill(c, 20, 0, 500)                      # shares nothing
    seqs = [1, 2, 11, 12, 13, 20, 0, 10]
    lens = [c.len(s) for s in seqs]
    st = c.plan_attention(seqs, lens, 32, 128)
    assert st["groups"] == 2 and st["grouped"] == 7
    assert st["shared_blocks"] == 320 // BLOCK + 200 // BLOCK


def test_short_prefixes_are_not_grouped():
    c = _meta()
    _fork(c, 0, 31, [1, 2], [10, 10])          # one full shared block only
    seqs = [0, 1, 2]
    st = c.plan_attention(seqs, [c.len(s) for s in seqs], 32, 128)
    assert st["groups"] == 0


def test_queries_of_one_sequence_form_a_causal_group():
    """Several queries of one sequence (the tokens of a prefill chunk, each
    reading its own prefix) form one group over the longest one's context,
    partial last block included; a lone query of a sequence does not."""
    c = _meta()
    _fill(c, 0, 0, 300)
    st = c.plan_attention([0, 0, 0], [300, 200, 37], 32, 128)
    assert st["groups"] == 1 and st["grouped"] == 3 and st["shared_blocks"] == -(-300 // BLOCK)
    _fill(c, 1, 0, 1000)
    _fill(c, 1, 1000, 1064)  # a 64-token chunk after a 1000-token context
    st = c.plan_attention([1] * 64 + [0], list(range(1001, 1065)) + [300], 32, 128)
    assert st["groups"] == 1 and st["grouped"] == 64 and st["shared_blocks"] == -(-1064 // BLOCK)
    st = c.plan_attention([1, 0], [1064, 300], 32, 128)
    assert st["groups"] == 0
    # too short a range to group; empty reads never join a group
    st = c.plan_attention([0, 0, 0], [31, 20, 0], 32, 128)
    assert st["groups"] == 0


def test_causal_groups_and_prefix_groups_together():
    """A prefill chunk of one sequence next to decode queries of forks of
    another: one causal group and one prefix group."""
    c = _meta()
    _fork(c, 0, 500, [1, 2, 3], [2, 2, 2])
    _fill(c, 9, 0, 700)
    seqs = [9] * 32 + [1, 2, 3]
    lens = list(range(669, 701)) + [c.len(1), c.len(2), c.len(3)]
    st = c.plan_attention(seqs, lens, 32, 128)
    assert st["groups"] == 2 and st["grouped"] == 35
    assert st["shared_blocks"] == -(-700 // BLOCK) + 500 // BLOCK


def test_f32_pools_and_unsupported_groups_plan_without_prefix_groups():
    from langtrain_studio_amd import KvCache

    c = KvCache(1, 256, 1 << 16, dtype="f32", device=None)
    _fork(c, 0, 320, [1, 2], [3, 3])
    st = c.plan_attention([1, 2], [c.len(1), c.len(2)], 32, 64)
    assert st["groups"] == 0


def test_plan_argument_errors():
    from langtrain_studio_amd import KvError

    c = _meta()
    _fill(c, 0, 0, 40)
    with pytest.raises(KvError, match="exceeds"):
        c.plan_attention([0], [41], 32, 128)
    with pytest.raises(KvError, match="exceeds"):
        c.plan_attention([7], [1], 32, 128)
    with pytest.raises(KvError, match="head_dim"):
        c.plan_attention([0], [40], 32, 96)
    with pytest.raises(KvError):
        c.plan_stats()  # the failed plan left none
    st = c.plan_attention([7, 0], [0, 0], 32, 128)  # empty reads are allowed
    assert st["queries"] == 2 and st["groups"] == 0
