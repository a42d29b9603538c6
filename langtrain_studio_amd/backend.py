"""The KV-cache half of the engine's compute backend, on one MI355X.

``PagedKvBackend`` is the part of ``NativeBackend`` (engine/crates/native/src/
lib.rs:136-198) that the paged KV path covers, with the ``Backend`` trait's
KV methods (engine/crates/engine/src/backend.rs:17-45): ``n_ctx``,
``kv_remove`` (-> KvCache::truncate), ``kv_copy`` (-> KvCache::share) and the
KV segment of ``decode`` (model.rs:380-475): claim every token's cell first
(copy-on-write copies land before any write), then per layer write K/V and
run GQA attention over the paged rows. Projections, RoPE and the rest of the
transformer stay with the caller.
"""

from __future__ import annotations

import math
from dataclasses import dataclass
from typing import Optional, Sequence

import numpy as np

from .kv import BLOCK, KvCache


@dataclass(frozen=True)
class BatchToken:
    """One token of a decode batch (backend.rs:7-15)."""

    token: int
    pos: int
    seq: int
    logits: bool = False


@dataclass
class StepPlan:
    """Device-resident description of one claimed batch."""

    n: int
    slot_mapping: "object"  # torch.int32 [n], cell block*16+slot per token
    tables: "object"        # torch.int32 [n][stride], the token's sequence table ("tables")
    lens: "object"          # torch.int32 [n], pos+1 (positions attended, model.rs:437)
    slot_mapping_host: np.ndarray
    rows: "object" = None   # torch.int32 [n], the token's resident table row ("resident")
    planned: bool = False   # the cache holds this step's attention plan ("planned")
    decode_only: bool = False  # one token per sequence: write and attention fuse into one launch

DESCRIPTORS = ("tables", "resident", "planned")


class PagedKvBackend:
    """descriptor selects how a step's block tables reach the device:
    "tables" uploads each token's full table per step; "resident" reads the
    cache's device-resident tables by sequence row (only changed entries are
    uploaded); "planned" builds one attention plan per step
    (ltkv_plan_attention, shared-prefix and prefill-chunk groups on the
    matrix cores) that every layer of the step reuses."""

    def __init__(self, n_layers: int, n_heads: int, n_kv_heads: int, head_dim: int, kv_tokens: int,
                 n_seq_max: int = 1, n_batch: int = 512, dtype: str = "f16", device: int = 0,
                 stream=None, descriptor: str = "tables"):
        if n_heads % n_kv_heads:
            raise ValueError("n_heads must be a multiple of n_kv_heads")
        if descriptor not in DESCRIPTORS:
            raise ValueError(f"descriptor must be one of {DESCRIPTORS}")
        self.descriptor = descriptor
        self.n_layers, self.n_heads, self.n_kv_heads, self.head_dim = n_layers, n_heads, n_kv_heads, head_dim
        self.kv = KvCache(n_layers, n_kv_heads * head_dim, kv_tokens, dtype=dtype, device=device,
                          stream=stream)
        self._n_seq_max, self._n_batch = n_seq_max, n_batch
        self.device = device
        self.scale = 1.0 / math.sqrt(head_dim)  # model.rs:402

    # Backend trait, KV part (backend.rs:23-26,37-40; lib.rs:140-148,192-198)
    def n_ctx(self) -> int:
        return self.kv.capacity()

    def n_seq_max(self) -> int:
        return self._n_seq_max

    def n_batch(self) -> int:
        return self._n_batch

    def kv_remove(self, seq: int, from_: int) -> None:
        self.kv.truncate(seq, from_)

    def kv_copy(self, src: int, dst: int, length: int) -> None:
        self.kv.share(src, dst, length)

    # decode, KV segment
    def begin_step(self, batch: Sequence[BatchToken]) -> StepPlan:
        """Claim every token's cell (model.rs:380-383) and upload the step's
        slot mapping, block tables and lengths. Raises KvCacheFull /
        NonContiguous like the reference's ``?``."""
        import torch

        if len(batch) > self._n_batch:
            raise ValueError(f"batch of {len(batch)} exceeds n_batch {self._n_batch}")
        seqs = np.array([b.seq for b in batch], dtype=np.uint32)
        pos = np.array([b.pos for b in batch], dtype=np.uint64)
        sm = self.kv.append_batch(seqs, pos)
        lens = (pos + 1).astype(np.int32)
        dev = torch.device("cuda", self.device)
        plan = StepPlan(n=len(batch), slot_mapping=torch.from_numpy(sm).to(dev), tables=None,
                        lens=torch.from_numpy(lens).to(dev), slot_mapping_host=sm)
        if self.descriptor == "tables":
            stride = max(1, int(math.ceil(lens.max() / BLOCK))) if len(batch) else 1
            plan.tables = torch.from_numpy(self.kv.block_tables(seqs, stride)).to(dev)
            plan.decode_only = len(batch) > 0 and np.unique(seqs).size == len(batch)
        elif self.descriptor == "resident":
            plan.rows = torch.from_numpy(self.kv.seq_rows(seqs)).to(dev)
        else:
            self.kv.plan_attention(seqs, lens, self.n_heads, self.head_dim, shared_prefix=True)
            plan.planned = True
        return plan

    def layer(self, plan: StepPlan, layer: int, q, k, v, out: Optional[object] = None):
        """model.rs:414-475 for one layer: write k, v ([n][kv_dim] f32, RoPE
        already applied) into the claimed cells, then attention of q
        ([n][n_heads*head_dim] f32) over each token's sequence."""
        if plan.decode_only:  # ltkv_append_decode_attention: bit-identical to write + attention
            return self.kv.append_decode_attention(layer, plan.slot_mapping, k, v, q, plan.tables, plan.lens,
                                                   self.n_heads, self.head_dim, self.scale, out=out)
        self.kv.write_batch(layer, plan.slot_mapping, k, v)
        if plan.planned:
            return self.kv.planned_attention(layer, q, self.scale, out=out)
        if plan.rows is not None:
            return self.kv.decode_attention_rows(layer, q, plan.rows, plan.lens, self.n_heads, self.head_dim,
                                                 self.scale, out=out)
        return self.kv.decode_attention(layer, q, plan.tables, plan.lens, self.n_heads, self.head_dim,
                                        self.scale, out=out)
