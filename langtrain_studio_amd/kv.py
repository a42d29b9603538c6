"""Paged KV cache on one MI355X: the Python face of libltkv.so.

``KvCache`` mirrors ``langtrain_native::kv::KvCache``
(engine/crates/native/src/kv.rs:15-188): same constructor arguments, same
method names, same errors ("KV cache full", "seq S: position P is not
contiguous (length L)"), same block-allocation order. K and V live in HBM;
``write``/``rows`` take and return host rows like the reference, and the
batched device ops take torch device tensors (torch supplies device memory
and streams only; all compute is the HIP kernels of libltkv.so).
"""

from __future__ import annotations

import ctypes as C
import math
from typing import Optional, Sequence

import numpy as np

from . import _lib

BLOCK = _lib.BLOCK  # kv.rs:13


class KvError(RuntimeError):
    """An error returned by the C ABI (code = LTKV_ERR_*)."""

    def __init__(self, code: int, message: str):
        super().__init__(message)
        self.code = code


class KvCacheFull(KvError):
    """kv.rs:71 "KV cache full"."""


class NonContiguous(KvError):
    """kv.rs:88-91 "seq S: position P is not contiguous (length L)"."""


_ERROR_TYPES = {_lib.ERR_FULL: KvCacheFull, _lib.ERR_NONCONTIG: NonContiguous}


def _check(rc: int) -> None:
    if rc != _lib.OK:
        raise _ERROR_TYPES.get(rc, KvError)(rc, _lib.last_error())


def _np_ptr(a: np.ndarray):
    return a.ctypes.data_as(C.c_void_p)


def _dev_ptr(t, dtype, name: str, device: int):
    """Device address of a contiguous torch tensor of the given dtype."""
    import torch

    if not isinstance(t, torch.Tensor) or not t.is_cuda:
        raise TypeError(f"{name} must be a HIP device tensor")
    if t.dtype != dtype:
        raise TypeError(f"{name} must be {dtype}, got {t.dtype}")
    if not t.is_contiguous():
        raise ValueError(f"{name} must be contiguous")
    if t.device.index != device:
        raise ValueError(f"{name} is on {t.device}, cache is on device {device}")
    return C.c_void_p(t.data_ptr())


class KvCache:
    """kv.rs KvCache with its pools in HBM.

    ``KvCache(n_layers, kv_dim, n_tokens)`` is ``KvCache::new`` (kv.rs:35-48);
    ``dtype`` selects the storage ("f16" as the reference, "f32", or
    "q8_0": int8 quants with one f16 scale per 32 elements, quant.rs:785-791)
    and ``device`` the HIP device (``None`` = a metadata-only cache with no
    pools, whose device ops raise).
    """

    def __init__(self, n_layers: int, kv_dim: int, n_tokens: int, dtype: str = "f16",
                 device: Optional[int] = 0, stream=None):
        codes = {"f16": _lib.F16, "f32": _lib.F32, "q8_0": _lib.Q8_0}
        if dtype not in codes:
            raise ValueError("dtype must be 'f16', 'f32' or 'q8_0'")
        self._lib = _lib.load()
        h = C.c_void_p()
        dev = _lib.NO_DEVICE if device is None else int(device)
        _check(self._lib.ltkv_create(n_layers, kv_dim, n_tokens, codes[dtype], dev, C.byref(h)))
        self._h = h
        self.n_layers = n_layers
        self.dtype = dtype
        self.elem = {"f16": 2, "f32": 4, "q8_0": 1}[dtype]
        self.device = device
        self.n_blocks = self._lib.ltkv_n_blocks(h)
        self._plan_shape = None
        if stream is not None:
            self.set_stream(stream)

    def close(self) -> None:
        h = getattr(self, "_h", None)
        if h:
            self._lib.ltkv_destroy(h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def set_stream(self, stream) -> None:
        """Enqueue device work on ``stream`` (a torch.cuda.Stream or a raw hipStream_t)."""
        raw = getattr(stream, "cuda_stream", stream)
        _check(self._lib.ltkv_set_stream(self._h, C.c_void_p(int(raw or 0))))

    # ---- kv.rs:17-18,50-60,185-187 --------------------------------------------------
    @property
    def kv_dim(self) -> int:
        return self._lib.ltkv_kv_dim(self._h)

    def capacity(self) -> int:
        return self._lib.ltkv_capacity(self._h)

    def bytes(self) -> int:
        return self._lib.ltkv_bytes(self._h)

    def len(self, seq: int) -> int:
        return self._lib.ltkv_len(self._h, seq)

    def free_blocks(self) -> int:
        return self._lib.ltkv_free_blocks(self._h)

    def refcount(self, block: int) -> int:
        return self._lib.ltkv_refcount(self._h, block)

    def cow_copies(self) -> int:
        return self._lib.ltkv_cow_copies(self._h)

    # ---- kv.rs:85-121 ---------------------------------------------------------------
    def append(self, seq: int, pos: int) -> tuple[int, int]:
        """Reserve the cell of ``pos`` (== len(seq)); returns (block, slot)."""
        b, s = C.c_uint32(), C.c_uint32()
        _check(self._lib.ltkv_append(self._h, seq, pos, C.byref(b), C.byref(s)))
        return b.value, s.value

    def append_batch(self, seqs, positions) -> np.ndarray:
        """The cell claim of model.rs:380-383: slot mapping block*16+slot per token."""
        seqs = np.ascontiguousarray(seqs, dtype=np.uint32)
        pos = np.ascontiguousarray(positions, dtype=np.uint64)
        if seqs.shape != pos.shape:
            raise ValueError("seqs and positions differ in length")
        out = np.full(seqs.size, -1, dtype=np.int32)
        done = C.c_size_t()
        rc = self._lib.ltkv_append_batch(self._h, seqs.size, _np_ptr(seqs), _np_ptr(pos), _np_ptr(out),
                                         C.byref(done))
        if rc != _lib.OK:
            err = _ERROR_TYPES.get(rc, KvError)(rc, _lib.last_error())
            err.n_done = done.value
            err.slot_mapping = out
            raise err
        return out

    # ---- kv.rs:123-131 --------------------------------------------------------------
    def write(self, layer: int, block: int, slot: int, k, v) -> None:
        """Write one token's K and V rows (f32, kv_dim each) into (block, slot)."""
        k = np.ascontiguousarray(k, dtype=np.float32).reshape(-1)
        v = np.ascontiguousarray(v, dtype=np.float32).reshape(-1)
        if k.size != self.kv_dim or v.size != self.kv_dim:
            raise ValueError(f"rows must have kv_dim={self.kv_dim} elements")
        _check(self._lib.ltkv_write_row(self._h, layer, block, slot, _np_ptr(k), _np_ptr(v)))

    # ---- kv.rs:133-150 --------------------------------------------------------------
    def rows(self, layer: int, seq: int, n: int) -> tuple[np.ndarray, np.ndarray]:
        """K and V rows of positions 0..n of seq as host [n][kv_dim] arrays
        (uint16 f16 bits, or float32)."""
        dt = np.uint16 if self.elem == 2 else np.float32
        k = np.empty((n, self.kv_dim), dtype=dt)
        v = np.empty((n, self.kv_dim), dtype=dt)
        _check(self._lib.ltkv_rows(self._h, layer, seq, n, _np_ptr(k), _np_ptr(v)))
        return k, v

    # ---- kv.rs:153-183 --------------------------------------------------------------
    def truncate(self, seq: int, from_: int) -> None:
        self._lib.ltkv_truncate(self._h, seq, from_)

    def share(self, src: int, dst: int, length: int) -> None:
        self._lib.ltkv_share(self._h, src, dst, length)

    # ---- tables ---------------------------------------------------------------------
    def block_table(self, seq: int) -> np.ndarray:
        n = C.c_size_t()
        self._lib.ltkv_block_table(self._h, seq, None, 0, C.byref(n))
        out = np.empty(n.value, dtype=np.int32)
        _check(self._lib.ltkv_block_table(self._h, seq, _np_ptr(out), out.size, C.byref(n)))
        return out

    def block_tables(self, seqs, stride: Optional[int] = None) -> np.ndarray:
        seqs = np.ascontiguousarray(seqs, dtype=np.uint32)
        if stride is None:
            stride = max([1] + [math.ceil(self.len(int(s)) / BLOCK) for s in seqs])
        out = np.empty((seqs.size, stride), dtype=np.int32)
        _check(self._lib.ltkv_block_tables(self._h, seqs.size, _np_ptr(seqs), _np_ptr(out), stride))
        return out

    def init_free_order(self, order) -> None:
        o = np.ascontiguousarray(order, dtype=np.uint32)
        _check(self._lib.ltkv_init_free_order(self._h, _np_ptr(o), o.size))

    # ---- device ops (torch device tensors) ------------------------------------------
    def write_batch(self, layer: int, slot_mapping, k, v) -> None:
        """Kernel 1: rows of k, v ([n][>=kv_dim] f32) into cells slot_mapping[n] (int32)."""
        import torch

        n = slot_mapping.numel()
        if k.dim() != 2 or k.shape != v.shape or k.shape[0] != n or k.shape[1] < self.kv_dim:
            raise ValueError("k and v must be [n][>=kv_dim] and match slot_mapping")
        _check(self._lib.ltkv_write(
            self._h, layer, n, _dev_ptr(slot_mapping, torch.int32, "slot_mapping", self.device),
            _dev_ptr(k, torch.float32, "k", self.device), _dev_ptr(v, torch.float32, "v", self.device),
            k.shape[1]))

    def cell_order(self, slot_mapping) -> np.ndarray:
        """Host: the rows of a claimed batch grouped by block in ascending
        block order (ltkv_cell_order), skipped cells left out (int32)."""
        sm = np.ascontiguousarray(slot_mapping, dtype=np.int32)
        order = np.empty(sm.size, dtype=np.int32)
        m = C.c_size_t(0)
        _check(self._lib.ltkv_cell_order(self._h, sm.size, _np_ptr(sm), _np_ptr(order), C.byref(m)))
        return order[:m.value]

    def write_batch_ordered(self, layer: int, slot_mapping, k, v, order) -> None:
        """Kernel 1 over the rows order[m] (int32, device) of a batch:
        row order[j] of k, v into cell slot_mapping[order[j]]."""
        import torch

        n = slot_mapping.numel()
        if k.dim() != 2 or k.shape != v.shape or k.shape[0] != n or k.shape[1] < self.kv_dim:
            raise ValueError("k and v must be [n][>=kv_dim] and match slot_mapping")
        _check(self._lib.ltkv_write_ordered(
            self._h, layer, n, _dev_ptr(slot_mapping, torch.int32, "slot_mapping", self.device),
            _dev_ptr(k, torch.float32, "k", self.device), _dev_ptr(v, torch.float32, "v", self.device),
            k.shape[1], order.numel(), _dev_ptr(order, torch.int32, "order", self.device)))

    def rope_init(self, base: float, rope_dim: int, head_dim: int, neox: bool, max_positions: int) -> None:
        """RoPE table of Model::rope (model.rs:263-265, 291-308) for write_rope."""
        _check(self._lib.ltkv_rope_init(self._h, float(base), rope_dim, head_dim, 1 if neox else 0,
                                        max_positions))

    def write_rope(self, layer: int, slot_mapping, positions, k, v, q=None, n_heads: int = 0) -> None:
        """Kernel 1 with RoPE (model.rs:414-429): k rotated into its cell, v appended,
        q ([n][n_heads*head_dim] f32, optional) rotated in place."""
        import torch

        n = slot_mapping.numel()
        if k.dim() != 2 or k.shape != v.shape or k.shape[0] != n or k.shape[1] < self.kv_dim:
            raise ValueError("k and v must be [n][>=kv_dim] and match slot_mapping")
        if positions.numel() != n:
            raise ValueError("positions must match slot_mapping")
        qp, qs = None, 0
        if q is not None:
            if q.dim() != 2 or q.shape[0] != n:
                raise ValueError("q must be [n][n_heads*head_dim]")
            qp, qs = _dev_ptr(q, torch.float32, "q", self.device), q.shape[1]
        _check(self._lib.ltkv_write_rope(
            self._h, layer, n, _dev_ptr(slot_mapping, torch.int32, "slot_mapping", self.device),
            _dev_ptr(positions, torch.int32, "positions", self.device),
            _dev_ptr(k, torch.float32, "k", self.device), _dev_ptr(v, torch.float32, "v", self.device),
            k.shape[1], qp, qs, n_heads))

    def copy_blocks(self, pairs) -> None:
        """Kernel 2: copy block pairs[i,0] -> pairs[i,1] (all layers, K and V)."""
        import torch

        if pairs.dim() != 2 or pairs.shape[1] != 2:
            raise ValueError("pairs must be [n][2]")
        _check(self._lib.ltkv_copy_blocks(self._h, pairs.shape[0],
                                          _dev_ptr(pairs, torch.int32, "pairs", self.device)))

    def gather(self, layer: int, tables, lens, out_offsets, k_out, v_out) -> None:
        """Kernel 3: rows 0..lens[i] of each table to k_out/v_out rows out_offsets[i]..."""
        import torch

        dt = {1: torch.int8, 2: torch.float16, 4: torch.float32}[self.elem]
        n = lens.numel()
        if tables.dim() != 2 or tables.shape[0] != n or out_offsets.numel() != n:
            raise ValueError("tables must be [n][stride]; lens and out_offsets [n]")
        if k_out.dim() != 2 or k_out.shape[1] != self.kv_dim or v_out.shape != k_out.shape:
            raise ValueError("k_out and v_out must be [rows][kv_dim]")
        _check(self._lib.ltkv_gather(
            self._h, layer, n, _dev_ptr(tables, torch.int32, "tables", self.device), tables.shape[1],
            _dev_ptr(lens, torch.int32, "lens", self.device),
            _dev_ptr(out_offsets, torch.int64, "out_offsets", self.device),
            _dev_ptr(k_out, dt, "k_out", self.device), _dev_ptr(v_out, dt, "v_out", self.device)))

    def decode_attention(self, layer: int, q, tables, lens, n_heads: int, head_dim: int,
                         scale: Optional[float] = None, out=None, noalloc: bool = False):
        """Kernel 4: GQA paged decode attention; q, out are [n][n_heads*head_dim] f32.
        noalloc: ltkv_decode_attention_noalloc (partials in the device's static
        scratch; nothing allocated, same result bits)."""
        import torch

        n = lens.numel()
        if q.dim() != 2 or q.shape != (n, n_heads * head_dim):
            raise ValueError("q must be [n][n_heads*head_dim]")
        if tables.dim() != 2 or tables.shape[0] != n:
            raise ValueError("tables must be [n][stride]")
        if out is None:
            out = torch.empty_like(q)
        elif out.shape != q.shape:
            raise ValueError("out must match q")
        if scale is None:
            scale = 1.0 / math.sqrt(head_dim)  # model.rs:402
        fn = self._lib.ltkv_decode_attention_noalloc if noalloc else self._lib.ltkv_decode_attention
        _check(fn(
            self._h, layer, n, n_heads, head_dim, float(scale),
            _dev_ptr(q, torch.float32, "q", self.device),
            _dev_ptr(tables, torch.int32, "tables", self.device), tables.shape[1],
            _dev_ptr(lens, torch.int32, "lens", self.device),
            _dev_ptr(out, torch.float32, "out", self.device)))
        return out

    # ---- resident block tables (device step descriptor)
    def seq_rows(self, seqs: Sequence[int]) -> np.ndarray:
        """Row of each sequence in the resident tables (-1: no blocks)."""
        seqs_a = np.ascontiguousarray(seqs, dtype=np.uint32)
        out = np.empty(seqs_a.shape, dtype=np.int32)
        _check(self._lib.ltkv_seq_rows(self._h, seqs_a.size, _np_ptr(seqs_a), _np_ptr(out)))
        return out

    def sync_tables(self) -> None:
        """Enqueue the upload of the block-table changes since the last one."""
        _check(self._lib.ltkv_sync_tables(self._h))

    def resident_tables(self):
        """(tables [rows][stride], lengths [rows]) of the resident tables,
        copied to host after pending uploads (synchronous)."""
        t, l = C.c_void_p(), C.c_void_p()
        stride, rows = C.c_size_t(), C.c_size_t()
        _check(self._lib.ltkv_resident_tables(self._h, C.byref(t), C.byref(l), C.byref(stride),
                                              C.byref(rows)))
        tables = np.empty((rows.value, stride.value), dtype=np.int32)
        lengths = np.empty((rows.value,), dtype=np.int32)
        _check(self._lib.ltkv_read_resident_tables(self._h, _np_ptr(tables), _np_ptr(lengths)))
        return tables, lengths

    def slot_mapping(self, rows, pos, out=None):
        """Slot mapping of tokens (row, position) from the resident tables,
        computed on the device; rows int32, pos int64 device tensors."""
        import torch

        n = rows.numel()
        if pos.numel() != n:
            raise ValueError("rows and pos must have equal length")
        if out is None:
            out = torch.empty((n,), dtype=torch.int32, device=rows.device)
        _check(self._lib.ltkv_slot_mapping(self._h, n, _dev_ptr(rows, torch.int32, "rows", self.device),
                                           _dev_ptr(pos, torch.int64, "pos", self.device),
                                           _dev_ptr(out, torch.int32, "out", self.device)))
        return out

    def decode_attention_rows(self, layer: int, q, rows, lens, n_heads: int, head_dim: int,
                              scale: Optional[float] = None, out=None):
        """decode_attention over the resident tables: query i reads the
        sequence in row rows[i] (device int32)."""
        import torch

        n = lens.numel()
        if q.dim() != 2 or q.shape != (n, n_heads * head_dim):
            raise ValueError("q must be [n][n_heads*head_dim]")
        if rows.numel() != n:
            raise ValueError("rows must have one entry per query")
        if out is None:
            out = torch.empty_like(q)
        elif out.shape != q.shape:
            raise ValueError("out must match q")
        if scale is None:
            scale = 1.0 / math.sqrt(head_dim)  # model.rs:402
        _check(self._lib.ltkv_decode_attention_rows(
            self._h, layer, n, n_heads, head_dim, float(scale),
            _dev_ptr(q, torch.float32, "q", self.device),
            _dev_ptr(rows, torch.int32, "rows", self.device),
            _dev_ptr(lens, torch.int32, "lens", self.device),
            _dev_ptr(out, torch.float32, "out", self.device)))
        return out

    def table_uploads(self) -> int:
        """Resident-table entries uploaded so far."""
        v = C.c_uint64()
        _check(self._lib.ltkv_table_uploads(self._h, C.byref(v)))
        return int(v.value)

    def append_decode_attention(self, layer: int, slot_mapping, k, v, q, tables, lens, n_heads: int,
                                head_dim: int, scale: Optional[float] = None, out=None):
        """write_batch(layer, slot_mapping, k, v) then decode_attention in one
        launch (f16 pools): slot_mapping[i] must be position lens[i] - 1 of
        query i's table, one new token per sequence."""
        import torch

        n = lens.numel()
        if q.dim() != 2 or q.shape != (n, n_heads * head_dim):
            raise ValueError("q must be [n][n_heads*head_dim]")
        if tables.dim() != 2 or tables.shape[0] != n:
            raise ValueError("tables must be [n][stride]")
        if k.shape != (n, self.kv_dim) or v.shape != k.shape or slot_mapping.numel() != n:
            raise ValueError("k, v must be [n][kv_dim] and slot_mapping [n]")
        if out is None:
            out = torch.empty_like(q)
        elif out.shape != q.shape:
            raise ValueError("out must match q")
        if scale is None:
            scale = 1.0 / math.sqrt(head_dim)  # model.rs:402
        _check(self._lib.ltkv_append_decode_attention(
            self._h, layer, n, n_heads, head_dim, float(scale),
            _dev_ptr(q, torch.float32, "q", self.device),
            _dev_ptr(tables, torch.int32, "tables", self.device), tables.shape[1],
            _dev_ptr(lens, torch.int32, "lens", self.device),
            _dev_ptr(slot_mapping, torch.int32, "slot_mapping", self.device),
            _dev_ptr(k, torch.float32, "k", self.device), _dev_ptr(v, torch.float32, "v", self.device),
            k.stride(0), _dev_ptr(out, torch.float32, "out", self.device)))
        return out

    def plan_attention(self, seqs: Sequence[int], lens: Sequence[int], n_heads: int, head_dim: int,
                       shared_prefix: bool = True, f16_products: bool = False) -> dict:
        """Step descriptor for planned_attention: query i reads positions
        [0, lens[i]) of sequence seqs[i]; with shared_prefix, queries forked
        from a common prefix attend to its shared blocks once, together (with
        f16_products, on products of f16-rounded Q and weights: faster, ~3e-4
        relative error instead of f32 accuracy). Returns the plan's figures."""
        seqs_a = np.ascontiguousarray(seqs, dtype=np.uint32)
        lens_a = np.ascontiguousarray(lens, dtype=np.uint32)
        if seqs_a.shape != lens_a.shape or seqs_a.ndim != 1:
            raise ValueError("seqs and lens must be 1-D of equal length")
        _check(self._lib.ltkv_plan_attention(self._h, len(seqs_a), _np_ptr(seqs_a), _np_ptr(lens_a),
                                             n_heads, head_dim,
                                             (1 if shared_prefix else 0) | (2 if f16_products else 0)))
        self._plan_shape = (len(seqs_a), n_heads * head_dim, head_dim)
        return self.plan_stats()

    def plan_stats(self) -> dict:
        out = np.zeros(6, dtype=np.uint64)
        _check(self._lib.ltkv_plan_stats(self._h, _np_ptr(out)))
        keys = ("queries", "groups", "grouped", "shared_blocks", "prefix_workgroups", "table_width")
        return {k: int(v) for k, v in zip(keys, out)}

    def planned_attention(self, layer: int, q, scale: Optional[float] = None, out=None):
        """Attention of the planned batch on one layer; q, out [n][n_heads*head_dim] f32."""
        import torch

        if self._plan_shape is None:
            raise KvError(_lib.ERR_ARG, "no attention plan (plan_attention)")
        n, width, head_dim = self._plan_shape
        if q.dim() != 2 or q.shape != (n, width):
            raise ValueError("q must be [n][n_heads*head_dim] of the plan")
        if out is None:
            out = torch.empty_like(q)
        elif out.shape != q.shape:
            raise ValueError("out must match q")
        if scale is None:
            scale = 1.0 / math.sqrt(head_dim)  # model.rs:402
        _check(self._lib.ltkv_planned_attention(
            self._h, layer, float(scale), _dev_ptr(q, torch.float32, "q", self.device),
            _dev_ptr(out, torch.float32, "out", self.device)))
        return out

    def set_attention_partition(self, tokens: int) -> None:
        _check(self._lib.ltkv_set_attention_partition(self._h, tokens))

    def set_attention_engine(self, engine: str) -> None:
        """'auto' (matrix cores for f16 and q8_0 pools) or 'valu' (f16 pools on
        the vector-ALU kernels, as f32 pools always are)."""
        codes = {"auto": _lib.ENGINE_AUTO, "valu": _lib.ENGINE_VALU}
        if engine not in codes:
            raise ValueError(f"engine must be one of {sorted(codes)}")
        _check(self._lib.ltkv_set_attention_engine(self._h, codes[engine]))

    def read_pool(self, layer: int = 0) -> tuple[np.ndarray, np.ndarray]:
        """Raw K and V pools of one layer, [n_blocks][16][kv_dim] on the host
        (f16 bits as uint16, float32, or q8_0 quants as int8)."""
        dt = {1: np.int8, 2: np.uint16, 4: np.float32}[self.elem]
        shape = (self.n_blocks, BLOCK, self.kv_dim)
        k = np.empty(shape, dtype=dt)
        v = np.empty(shape, dtype=dt)
        _check(self._lib.ltkv_read_pool(self._h, layer, _np_ptr(k), _np_ptr(v)))
        return k, v

    def read_scales(self, layer: int = 0) -> tuple[np.ndarray, np.ndarray]:
        """K and V scale pools of one layer of a q8_0 cache,
        [n_blocks][kv_dim/32][16] f16 bits (uint16) on the host: the scale of
        slot s, 32-element group g of block b is [b][g][s]."""
        shape = (self.n_blocks, self.kv_dim // 32, BLOCK)
        k = np.empty(shape, dtype=np.uint16)
        v = np.empty(shape, dtype=np.uint16)
        _check(self._lib.ltkv_read_scales(self._h, layer, _np_ptr(k), _np_ptr(v)))
        return k, v

    def synchronize(self) -> None:
        _check(self._lib.ltkv_synchronize(self._h))
