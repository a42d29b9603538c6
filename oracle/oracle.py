"""ctypes front end of the C++ oracle (libltkv_oracle.so).

Test infrastructure only: a checker for the HIP product and the CPU
baseline timed beside it. Method names follow
engine/crates/native/src/kv.rs:50-187 (KvCache) so the parity tests read
like the reference's own tests.
"""

from __future__ import annotations

import ctypes as C
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "libltkv_oracle.so")
_lib_path = _LIB_PATH
_lib = None

F16, F32, Q8_0 = 0, 1, 2
BLOCK = 16

_ERRORS = {1: "full", 2: "noncontig", 3: "range", 5: "arg"}


class OracleError(RuntimeError):
    def __init__(self, code: int, msg: str):
        super().__init__(msg)
        self.code = code


def build() -> str:
    """Compile the oracle with its Makefile (g++ only, no GPU)."""
    subprocess.run(["make", "-s", "-C", _HERE], check=True)
    return _LIB_PATH


def build_native(out_dir: str) -> str:
    """Compile the oracle with -march=native for the host this runs on (the
    CPU baseline's build; every other flag as the Makefile's) into out_dir."""
    out = os.path.join(out_dir, "libltkv_oracle_native.so")
    subprocess.run(["make", "-s", "-C", _HERE, "MARCH=native", f"OUT={out}"], check=True,
                   capture_output=True, text=True, timeout=300)
    return out


def use_library(path: str) -> None:
    """Load the oracle from `path` for OracleKv objects created from now on
    (the CPU baseline switches to its -march=native build this way)."""
    global _lib, _lib_path
    _lib = None
    _lib_path = path
    load()


def load():
    global _lib
    if _lib is not None:
        return _lib
    if _lib_path == _LIB_PATH and not os.path.exists(_LIB_PATH):
        build()
    lib = C.CDLL(_lib_path)
    sz, u32, i32, u64, vp = C.c_size_t, C.c_uint32, C.c_int32, C.c_uint64, C.c_void_p
    P = C.POINTER
    sig = {
        "ora_last_error": (C.c_char_p, []),
        "ora_f32_to_f16": (None, [vp, vp, sz]),
        "ora_f32_to_f16_simd": (None, [vp, vp, sz]),
        "ora_f16_to_f32": (None, [vp, vp, sz]),
        "ora_f16_to_f32_simd": (None, [vp, vp, sz]),
        "ora_has_f16c": (C.c_int, []),
        "ora_create": (vp, [sz, sz, sz, C.c_int]),
        "ora_destroy": (None, [vp]),
        "ora_capacity": (sz, [vp]),
        "ora_bytes": (sz, [vp]),
        "ora_n_blocks": (sz, [vp]),
        "ora_len": (sz, [vp, u32]),
        "ora_free_blocks": (sz, [vp]),
        "ora_refcount": (u32, [vp, sz]),
        "ora_cow_copies": (u64, [vp]),
        "ora_has_seq": (C.c_int, [vp, u32]),
        "ora_init_free_order": (C.c_int, [vp, vp, sz]),
        "ora_append": (C.c_int, [vp, u32, sz, P(u32), P(u32)]),
        "ora_append_batch": (C.c_int, [vp, sz, vp, vp, vp, P(sz)]),
        "ora_write": (None, [vp, sz, sz, sz, vp, vp]),
        "ora_write_batch": (None, [vp, sz, sz, vp, vp, vp]),
        "ora_write_rope_batch": (None, [vp, sz, sz, vp, vp, vp, vp, vp, sz, sz, C.c_float, sz, sz, C.c_int]),
        "ora_rows": (C.c_int, [vp, sz, u32, sz, vp, vp]),
        "ora_block_table": (C.c_int, [vp, u32, vp, sz, P(sz)]),
        "ora_truncate": (None, [vp, u32, sz]),
        "ora_copy_blocks": (sz, [vp, sz, vp]),
        "ora_share": (None, [vp, u32, u32, sz]),
        "ora_pool": (None, [vp, sz, vp, vp]),
        "ora_load_pool": (None, [vp, sz, vp, vp]),
        "ora_attention": (C.c_int, [vp, sz, sz, vp, vp, sz, sz, C.c_float, vp, vp, sz]),
        "ora_attention_tables": (C.c_int, [vp, sz, sz, vp, sz, vp, sz, sz, C.c_float, vp, vp, sz]),
        "ora_pool_selftest": (u64, [sz, sz, vp]),
        "ora_quantize_block": (C.c_float, [vp, vp]),
        "ora_scales": (C.c_int, [vp, sz, vp, vp]),
        "ora_load_scales": (C.c_int, [vp, sz, vp, vp]),
    }
    for name, (res, args) in sig.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    _lib = lib
    return lib


def _ptr(a: np.ndarray):
    return a.ctypes.data_as(C.c_void_p)


def f32_to_f16(x, simd: bool = False) -> np.ndarray:
    """IEEE binary16 RNE rounding (f16::from_f32), returned as uint16 bits."""
    lib = load()
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty(x.shape, dtype=np.uint16)
    (lib.ora_f32_to_f16_simd if simd else lib.ora_f32_to_f16)(_ptr(x), _ptr(out), x.size)
    return out


def f16_to_f32(bits, simd: bool = False) -> np.ndarray:
    lib = load()
    b = np.ascontiguousarray(bits, dtype=np.uint16)
    out = np.empty(b.shape, dtype=np.float32)
    (lib.ora_f16_to_f32_simd if simd else lib.ora_f16_to_f32)(_ptr(b), _ptr(out), b.size)
    return out


def has_f16c() -> bool:
    return bool(load().ora_has_f16c())


def quantize_block(x) -> tuple[float, np.ndarray]:
    """quant.rs:785-791 on one 32-element block: (d as f32, int8 quants)."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    assert x.size == 32
    q = np.empty(32, dtype=np.int8)
    d = load().ora_quantize_block(_ptr(x), _ptr(q))
    return float(d), q


def pool_selftest(threads: int, n: int) -> np.ndarray:
    hits = np.zeros(max(n, 1), dtype=np.uint32)
    load().ora_pool_selftest(threads, n, _ptr(hits))
    return hits[:n]


class OracleKv:
    """kv.rs KvCache restated in C++ (host memory, reference layout)."""

    def __init__(self, n_layers: int, kv_dim: int, n_tokens: int, dtype: str = "f16"):
        self._lib = load()
        codes = {"f16": F16, "f32": F32, "q8_0": Q8_0}
        self.dtype = dtype
        self.elem = {"f16": 2, "f32": 4, "q8_0": 1}[dtype]
        self.kv_dim = kv_dim
        self.n_layers = n_layers
        h = self._lib.ora_create(n_layers, kv_dim, n_tokens, codes[dtype])
        if not h:
            raise OracleError(5, "bad arguments")
        self._h = h
        self.n_blocks = self._lib.ora_n_blocks(h)

    def __del__(self):
        h = getattr(self, "_h", None)
        if h:
            self._lib.ora_destroy(h)
            self._h = None

    def _raise(self, rc: int):
        raise OracleError(rc, self._lib.ora_last_error().decode())

    # -- kv.rs:50-60,185-187
    def capacity(self) -> int:
        return self._lib.ora_capacity(self._h)

    def bytes(self) -> int:
        return self._lib.ora_bytes(self._h)

    def len(self, seq: int) -> int:
        return self._lib.ora_len(self._h, seq)

    def free_blocks(self) -> int:
        return self._lib.ora_free_blocks(self._h)

    def refcount(self, block: int) -> int:
        return self._lib.ora_refcount(self._h, block)

    def cow_copies(self) -> int:
        return self._lib.ora_cow_copies(self._h)

    def has_seq(self, seq: int) -> bool:
        return bool(self._lib.ora_has_seq(self._h, seq))

    def init_free_order(self, order) -> None:
        o = np.ascontiguousarray(order, dtype=np.uint32)
        rc = self._lib.ora_init_free_order(self._h, _ptr(o), o.size)
        if rc:
            raise OracleError(rc, "init_free_order needs a full permutation on a fresh cache")

    # -- kv.rs:85-121
    def append(self, seq: int, pos: int):
        b, s = C.c_uint32(), C.c_uint32()
        rc = self._lib.ora_append(self._h, seq, pos, C.byref(b), C.byref(s))
        if rc:
            self._raise(rc)
        return b.value, s.value

    def append_batch(self, seqs, positions):
        seqs = np.ascontiguousarray(seqs, dtype=np.uint32)
        pos = np.ascontiguousarray(positions, dtype=np.uint64)
        out = np.full(seqs.size, -1, dtype=np.int32)
        done = C.c_size_t()
        rc = self._lib.ora_append_batch(self._h, seqs.size, _ptr(seqs), _ptr(pos), _ptr(out), C.byref(done))
        if rc:
            err = OracleError(rc, self._lib.ora_last_error().decode())
            err.n_done = done.value
            err.slot_mapping = out
            raise err
        return out

    # -- kv.rs:123-131
    def write(self, layer: int, block: int, slot: int, k, v) -> None:
        k = np.ascontiguousarray(k, dtype=np.float32)
        v = np.ascontiguousarray(v, dtype=np.float32)
        assert k.size == self.kv_dim and v.size == self.kv_dim
        self._lib.ora_write(self._h, layer, block, slot, _ptr(k), _ptr(v))

    def write_batch(self, layer: int, slot_mapping, k, v) -> None:
        sm = np.ascontiguousarray(slot_mapping, dtype=np.int32)
        k = np.ascontiguousarray(k, dtype=np.float32)
        v = np.ascontiguousarray(v, dtype=np.float32)
        assert k.shape == (sm.size, self.kv_dim) and v.shape == k.shape
        self._lib.ora_write_batch(self._h, layer, sm.size, _ptr(sm), _ptr(k), _ptr(v))

    # -- model.rs:291-308 + 414-429: RoPE on q (in place) and k, then write
    def write_rope_batch(self, layer: int, slot_mapping, positions, k, v, base: float, rope_dim: int,
                         head_dim: int, neox: bool, q=None, n_heads: int = 0) -> None:
        sm = np.ascontiguousarray(slot_mapping, dtype=np.int32)
        pos = np.ascontiguousarray(positions, dtype=np.int32)
        k = np.ascontiguousarray(k, dtype=np.float32)
        v = np.ascontiguousarray(v, dtype=np.float32)
        assert k.shape == (sm.size, self.kv_dim) and v.shape == k.shape and pos.shape == sm.shape
        qp, qs = None, 0
        if q is not None:
            assert q.dtype == np.float32 and q.flags.c_contiguous and q.shape[0] == sm.size
            qp, qs = _ptr(q), q.shape[1]
        self._lib.ora_write_rope_batch(self._h, layer, sm.size, _ptr(sm), _ptr(pos), _ptr(k), _ptr(v), qp,
                                       qs, n_heads, float(base), rope_dim, head_dim, 1 if neox else 0)

    # -- kv.rs:133-150 (collected)
    def rows(self, layer: int, seq: int, n: int):
        dt = {1: np.int8, 2: np.uint16, 4: np.float32}[self.elem]
        k = np.empty((n, self.kv_dim), dtype=dt)
        v = np.empty((n, self.kv_dim), dtype=dt)
        rc = self._lib.ora_rows(self._h, layer, seq, n, _ptr(k), _ptr(v))
        if rc:
            self._raise(rc)
        return k, v

    def block_table(self, seq: int) -> np.ndarray:
        n = C.c_size_t()
        self._lib.ora_block_table(self._h, seq, None, 0, C.byref(n))
        out = np.empty(n.value, dtype=np.int32)
        rc = self._lib.ora_block_table(self._h, seq, _ptr(out), out.size, C.byref(n))
        if rc:
            self._raise(rc)
        return out

    # -- kv.rs:153-183
    def copy_blocks(self, pairs) -> int:
        """The copy-on-write body (kv.rs:99-110) for (src, dst) block pairs."""
        pairs = np.ascontiguousarray(pairs, dtype=np.int32).reshape(-1, 2)
        return int(self._lib.ora_copy_blocks(self._h, pairs.shape[0], _ptr(pairs)))

    def truncate(self, seq: int, from_: int) -> None:
        self._lib.ora_truncate(self._h, seq, from_)

    def share(self, src: int, dst: int, length: int) -> None:
        self._lib.ora_share(self._h, src, dst, length)

    def pool(self, layer: int = 0):
        dt = {1: np.int8, 2: np.uint16, 4: np.float32}[self.elem]
        shape = (self.n_blocks, BLOCK, self.kv_dim)
        k = np.empty(shape, dtype=dt)
        v = np.empty(shape, dtype=dt)
        self._lib.ora_pool(self._h, layer, _ptr(k), _ptr(v))
        return k, v

    def load_pool(self, layer, k, v) -> None:
        dt = {1: np.int8, 2: np.uint16, 4: np.float32}[self.elem]
        shape = (self.n_blocks, BLOCK, self.kv_dim)
        k = np.ascontiguousarray(k, dtype=dt).reshape(shape)
        v = np.ascontiguousarray(v, dtype=dt).reshape(shape)
        self._lib.ora_load_pool(self._h, layer, _ptr(k), _ptr(v))

    def scales(self, layer: int = 0):
        """Q8_0 scale pools of one layer, [n_blocks][16][kv_dim/32] f16 bits."""
        shape = (self.n_blocks, BLOCK, self.kv_dim // 32)
        k = np.empty(shape, dtype=np.uint16)
        v = np.empty(shape, dtype=np.uint16)
        rc = self._lib.ora_scales(self._h, layer, _ptr(k), _ptr(v))
        if rc:
            self._raise(rc)
        return k, v

    def load_scales(self, layer, k, v) -> None:
        shape = (self.n_blocks, BLOCK, self.kv_dim // 32)
        k = np.ascontiguousarray(k, dtype=np.uint16).reshape(shape)
        v = np.ascontiguousarray(v, dtype=np.uint16).reshape(shape)
        rc = self._lib.ora_load_scales(self._h, layer, _ptr(k), _ptr(v))
        if rc:
            self._raise(rc)

    # -- model.rs:431-475
    def attention(self, layer, seqs, positions, q, n_heads, head_dim, scale=None, threads=1):
        seqs = np.ascontiguousarray(seqs, dtype=np.uint32)
        pos = np.ascontiguousarray(positions, dtype=np.uint64)
        q = np.ascontiguousarray(q, dtype=np.float32)
        n = seqs.size
        assert q.shape == (n, n_heads * head_dim)
        out = np.empty_like(q)
        scale = float(1.0 / np.sqrt(np.float32(head_dim))) if scale is None else scale
        rc = self._lib.ora_attention(self._h, layer, n, _ptr(seqs), _ptr(pos), n_heads, head_dim,
                                     C.c_float(scale), _ptr(q), _ptr(out), threads)
        if rc:
            raise OracleError(rc, "attention: bad arguments or table too short")
        return out

    def attention_tables(self, layer, tables, lens, q, n_heads, head_dim, scale=None, threads=1):
        tables = np.ascontiguousarray(tables, dtype=np.int32)
        lens = np.ascontiguousarray(lens, dtype=np.int32)
        q = np.ascontiguousarray(q, dtype=np.float32)
        n = lens.size
        assert q.shape == (n, n_heads * head_dim) and tables.shape[0] == n
        out = np.empty_like(q)
        scale = float(1.0 / np.sqrt(np.float32(head_dim))) if scale is None else scale
        rc = self._lib.ora_attention_tables(self._h, layer, n, _ptr(tables), tables.shape[1], _ptr(lens),
                                            n_heads, head_dim, C.c_float(scale), _ptr(q), _ptr(out), threads)
        if rc:
            raise OracleError(rc, "attention_tables: bad arguments or table too short")
        return out
