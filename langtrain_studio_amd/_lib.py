"""ctypes binding of libltkv.so (the C ABI declared in include/ltkv.h).

The library is built in-tree by ``python -m langtrain_studio_amd.build``.
There is no fallback: if it is missing, importing this module fails.
"""

from __future__ import annotations

import ctypes as C
import os

LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "libltkv.so")

OK, ERR_FULL, ERR_NONCONTIG, ERR_RANGE, ERR_HIP, ERR_ARG = 0, 1, 2, 3, 4, 5
F16, F32, Q8_0 = 0, 1, 2
PLAN_SHARED_PREFIX, PLAN_F16_PRODUCTS = 1, 2
ENGINE_AUTO, ENGINE_VALU = 0, 1
NO_DEVICE = -1
BLOCK = 16
NOALLOC_SCRATCH_BYTES = 32 << 20  # LTKV_NOALLOC_SCRATCH_BYTES

_sz, _u32, _i32, _u64, _vp, _int, _f32 = (C.c_size_t, C.c_uint32, C.c_int32, C.c_uint64, C.c_void_p,
                                          C.c_int, C.c_float)
_P = C.POINTER

# name -> (restype, argtypes); mirrors include/ltkv.h one to one.
SIGNATURES = {
    "ltkv_last_error": (C.c_char_p, []),
    "ltkv_create": (_int, [_sz, _sz, _sz, _int, _int, _P(_vp)]),
    "ltkv_destroy": (None, [_vp]),
    "ltkv_set_stream": (_int, [_vp, _vp]),
    "ltkv_capacity": (_sz, [_vp]),
    "ltkv_bytes": (_sz, [_vp]),
    "ltkv_len": (_sz, [_vp, _u32]),
    "ltkv_free_blocks": (_sz, [_vp]),
    "ltkv_n_blocks": (_sz, [_vp]),
    "ltkv_kv_dim": (_sz, [_vp]),
    "ltkv_refcount": (_u32, [_vp, _u32]),
    "ltkv_cow_copies": (_u64, [_vp]),
    "ltkv_append": (_int, [_vp, _u32, _sz, _P(_u32), _P(_u32)]),
    "ltkv_append_batch": (_int, [_vp, _sz, _vp, _vp, _vp, _P(_sz)]),
    "ltkv_truncate": (None, [_vp, _u32, _sz]),
    "ltkv_share": (None, [_vp, _u32, _u32, _sz]),
    "ltkv_block_table": (_int, [_vp, _u32, _vp, _sz, _P(_sz)]),
    "ltkv_block_tables": (_int, [_vp, _sz, _vp, _vp, _sz]),
    "ltkv_init_free_order": (_int, [_vp, _vp, _sz]),
    "ltkv_write": (_int, [_vp, _sz, _sz, _vp, _vp, _vp, _sz]),
    "ltkv_cell_order": (_int, [_vp, _sz, _vp, _vp, _P(_sz)]),
    "ltkv_write_ordered": (_int, [_vp, _sz, _sz, _vp, _vp, _vp, _sz, _sz, _vp]),
    "ltkv_rope_init": (_int, [_vp, _f32, _sz, _sz, _int, _sz]),
    "ltkv_write_rope": (_int, [_vp, _sz, _sz, _vp, _vp, _vp, _vp, _sz, _vp, _sz, _sz]),
    "ltkv_copy_blocks": (_int, [_vp, _sz, _vp]),
    "ltkv_gather": (_int, [_vp, _sz, _sz, _vp, _sz, _vp, _vp, _vp, _vp]),
    "ltkv_decode_attention": (_int, [_vp, _sz, _sz, _sz, _sz, _f32, _vp, _vp, _sz, _vp, _vp]),
    "ltkv_decode_attention_noalloc": (_int, [_vp, _sz, _sz, _sz, _sz, _f32, _vp, _vp, _sz, _vp, _vp]),
    "ltkv_append_decode_attention": (_int, [_vp, _sz, _sz, _sz, _sz, _f32, _vp, _vp, _sz, _vp, _vp, _vp, _vp,
                                            _sz, _vp]),
    "ltkv_set_attention_partition": (_int, [_vp, _sz]),
    "ltkv_set_attention_engine": (_int, [_vp, _int]),
    "ltkv_plan_attention": (_int, [_vp, _sz, _vp, _vp, _sz, _sz, _u32]),
    "ltkv_planned_attention": (_int, [_vp, _sz, _f32, _vp, _vp]),
    "ltkv_plan_stats": (_int, [_vp, _vp]),
    "ltkv_read_pool": (_int, [_vp, _sz, _vp, _vp]),
    "ltkv_read_scales": (_int, [_vp, _sz, _vp, _vp]),
    "ltkv_rows": (_int, [_vp, _sz, _u32, _sz, _vp, _vp]),
    "ltkv_write_row": (_int, [_vp, _sz, _u32, _u32, _vp, _vp]),
    "ltkv_synchronize": (_int, [_vp]),
    "ltkv_seq_rows": (_int, [_vp, _sz, _vp, _vp]),
    "ltkv_sync_tables": (_int, [_vp]),
    "ltkv_resident_tables": (_int, [_vp, _P(_vp), _P(_vp), _P(_sz), _P(_sz)]),
    "ltkv_slot_mapping": (_int, [_vp, _sz, _vp, _vp, _vp]),
    "ltkv_decode_attention_rows": (_int, [_vp, _sz, _sz, _sz, _sz, _f32, _vp, _vp, _vp, _vp]),
    "ltkv_table_uploads": (_int, [_vp, _P(_u64)]),
    "ltkv_read_resident_tables": (_int, [_vp, _vp, _vp]),
}

_lib = None


def load() -> C.CDLL:
    """Load libltkv.so from the package directory (raises if it is not built)."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise ImportError(
            f"{LIB_PATH} is missing: build it with `python -m langtrain_studio_amd.build` "
            "(hipcc, gfx950). There is no fallback implementation.")
    lib = C.CDLL(LIB_PATH)
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    _lib = lib
    return lib


def last_error() -> str:
    return load().ltkv_last_error().decode(errors="replace")
