"""MI355X-native paged KV cache for the Langtrain engine.

The product is libltkv.so (HIP kernels for gfx950 + the host block manager,
C ABI in include/ltkv.h). This package is its Python face:

* ``kv.KvCache`` mirrors ``langtrain_native::kv::KvCache``
  (engine/crates/native/src/kv.rs:15-188);
* ``backend.PagedKvBackend`` mirrors the KV part of ``NativeBackend``
  (engine/crates/native/src/lib.rs:136-198) and the KV segment of
  ``Model::forward`` (engine/crates/native/src/model.rs:380-475).
"""

from .kv import BLOCK, KvCache, KvCacheFull, KvError, NonContiguous  # noqa: F401
from .backend import BatchToken, PagedKvBackend, StepPlan  # noqa: F401

__all__ = ["BLOCK", "KvCache", "KvCacheFull", "KvError", "NonContiguous", "BatchToken",
           "PagedKvBackend", "StepPlan"]
