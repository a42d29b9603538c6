"""CPU oracle for the paged KV-cache path (test infrastructure only).

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg import
this package; the product (langtrain_studio_amd) never does. See
ltkv_oracle.cpp for the reference file:line each function restates.
"""

from .oracle import (OracleError, OracleKv, f16_to_f32, f32_to_f16, has_f16c, load,  # noqa: F401
                     pool_selftest, quantize_block)
