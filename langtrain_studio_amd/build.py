"""Build recipe for libltkv.so (HIP kernels + host block manager, gfx950).

Run as ``python -m langtrain_studio_amd.build``. Cross-compiles without a GPU.
"""

from __future__ import annotations

import os
import shlex
import subprocess
import sys

PKG = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(PKG, "csrc")
LIB = os.path.join(PKG, "libltkv.so")
SOURCES = [os.path.join(CSRC, "ltkv_cache.cpp"), os.path.join(CSRC, "ltkv_kernels.hip")]
HEADERS = [os.path.join(CSRC, "ltkv_kernels.h"), os.path.join(os.path.dirname(PKG), "include", "ltkv.h")]

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = "gfx950"
# Packed FP32 (v_pk_*_f32) is disabled for all device code. MFMA operands and
# results live in VGPRs: with AGPR accumulators the decode attention kernel
# copied its 32 accumulators between AGPRs and VGPRs on every tile.
DEVICE_FLAGS = ["-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops", "-mllvm", "-amdgpu-mfma-vgpr-form"]
COMMON = ["-O3", "-std=c++17", "-fPIC", "-fvisibility=hidden", "-Wall", "-Wno-unused-command-line-argument"]


VERSION_SCRIPT = os.path.join(CSRC, "ltkv.map")


def command() -> list[str]:
    return [HIPCC, f"--offload-arch={ARCH}", *COMMON, *DEVICE_FLAGS, "-shared",
            f"-Wl,--version-script={VERSION_SCRIPT}", "-o", LIB, *SOURCES]


def build(verbose: bool = True) -> str:
    """Compile every source into libltkv.so (always recompiles)."""
    cmd = command()
    if verbose:
        print("+", " ".join(shlex.quote(c) for c in cmd), flush=True)
    tmp = LIB + ".tmp"
    cmd[cmd.index(LIB)] = tmp
    res = subprocess.run(cmd, capture_output=True, text=True)
    # hipcc's host pass warns that it does not know the packed-fp32 feature: harmless.
    noise = ("packed-fp32-ops", "not a recognized feature", "warning: unknown target feature")
    err = "\n".join(l for l in res.stderr.splitlines() if not any(n in l for n in noise))
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed ({res.returncode}):\n{err}")
    if verbose and err.strip():
        print(err, file=sys.stderr)
    os.replace(tmp, LIB)
    return LIB


if __name__ == "__main__":
    build()
