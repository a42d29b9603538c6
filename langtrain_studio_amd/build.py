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
# The profiling build: the same sources with -DLTKV_TIMELINE (per-wave phase
# stamps of the decode kernel, ltkv_timeline_read), for bench.py's timeline
# workloads; the product never loads it.
TIMELINE_LIB = os.path.join(PKG, "libltkv_timeline.so")
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


def command(timeline: bool = False) -> list[str]:
    out = TIMELINE_LIB if timeline else LIB
    return [HIPCC, f"--offload-arch={ARCH}", *COMMON, *DEVICE_FLAGS, *(["-DLTKV_TIMELINE"] if timeline else []),
            "-shared", f"-Wl,--version-script={VERSION_SCRIPT}", "-o", out, *SOURCES]


def build(verbose: bool = True, timeline: bool = True) -> str:
    """Compile every source into libltkv.so (always recompiles), and the
    profiling build libltkv_timeline.so beside it (in parallel)."""
    jobs = []
    for tl in ((False, True) if timeline else (False,)):
        cmd = command(tl)
        out = TIMELINE_LIB if tl else LIB
        if verbose:
            print("+", " ".join(shlex.quote(c) for c in cmd), flush=True)
        tmp = out + ".tmp"
        cmd[cmd.index(out)] = tmp
        jobs.append((subprocess.Popen(cmd, stderr=subprocess.PIPE, stdout=subprocess.DEVNULL, text=True), tmp, out))
    # hipcc's host pass warns that it does not know the packed-fp32 feature: harmless.
    noise = ("packed-fp32-ops", "not a recognized feature", "warning: unknown target feature")
    failed = []
    for proc, tmp, out in jobs:
        stderr = proc.communicate()[1]
        err = "\n".join(l for l in stderr.splitlines() if not any(n in l for n in noise))
        if proc.returncode != 0:
            failed.append(f"hipcc failed ({proc.returncode}) for {os.path.basename(out)}:\n{err}")
            continue
        if verbose and err.strip():
            print(err, file=sys.stderr)
        os.replace(tmp, out)
    if failed:
        raise RuntimeError("\n".join(failed))
    return LIB


if __name__ == "__main__":
    build(timeline="--no-timeline" not in sys.argv[1:])
