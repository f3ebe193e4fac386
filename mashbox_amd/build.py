"""Build libmbq.so in-tree for gfx950 with hipcc (no JIT cache: the built library travels with the source tree).

    python -m mashbox_amd.build        # or __graft_entry__.build()
"""
from __future__ import annotations

import os
import shutil
import subprocess
import sys
import time

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
LIB = os.path.join(HERE, "libmbq.so")
SOURCES = ["mbq_kernels.hip", "mbq_gemv.hip", "mbq_gemm.hip", "mbq_wsgemm.hip", "mbq_abi.cpp"]
ARCH = os.environ.get("MBQ_OFFLOAD_ARCH", "gfx950")


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found: the HIP toolchain is needed to build libmbq.so")


def command(out: str = LIB) -> list[str]:
    return [hipcc(), f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC", "-shared",
            # no packed FP32 (v_pk_*_f32) in the device code
            "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
            "-Wall", "-Wno-unused-function", "-Wno-unknown-warning-option",
            *[os.path.join(CSRC, s) for s in SOURCES], "-o", out]


def build(verbose: bool = True) -> str:
    """compile libmbq.so (every call compiles); returns its path"""
    tmp = LIB + f".tmp{os.getpid()}"
    cmd = command(tmp)
    t0 = time.time()
    r = subprocess.run(cmd, cwd=CSRC, capture_output=True, text=True)
    if r.returncode != 0:
        sys.stderr.write(r.stdout + r.stderr)
        raise RuntimeError(f"hipcc failed ({r.returncode}) building libmbq.so")
    warn = "\n".join(l for l in (r.stdout + r.stderr).splitlines() if "packed-fp32-ops" not in l and l.strip())
    if verbose and warn:
        sys.stderr.write(warn + "\n")
    os.replace(tmp, LIB)
    if verbose:
        print(f"built {LIB} for {ARCH} in {time.time() - t0:.1f}s", flush=True)
    return LIB


if __name__ == "__main__":
    build()
