"""Build libmbq.so in-tree for gfx950 with hipcc (no JIT cache: the built library travels with the source tree).

    python -m mashbox_amd.build        # or __graft_entry__.build()
"""
from __future__ import annotations

import concurrent.futures
import os
import shutil
import subprocess
import sys
import tempfile
import time

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
LIB = os.path.join(HERE, "libmbq.so")
SOURCES = ["mbq_kernels.hip", "mbq_gemv.hip", "mbq_tgemv.hip", "mbq_gemm.hip", "mbq_wsgemm.hip", "mbq_kgemm.hip", "mbq_probe.hip", "mbq_abi.cpp"]
ARCH = os.environ.get("MBQ_OFFLOAD_ARCH", "gfx950")


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found: the HIP toolchain is needed to build libmbq.so")


FLAGS = ["-O3", "-std=c++17", "-fPIC",
         # no packed FP32 (v_pk_*_f32) in the device code
         "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
         "-Wall", "-Wno-unused-function", "-Wno-unknown-warning-option"]


def command(out: str = LIB) -> list[str]:
    """one hipcc line that compiles and links every source (the parallel build below runs the same flags per file)"""
    return [hipcc(), f"--offload-arch={ARCH}", *FLAGS, "-shared", *[os.path.join(CSRC, s) for s in SOURCES], "-o", out]


def _run(cmd: list[str]) -> str:
    r = subprocess.run(cmd, cwd=CSRC, capture_output=True, text=True)
    if r.returncode != 0:
        sys.stderr.write(r.stdout + r.stderr)
        raise RuntimeError(f"hipcc failed ({r.returncode}): {' '.join(cmd[-3:])}")
    return "\n".join(l for l in (r.stdout + r.stderr).splitlines() if "packed-fp32-ops" not in l and l.strip())


def build(verbose: bool = True) -> str:
    """compile libmbq.so (every call compiles every source, one hipcc per source in parallel); returns its path"""
    t0 = time.time()
    tmpdir = tempfile.mkdtemp(prefix="mbq_build_")
    try:
        objs = [os.path.join(tmpdir, os.path.splitext(s)[0] + ".o") for s in SOURCES]
        cmds = [[hipcc(), f"--offload-arch={ARCH}", *FLAGS, "-c", os.path.join(CSRC, s), "-o", o] for s, o in zip(SOURCES, objs)]
        jobs = max(1, min(len(cmds), os.cpu_count() or 1, 16))
        with concurrent.futures.ThreadPoolExecutor(jobs) as ex:
            warns = list(ex.map(_run, cmds))
        tmp = LIB + f".tmp{os.getpid()}"
        warns.append(_run([hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", *objs, "-o", tmp]))
        os.replace(tmp, LIB)
    finally:
        shutil.rmtree(tmpdir, ignore_errors=True)
    warn = "\n".join(w for w in warns if w)
    if verbose and warn:
        sys.stderr.write(warn + "\n")
    if verbose:
        print(f"built {LIB} for {ARCH} in {time.time() - t0:.1f}s", flush=True)
    return LIB


if __name__ == "__main__":
    build()
