"""The kernels that issue v_mfma through inline asm (mfma_acc / mfma32_acc in mbq_device.h: mbq_gemm.hip's specialized
kernel) pin their accumulators the compiler cannot see as MFMA results, so the compiler inserts no wait
states after them. This test compiles the sources to gfx950 assembly (hipcc, no GPU) and checks that within 20 wait
states after every MFMA (one per instruction, N + 1 per s_nop N) no non-MFMA instruction reads or writes its
destination registers: the copies the compiler may place at loop edges must come after the kernels' mfma_drain."""
import os
import re
import shutil
import subprocess
import tempfile
from concurrent.futures import ThreadPoolExecutor

import pytest

CSRC = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "mashbox_amd", "csrc")
HIPCC = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
WINDOW = 20


def _asm(src: str, out: str) -> str:
    cmd = [HIPCC, "--offload-arch=gfx950", "-O3", "-std=c++17", "-fPIC", "--cuda-device-only", "-S",
           "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops", os.path.join(CSRC, src), "-o", out]
    r = subprocess.run(cmd, cwd=CSRC, capture_output=True, text=True)
    assert r.returncode == 0, r.stderr[-2000:]
    return open(out).read()


def _regs(tok: str):
    s = set()
    for m in re.finditer(r"\b([av])\[(\d+):(\d+)\]", tok):
        s |= {(m.group(1), i) for i in range(int(m.group(2)), int(m.group(3)) + 1)}
    for m in re.finditer(r"(?<![\w\[:])([av])(\d+)\b", tok):
        s.add((m.group(1), int(m.group(2))))
    return s


def _hazards(text: str, kernel_substr: str):
    """(kernels checked, MFMAs checked, violations) over the kernels whose symbol contains kernel_substr"""
    lines = text.splitlines()
    kernels = mfmas = 0
    bad = []
    for st, l in enumerate(lines):
        m = re.match(r"^(_ZN3mbq\S*:)", l)
        if not m or kernel_substr not in m.group(1):
            continue
        kernels += 1
        end = st
        while not lines[end].startswith(".Lfunc_end"):
            end += 1
        body = [x.strip() for x in lines[st + 1:end]]
        body = [x for x in body if x and not x.startswith(";") and not (x.startswith(".") and not x.startswith(".LBB"))]
        for k, ins in enumerate(body):
            if not ins.startswith("v_mfma"):
                continue
            mfmas += 1
            dst = _regs(ins.split(None, 1)[1].split(",")[0])
            ws, j = 0, k + 1
            while j < len(body) and ws < WINDOW:
                x = body[j]
                j += 1
                if x.startswith(".LBB"):
                    continue
                op = x.split()[0]
                if op == "s_nop":
                    ws += int(x.split()[1]) + 1
                    continue
                if not op.startswith("v_mfma") and not op.startswith("s_") and _regs(x) & dst:
                    bad.append((m.group(1)[:60], ins, x, ws))
                    break
                ws += 1
    return kernels, mfmas, bad


@pytest.mark.skipif(not os.path.exists(HIPCC), reason="hipcc is needed to compile the kernels to assembly")
def test_asm_mfma_results_are_never_read_early():
    with tempfile.TemporaryDirectory() as d:
        jobs = {"mbq_gemm.hip": "sgemm_kernel"}
        with ThreadPoolExecutor(len(jobs)) as ex:
            texts = dict(zip(jobs, ex.map(lambda s: _asm(s, os.path.join(d, s + ".s")), jobs)))
    for src, kern in jobs.items():
        kernels, mfmas, bad = _hazards(texts[src], kern)
        assert kernels >= 6 and mfmas > 0, (src, kernels, mfmas)
        assert not bad, f"{src}: {len(bad)} MFMA results read within {WINDOW} wait states, first {bad[0]}"
