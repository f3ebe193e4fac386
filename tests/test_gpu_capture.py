"""The split-K workspace and HIP graph capture, in a fresh process.

mbq_matmul allocates its split-K workspace on the first call that splits K on a device. An allocation cannot be
recorded into a graph, so in a fresh process whose first split-K call is made on a stream that is capturing, the call
returns an error that says so and launches nothing; after one eager call, the same call records into a graph and every
replay equals the eager result bit for bit. A fresh process is needed because the workspace lives until the process
ends (the test runner's own process has long allocated it).
"""
import os
import subprocess
import sys

import pytest

pytestmark = pytest.mark.gpu

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))

SCRIPT = r"""
import sys
sys.path.insert(0, sys.argv[1])
import numpy as np
import torch
from oracle import gen as G
import mashbox_amd.kernels as KQ
from mashbox_amd import _lib as LIB

dev = torch.device("cuda", 0)
rng = np.random.default_rng(5)
n, k, m = 1024, 5120, 16
print("case: Q4_K 16 x 1024 x 5120, first split-K call under capture", flush=True)
planes = KQ.repack_host(12, G.q4_k_raw(rng, n, k), (n, k)).to(dev)
assert LIB.gemm_plan(12, m, n, k)[3] > 1, "the case must split K"
x = torch.from_numpy(G.acts(rng, m, k).astype(np.int16)).view(torch.bfloat16).to(dev)
torch.cuda.synchronize()
g = torch.cuda.CUDAGraph()
err = ""
try:
    with torch.cuda.graph(g):
        KQ.matmul(x, planes)
except LIB.MbqError as e:
    err = str(e)
assert "eager call first" in err, f"expected the capture refusal, got {err!r}"
del g
torch.cuda.synchronize()
eager = KQ.matmul(x, planes)
torch.cuda.synchronize()
g = torch.cuda.CUDAGraph()
with torch.cuda.graph(g):
    y = KQ.matmul(x, planes)
for _ in range(3):
    g.replay()
    torch.cuda.synchronize()
    assert torch.equal(y.view(torch.int32), eager.view(torch.int32)), "replay differs from the eager call"
    KQ.matmul(x, planes)
    torch.cuda.synchronize()
print("capture ok", flush=True)
"""


def test_first_split_k_call_under_capture_is_refused_then_captures():
    r = subprocess.run([sys.executable, "-c", SCRIPT, ROOT], capture_output=True, text=True, timeout=240)
    sys.stdout.write(r.stdout)
    sys.stderr.write(r.stderr[-4000:])
    assert r.returncode == 0 and "capture ok" in r.stdout


TGEMV_SCRIPT = r"""
import sys
sys.path.insert(0, sys.argv[1])
import numpy as np
import torch
from oracle import gen as G
import mashbox_amd.kernels as KQ
from mashbox_amd import _lib as LIB

dev = torch.device("cuda", 0)
rng = np.random.default_rng(6)
for t, n, k in ((12, 5120, 6144), (14, 17408, 5120), (8, 1000, 2048)):
    print(f"case: type {t} tiles 1 x {n} x {k}, the tile GEMV's first call under capture", flush=True)
    planes = KQ.repack_host(t, G.RAW[t](rng, n, k), (n, k), tiled=True).to(dev)
    assert LIB.gemm_plan(planes.t, 1, n, k)[0] == LIB.KERNEL_GEMV
    x = torch.from_numpy(G.acts(rng, 1, k).astype(np.int16)).view(torch.bfloat16).to(dev)
    x2 = torch.from_numpy(G.acts(rng, 1, k).astype(np.int16)).view(torch.bfloat16).to(dev)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        y = KQ.matmul(x, planes, out_dtype=torch.bfloat16)
    torch.cuda.synchronize()
    eager = KQ.matmul(x, planes, out_dtype=torch.bfloat16)
    for _ in range(3):
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(y.view(torch.int16), eager.view(torch.int16)), "replay differs from the eager call"
        KQ.matmul(x2, planes, out_dtype=torch.bfloat16)
        torch.cuda.synchronize()
print("tile GEMV capture ok", flush=True)
"""


def test_tile_gemv_first_call_under_capture():
    """the tile GEMV needs no workspace: in a fresh process its first call (which raises the kernel's LDS limit) records
    into a HIP graph, and every replay equals the eager call bit for bit, with eager calls of other inputs between"""
    r = subprocess.run([sys.executable, "-c", TGEMV_SCRIPT, ROOT], capture_output=True, text=True, timeout=240)
    sys.stdout.write(r.stdout)
    sys.stderr.write(r.stderr[-4000:])
    assert r.returncode == 0 and "tile GEMV capture ok" in r.stdout
