"""mbq_matmul_noalloc, through the C ABI: the entry point that allocates nothing (its split-K partials live in the
library's static scratch array) equals mbq_matmul bit for bit on the same inputs, and both meet the product bars against
the oracle's exact weights. Two calls in a row, the second with a smaller input, each splitting K (LDS tiles, then the
weight stream); a decode call that needs no scratch; and a forced plan whose partials exceed the scratch, which the
entry point refuses with an error while mbq_matmul (whose workspace is larger) runs it.
"""
import ctypes

import numpy as np
import pytest
import torch

from oracle import gen as G
from oracle import ref as R
from tests._check import assert_product_dev

from mashbox_amd import _lib as LIB

pytestmark = pytest.mark.gpu

CASES = [  # (type, activation rows, weight rows, K): the second smaller than the first
    (R.Q8_0, 64, 17408, 5120),      # LDS tiles 64 x 128, K in 3 ranges: 13.4 MB of partials
    (R.Q4_K, 16, 1024, 5120),       # weight stream, K in 8 ranges
    (R.Q5_K, 4, 5120, 17408),       # decode rows too long for the GEMV: weight stream, K in 3 ranges
    (R.Q6_K, 1, 2048, 2560),        # decode GEMV: no scratch
]


def _call(fn, t, planes, x, m, n, k, y):
    return fn(t, ctypes.c_void_p(planes.data_ptr()), 0, None, 1, ctypes.c_void_p(x.data_ptr()), m, n, k,
              ctypes.c_void_p(y.data_ptr()), LIB.OUT_F32, ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))


def _case(t, m, n, k, seed, dev):
    rng = np.random.default_rng(seed)
    raw = G.RAW[t](rng, n, k)
    pb = LIB.check(LIB.lib().mbq_plane_bytes(t, n, k), "plane_bytes")
    host = torch.empty(pb, dtype=torch.uint8)
    LIB.check(LIB.lib().mbq_repack_host(t, raw.ctypes.data_as(ctypes.c_void_p), n, k, ctypes.c_void_p(host.data_ptr()),
                                        pb, 0), "repack_host")
    xb = G.acts(rng, m, k)
    x = torch.from_numpy(xb.astype(np.int16)).view(torch.bfloat16).to(dev)
    w64 = torch.from_numpy(R.dequant(raw, t, k)).to(dev).to(torch.float64)
    return host.to(dev), x, x.to(torch.float64) @ w64.T


def test_noalloc_equals_matmul_on_consecutive_calls():
    dev = torch.device("cuda", 0)
    L = LIB.lib()
    for i, (t, m, n, k) in enumerate(CASES):
        print(f"case {i}: type {t} {m}x{n}x{k} plan {LIB.plan_str(t, m, n, k)}", flush=True)
        if i < 3:
            assert LIB.gemm_plan(t, m, n, k)[3] > 1, "the case must split K"
        planes, x, ref = _case(t, m, n, k, 100 + i, dev)
        y_ref = torch.full((m, n), float("nan"), dtype=torch.float32, device=dev)
        y = torch.full((m, n), float("nan"), dtype=torch.float32, device=dev)
        LIB.check(_call(L.mbq_matmul, t, planes, x, m, n, k, y_ref), "mbq_matmul")
        LIB.check(_call(L.mbq_matmul_noalloc, t, planes, x, m, n, k, y), "mbq_matmul_noalloc")
        torch.cuda.synchronize()
        assert torch.equal(y.view(torch.int32), y_ref.view(torch.int32)), f"case {i}: noalloc differs from mbq_matmul"
        assert_product_dev(y, ref, f"case {i}")
        # the same call again: the scratch keeps the last call's contents, and the arrival counters are back at zero
        y.fill_(float("nan"))
        LIB.check(_call(L.mbq_matmul_noalloc, t, planes, x, m, n, k, y), "mbq_matmul_noalloc again")
        torch.cuda.synchronize()
        assert torch.equal(y.view(torch.int32), y_ref.view(torch.int32)), f"case {i}: a repeated call differs"


def test_noalloc_refuses_a_plan_beyond_its_scratch():
    """the scratch holds as many partials as the allocated workspace (every automatic plan fits both), so a forced plan
    beyond it is refused by both entry points with nothing launched; the automatic plan then runs in both, bit for bit
    alike"""
    dev = torch.device("cuda", 0)
    L = LIB.lib()
    t, m, n, k = R.Q8_0, 512, 17408, 1024
    planes, x, ref = _case(t, m, n, k, 7, dev)
    LIB.force_gemm_plan(LIB.KERNEL_TILES, 64, 64, 4)        # 2176 tiles x 4 ranges x 16 KiB = 142.6 MB of partials
    try:
        for fn in (L.mbq_matmul_noalloc, L.mbq_matmul):
            y = torch.full((m, n), float("nan"), dtype=torch.float32, device=dev)
            rc = _call(fn, t, planes, x, m, n, k, y)
            assert rc == -1 and b"does not fit" in L.mbq_last_error(), L.mbq_last_error()
            torch.cuda.synchronize()
            assert bool(torch.isnan(y).all()), "a refused call must launch nothing"
    finally:
        LIB.force_gemm_plan()
    y_ref = torch.full((m, n), float("nan"), dtype=torch.float32, device=dev)
    y = torch.full((m, n), float("nan"), dtype=torch.float32, device=dev)
    LIB.check(_call(L.mbq_matmul, t, planes, x, m, n, k, y_ref), "mbq_matmul")
    LIB.check(_call(L.mbq_matmul_noalloc, t, planes, x, m, n, k, y), "mbq_matmul_noalloc")
    torch.cuda.synchronize()
    assert torch.equal(y.view(torch.int32), y_ref.view(torch.int32))
    assert_product_dev(y, ref, f"automatic plan ({LIB.plan_str(t, m, n, k)})")


def test_noalloc_int8_planes_split_k():
    """tiled int8 planes at decode batches run the K-group kernel; with K splits its partials sit in the scratch too:
    two calls in a row (the second smaller), bit for bit equal to mbq_matmul and within the product bars"""
    dev = torch.device("cuda", 0)
    L = LIB.lib()
    for i, (m, n, k) in enumerate([(64, 5120, 17408), (40, 1024, 5120)]):
        plan = LIB.gemm_plan(LIB.I8T, m, n, k)
        print(f"int8 planes case {i}: {m}x{n}x{k} plan {plan}", flush=True)
        assert plan[0] == LIB.KERNEL_KGROUP and plan[3] > 1, "the case must split K"
        rng = np.random.default_rng(300 + i)
        q, s = G.int8_weights(rng, n, k)
        pb = LIB.check(L.mbq_plane_bytes(LIB.I8T, n, k), "plane_bytes")
        host = torch.empty(pb, dtype=torch.uint8)
        LIB.check(L.mbq_int8_repack_host(q.ctypes.data_as(ctypes.c_void_p), s.ctypes.data_as(ctypes.c_void_p), n, k,
                                         ctypes.c_void_p(host.data_ptr()), pb, 0), "int8 repack_host")
        planes = host.to(dev)
        xb = G.acts(rng, m, k)
        x = torch.from_numpy(xb.astype(np.int16)).view(torch.bfloat16).to(dev)
        ref = (x.to(torch.float64) @ torch.from_numpy(q).to(dev).to(torch.float64).T) * torch.from_numpy(s).to(dev).to(torch.float64)
        y_ref = torch.full((m, n), float("nan"), dtype=torch.float32, device=dev)
        y = torch.full((m, n), float("nan"), dtype=torch.float32, device=dev)
        LIB.check(_call(L.mbq_matmul, LIB.I8T, planes, x, m, n, k, y_ref), "mbq_matmul")
        LIB.check(_call(L.mbq_matmul_noalloc, LIB.I8T, planes, x, m, n, k, y), "mbq_matmul_noalloc")
        torch.cuda.synchronize()
        assert torch.equal(y.view(torch.int32), y_ref.view(torch.int32)), f"int8 case {i}: noalloc differs"
        assert_product_dev(y, ref, f"int8 planes case {i}")


CAPTURE_SCRIPT = r"""
import ctypes, sys
sys.path.insert(0, sys.argv[1])
import numpy as np
import torch
from oracle import gen as G
from oracle import ref as R
from mashbox_amd import _lib as LIB

dev = torch.device("cuda", 0)
L = LIB.lib()
t, m, n, k = R.Q4_K, 16, 1024, 5120
print(f"case: Q4_K {m} x {n} x {k}, first split-K call = mbq_matmul_noalloc under capture", flush=True)
assert LIB.gemm_plan(t, m, n, k)[3] > 1, "the case must split K"
rng = np.random.default_rng(11)
raw = G.q4_k_raw(rng, n, k)
pb = LIB.check(L.mbq_plane_bytes(t, n, k), "plane_bytes")
host = torch.empty(pb, dtype=torch.uint8)
LIB.check(L.mbq_repack_host(t, raw.ctypes.data_as(ctypes.c_void_p), n, k, ctypes.c_void_p(host.data_ptr()), pb, 0), "repack")
planes = host.to(dev)
x = torch.from_numpy(G.acts(rng, m, k).astype(np.int16)).view(torch.bfloat16).to(dev)
y = torch.full((m, n), float("nan"), dtype=torch.float32, device=dev)
def call(fn, out):
    return fn(t, ctypes.c_void_p(planes.data_ptr()), 0, None, 1, ctypes.c_void_p(x.data_ptr()), m, n, k,
              ctypes.c_void_p(out.data_ptr()), LIB.OUT_F32, ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
torch.cuda.synchronize()
g = torch.cuda.CUDAGraph()
with torch.cuda.graph(g):
    LIB.check(call(L.mbq_matmul_noalloc, y), "mbq_matmul_noalloc under capture")
torch.cuda.synchronize()
eager = torch.full_like(y, float("nan"))
for i in range(4):
    g.replay()
    torch.cuda.synchronize()
    if i == 0:
        LIB.check(call(L.mbq_matmul, eager), "mbq_matmul")        # the allocating entry point, after the capture
        torch.cuda.synchronize()
    assert torch.equal(y.view(torch.int32), eager.view(torch.int32)), f"replay {i} differs from mbq_matmul"
    y.fill_(float("nan"))
    other = torch.empty_like(y)
    LIB.check(call(L.mbq_matmul_noalloc, other), "eager mbq_matmul_noalloc between replays")
    torch.cuda.synchronize()
    assert torch.equal(other.view(torch.int32), eager.view(torch.int32)), "eager noalloc differs"
print("noalloc capture ok", flush=True)
"""


def test_noalloc_first_call_under_graph_capture():
    """in a fresh process (no workspace or scratch set up yet), the first split-K call is mbq_matmul_noalloc recorded
    into a HIP graph: it needs no allocation, so it records; every replay equals mbq_matmul's eager result bit for bit,
    with eager noalloc calls between the replays"""
    import os
    import subprocess
    import sys
    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    r = subprocess.run([sys.executable, "-c", CAPTURE_SCRIPT, root], capture_output=True, text=True, timeout=240)
    sys.stdout.write(r.stdout)
    sys.stderr.write(r.stderr[-4000:])
    assert r.returncode == 0 and "noalloc capture ok" in r.stdout


def test_noalloc_wide_batch_split():
    """batches of more than 64 rows whose automatic plan splits K (LDS tiles, partials of up to 64 MiB in the scratch):
    two calls in a row, the second smaller, bit for bit equal to mbq_matmul and within the product bars"""
    dev = torch.device("cuda", 0)
    L = LIB.lib()
    t, n, k = R.Q4_K, 6144, 5120
    for m in (256, 200):
        planes, x, ref = _case(t, m, n, k, 8, dev)
        plan = LIB.gemm_plan(t, m, n, k)
        print(f"Q4_K m={m} {n}x{k} ({LIB.plan_str(t, m, n, k)})", flush=True)
        assert plan[0] == LIB.KERNEL_TILES and plan[3] > 1, plan
        y_ref = torch.full((m, n), float("nan"), dtype=torch.float32, device=dev)
        y = torch.full((m, n), float("nan"), dtype=torch.float32, device=dev)
        LIB.check(_call(L.mbq_matmul, t, planes, x, m, n, k, y_ref), "mbq_matmul")
        LIB.check(_call(L.mbq_matmul_noalloc, t, planes, x, m, n, k, y), "mbq_matmul_noalloc")
        torch.cuda.synchronize()
        assert torch.equal(y.view(torch.int32), y_ref.view(torch.int32)), f"m={m}: noalloc differs from mbq_matmul"
        assert_product_dev(y, ref, f"m={m}")
