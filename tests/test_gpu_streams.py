"""Split-K calls on two streams that overlap in time, through the C ABI.

mbq_matmul keeps one split-K workspace (float32 partial tiles and arrival counters) per (device, stream). Two split-K
GEMMs queued alternately on two streams, many launches deep with no synchronisation between them, therefore run side by
side without sharing partials or counters: every result equals the same call made alone on one stream bit for bit, and
meets the product bars against the oracle's exact weights. The cases are a K-group launch on tiled int8 planes (4 K
ranges) and a weight-stream launch on Q4_K planes (8 K ranges), both automatic plans.
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


def _int8_case(dev, m=64, n=5120, k=17408, seed=71):
    L = LIB.lib()
    rng = np.random.default_rng(seed)
    q, s = G.int8_weights(rng, n, k)
    pb = LIB.check(L.mbq_plane_bytes(LIB.I8T, n, k), "plane_bytes")
    host = torch.empty(pb, dtype=torch.uint8)
    LIB.check(L.mbq_int8_repack_host(q.ctypes.data_as(ctypes.c_void_p), s.ctypes.data_as(ctypes.c_void_p), n, k,
                                     ctypes.c_void_p(host.data_ptr()), pb, 0), "int8 repack_host")
    x = torch.from_numpy(G.acts(rng, m, k).astype(np.int16)).view(torch.bfloat16).to(dev)
    ref = (x.to(torch.float64) @ torch.from_numpy(q).to(dev).to(torch.float64).T) * \
        torch.from_numpy(s).to(dev).to(torch.float64)
    return LIB.I8T, host.to(dev), x, (m, n, k), ref


def _q4k_case(dev, m=16, n=1024, k=5120, seed=72):
    L = LIB.lib()
    rng = np.random.default_rng(seed)
    raw = G.q4_k_raw(rng, n, k)
    pb = LIB.check(L.mbq_plane_bytes(R.Q4_K, n, k), "plane_bytes")
    host = torch.empty(pb, dtype=torch.uint8)
    LIB.check(L.mbq_repack_host(R.Q4_K, raw.ctypes.data_as(ctypes.c_void_p), n, k, ctypes.c_void_p(host.data_ptr()),
                                pb, 0), "repack_host")
    x = torch.from_numpy(G.acts(rng, m, k).astype(np.int16)).view(torch.bfloat16).to(dev)
    ref = x.to(torch.float64) @ torch.from_numpy(R.dequant(raw, R.Q4_K, k)).to(dev).to(torch.float64).T
    return R.Q4_K, host.to(dev), x, (m, n, k), ref


def _launch(case, y, stream):
    t, planes, x, (m, n, k), _ = case
    return LIB.check(LIB.lib().mbq_matmul(t, ctypes.c_void_p(planes.data_ptr()), 0, None, 1,
                                          ctypes.c_void_p(x.data_ptr()), m, n, k, ctypes.c_void_p(y.data_ptr()),
                                          LIB.OUT_F32, ctypes.c_void_p(stream.cuda_stream)), "mbq_matmul")


def test_split_k_on_two_overlapping_streams():
    dev = torch.device("cuda", 0)
    cases = [_int8_case(dev), _q4k_case(dev)]
    for t, _, _, (m, n, k), _ in cases:
        plan = LIB.gemm_plan(t, m, n, k)
        print(f"case type {t} {m}x{n}x{k} plan {plan}", flush=True)
        assert plan[3] > 1, "each case must split K"
    streams = [torch.cuda.Stream(device=dev) for _ in cases]
    # each case alone on its stream: the result every overlapped launch must repeat
    alone = []
    for c, st in zip(cases, streams):
        y = torch.full((c[3][0], c[3][1]), float("nan"), dtype=torch.float32, device=dev)
        _launch(c, y, st)
        torch.cuda.synchronize()
        assert_product_dev(y, c[4], f"type {c[0]} alone")
        alone.append(y)
    # both streams, launches queued alternately and never waited for in between: the two streams' kernels overlap
    reps = 24
    outs = [[torch.full_like(alone[i], float("nan")) for _ in range(reps)] for i in range(len(cases))]
    torch.cuda.synchronize()
    for r in range(reps):
        for i, (c, st) in enumerate(zip(cases, streams)):
            _launch(c, outs[i][r], st)
    torch.cuda.synchronize()
    for i, c in enumerate(cases):
        bad = [r for r in range(reps) if not torch.equal(outs[i][r].view(torch.int32), alone[i].view(torch.int32))]
        assert not bad, f"type {c[0]}: launches {bad} differ from the call made alone"
        assert_product_dev(outs[i][-1], c[4], f"type {c[0]} overlapped")
