"""Every tail of the DMA pipelines, through forced plans: the steps after each kernel's unrolled loop issue no loads
for steps past the end and wait for exactly what they issued, so each count of such steps is run here once.

* sgemm_kernel (256 x 192 tiles, one K range): n = ceil(K / 64) K steps, n - 1 producer steps, (n - 1) % 3 of them
  after the loop; also n = 1-3, where the loop never runs (row-major and tiled Q4_K, Q6_K with its uneven producer
  split, Q8_0 with K not a multiple of 64);
* gemm_kernel with P = 3 (64 x 64 tiles: n % 4 tail steps) and P = 1 (128 x 256: n % 2), n per K range, also split;
* wsgemm_kernel (the weight stream: ceil(K / KI) iterations per range, 4 in flight, n % 4 tail steps);
* kgemm_kernel (tiled planes at 16 rows: ceil(chunks / K groups) steps, 2 or 3 stages).

Each case names the plan the forced kernel reports, the tail steps it takes, and checks two calls bit for bit and the
output against the oracle's float64 product (tests/_check.py bars)."""
import numpy as np
import pytest
import torch

from oracle import gen as G
from oracle import ref as R
from tests._check import assert_product_dev

import mashbox_amd.kernels as KQ
from mashbox_amd import _lib as LIB

pytestmark = pytest.mark.gpu

NAME = {R.Q8_0: "Q8_0", R.Q4_K: "Q4_K", R.Q6_K: "Q6_K"}
TILES, STREAM, KGROUP = LIB.KERNEL_TILES, LIB.KERNEL_STREAM, LIB.KERNEL_KGROUP


def _tails(kernel, bm, bn, s, t, k):
    """the tail steps each K range of the forced plan takes (the kernels' loop structure), for the case's label"""
    ranges = lambda n: [min(n, (z + 1) * -(-n // s)) - z * -(-n // s) for z in range(s) if z * -(-n // s) < n]
    if kernel == TILES:
        n = -(-k // 64)
        if (bm, bn) == (256, 192) and s == 1:
            return [(n - 1) % 3 if n > 1 else 0]
        na = 2 if bm == 128 else 4
        return [r % na for r in ranges(n)]
    if kernel == STREAM:
        ki = 64 if t == R.Q8_0 else 128
        return [r % 4 for r in ranges(-(-k // ki))]
    return []


CASES = [
    # sgemm: 0, 1 and 2 steps after the loop, and the short K ranges whose steps are all tail steps
    *[(TILES, 256, 192, 1, t, lay, 300, 400, k) for t in (R.Q4_K, R.Q6_K) for lay in ("rowmajor", "tiles")
      for k in (256, 512, 768)],
    *[(TILES, 256, 192, 1, R.Q8_0, "rowmajor", 300, 400, k) for k in (64, 128, 192, 224, 288, 352)],
    # gemm_kernel, P = 3: 0-3 tail steps, one range and split ranges; P = 1: 0-1
    *[(TILES, 64, 64, 1, R.Q8_0, "rowmajor", 100, 300, k) for k in (64, 128, 192, 320, 384, 448, 512)],
    (TILES, 64, 64, 2, R.Q8_0, "rowmajor", 100, 300, 640),
    (TILES, 64, 64, 3, R.Q4_K, "tiles", 100, 300, 1792),
    *[(TILES, 128, 256, 1, R.Q8_0, "rowmajor", 200, 300, k) for k in (320, 384)],
    (TILES, 128, 256, 3, R.Q4_K, "rowmajor", 200, 300, 1280),
    # weight stream: 0-3 tail iterations
    *[(STREAM, 16, 64, 1, R.Q8_0, "rowmajor", 8, 300, k) for k in (96, 320, 384, 448, 512)],
    *[(STREAM, 16, 128, s, R.Q4_K, "rowmajor", 8, 300, k) for s, k in ((1, 768), (2, 1792), (3, 1792))],
    # K-group: chunk counts whose steps leave 0, 1 or 2 tail steps at the planner's row groups
    *[(KGROUP, 0, 0, s, R.Q4_K, "tiles", 16, 300, k) for s, k in ((1, 1024), (1, 2048), (1, 3072), (2, 2304), (3, 2304))],
]


def _id(c):
    kernel, bm, bn, s, t, lay, m, n, k = c
    kn = LIB.KERNEL_NAMES[kernel]
    return f"{kn}-{bm}x{bn}/{s}-{NAME[t]}-{lay}-m{m}-{n}x{k}"


@pytest.mark.parametrize("kernel,bm,bn,s,t,lay,m,n,k", CASES, ids=[_id(c) for c in CASES])
def test_pipeline_tail(kernel, bm, bn, s, t, lay, m, n, k, cuda):
    rng = np.random.default_rng([m, n, k, s])
    raw = G.RAW[t](rng, n, k)
    p = KQ.repack(t, torch.from_numpy(raw).to(cuda), (n, k), tiled=lay == "tiles")
    xb = G.acts(rng, m, k)
    x = torch.from_numpy(xb.astype(np.int16)).view(torch.bfloat16).to(cuda)
    try:
        LIB.force_gemm_plan(kernel, bm, bn, s)
        plan = LIB.plan_str(p.t, m, n, k)
        label = f"{NAME[t]} {lay} m={m} {n}x{k} ({plan}; tail steps per K range {_tails(kernel, bm, bn, s, t, k)})"
        print(label, flush=True)
        assert plan.startswith(LIB.KERNEL_NAMES[kernel]), f"the forced plan did not take: {plan}"
        if kernel != KGROUP:
            assert plan.startswith(f"{LIB.KERNEL_NAMES[kernel]} {bm}x{bn}/"), plan
        y1 = KQ.matmul(x, p)
        y2 = KQ.matmul(x, p)
    finally:
        LIB.force_gemm_plan()
    assert torch.equal(y1.view(torch.int32), y2.view(torch.int32)), f"{label}: two calls differ"
    w64 = torch.from_numpy(R.dequant(raw, t, k)).to(cuda).to(torch.float64)
    assert_product_dev(y1, x.to(torch.float64) @ w64.T, label)
