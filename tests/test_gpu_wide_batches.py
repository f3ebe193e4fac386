"""GPU parity of the automatic plans at 65-2048 activation rows on the weights of a 27B-class layer: the LDS-tile and
specialized-wave GEMMs, with the tile shapes and K splits the planner picks there (reference engine: prefill chunks of
up to 512 tokens and 2048 per call, src/mashbox/runtime/engine.py:168; north star 2: M = 64-2048).

Oracle: the oracle's seeded generators and its dequantization of every row; every output against the float64 product
on the GPU, within the bars of tests/_check.py (int8: the float32 y * s before the rounding, through the pj hook), and a
second call repeats bit for bit."""
import numpy as np
import pytest
import torch

from oracle import gen as G
from oracle import ref as R
from tests._check import assert_product_dev

import mashbox_amd.kernels as KQ
from mashbox_amd import _lib as LIB
from mashbox_amd import int8 as I8

pytestmark = pytest.mark.gpu

SHAPES = [(17408, 5120), (5120, 17408), (6144, 5120), (1024, 5120)]
MS = (128, 256, 512, 1024)
SEEN = []


@pytest.mark.parametrize("t", [R.Q4_K, "int8"], ids=["Q4_K", "int8"])
@pytest.mark.parametrize("n,k", SHAPES, ids=[f"{n}x{k}" for n, k in SHAPES])
def test_wide_batch_plans(t, n, k, cuda):
    rng = np.random.default_rng([n, k, 0 if t == "int8" else t, 133])
    if t == "int8":
        q, s = G.int8_weights(rng, n, k)
        qd, sd = torch.from_numpy(q).to(cuda), torch.from_numpy(s).to(cuda)
        w = I8.repack(qd, sd)
        w64 = qd.to(torch.float64)
        s64 = sd.to(torch.float64)
        tt = LIB.I8T
    else:
        raw = G.RAW[t](rng, n, k)
        p = KQ.repack(t, torch.from_numpy(raw).to(cuda), (n, k), tiled=True)
        w64 = torch.from_numpy(R.dequant(raw, t, k)).to(cuda).to(torch.float64)
        tt = KQ.TILED[t]
    for m in MS:
        plan = LIB.gemm_plan(tt, m, n, k)
        SEEN.append(plan)
        what = f"{'int8' if t == 'int8' else 'Q4_K'} tiles m={m} {n}x{k} ({LIB.plan_str(tt, m, n, k)})"
        print(what, flush=True)
        xb = G.acts(rng, m, k)
        x = torch.from_numpy(xb.astype(np.int16)).view(torch.bfloat16).to(cuda)
        ref = x.to(torch.float64) @ w64.T
        if t == "int8":
            got = []
            I8.linear(x, w, pj=lambda v: got.append(v.clone()) or v)
            I8.linear(x, w, pj=lambda v: got.append(v.clone()) or v)
            assert_product_dev(got[0], ref * s64, what)
            assert torch.equal(got[0].view(torch.int32), got[1].view(torch.int32)), what
        else:
            y = KQ.matmul(x, p)
            assert_product_dev(y, ref, what)
            assert torch.equal(KQ.matmul(x, p).view(torch.int32), y.view(torch.int32)), what
    del w64
    torch.cuda.empty_cache()


def test_wide_plans_cover_split_tiles():
    """the cases above include LDS tiles of 256 rows or columns with K split, which only these batch sizes plan"""
    if not SEEN:
        pytest.skip("runs after test_wide_batch_plans")
    assert any(kn == LIB.KERNEL_TILES and sp > 1 and max(bm, bn) >= 256 for kn, bm, bn, sp in SEEN), SEEN
