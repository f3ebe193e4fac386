"""A seeded sweep of random valid shapes through every weight type and layout, so that the plans of uncommon shapes are
exercised too. The named tests cover the BASELINE configs and the 27B-class layer. Here the cases are:

* every GGUF type on row-major planes and on 16-row tiles, and the int8 linear on its row-major weights and on its
  tiles;
* rows N from 1 to 4000 (mostly not a multiple of 16);
* K any multiple of the type's block up to 12288;
* activation rows M over the kernels' boundaries (1-4 the GEMVs, 5-64 the weight stream and K-group kernels, 65-2048
  the LDS-tile and specialized-wave GEMMs with the wide-batch planner's tile shapes and K splits).

Each case uses automatic plans.

Oracle: the oracle's seeded generators and its dequantization of every row; every output against the float64 product
on the GPU, within the bars of tests/_check.py (the int8 linear: its float32 y * s before the rounding, through the pj
hook)."""
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

BLOCK = {R.Q4_0: 32, R.Q8_0: 32, R.Q4_K: 256, R.Q5_K: 256, R.Q6_K: 256, "int8": 16}
NAME = {R.Q4_0: "Q4_0", R.Q8_0: "Q8_0", R.Q4_K: "Q4_K", R.Q5_K: "Q5_K", R.Q6_K: "Q6_K", "int8": "int8"}
KINDS = [(t, lay) for t in (R.Q4_0, R.Q8_0, R.Q4_K, R.Q5_K, R.Q6_K, "int8") for lay in ("rowmajor", "tiles")]
MS = (1, 2, 3, 4, 5, 7, 8, 9, 15, 16, 17, 31, 33, 47, 63, 64, 65, 100, 129, 257, 300, 384, 512, 700, 1024, 2048)


def _cases(count=192, seed=2026):
    rng = np.random.default_rng(seed)
    out = []
    for i in range(count):
        t, lay = KINDS[i % len(KINDS)]
        b = BLOCK[t]
        k = b * int(rng.integers(1, 12288 // b + 1))
        n = int(rng.integers(1, 4001))
        while n * k > 6_000_000:                        # the oracle's dequantization stays a fraction of a second
            n = max(1, n // 2)
        m = int(MS[int(rng.integers(0, len(MS)))])
        while m * (n + k) > 12_000_000:                  # and the float64 reference product small
            m = max(1, m // 2)
        out.append((t, lay, m, n, k, i))
    return out


CASES = _cases()


@pytest.mark.parametrize("t,lay,m,n,k,i", CASES, ids=[f"{NAME[c[0]]}-{c[1]}-m{c[2]}-{c[3]}x{c[4]}" for c in CASES])
def test_random_shape(t, lay, m, n, k, i, cuda):
    rng = np.random.default_rng([i, 2027])
    xb = G.acts(rng, m, k)
    x = torch.from_numpy(xb.astype(np.int16)).view(torch.bfloat16).to(cuda)
    x64 = x.to(torch.float64)
    if t == "int8":
        q, s = G.int8_weights(rng, n, k)
        qd, sd = torch.from_numpy(q).to(cuda), torch.from_numpy(s).to(cuda)
        w = {"q": qd, "s": sd} if lay == "rowmajor" else I8.repack(qd, sd)
        tt = LIB.INT8 if lay == "rowmajor" else LIB.I8T
        print(f"int8 {lay} m={m} {n}x{k} ({LIB.plan_str(tt, m, n, k)})", flush=True)
        got = []
        I8.linear(x, w, pj=lambda v: got.append(v.clone()) or v)
        ref = (x64 @ qd.to(torch.float64).T) * sd.to(torch.float64)
        assert_product_dev(got[0], ref, f"int8 {lay} m={m} {n}x{k}")
        return
    raw = G.RAW[t](rng, n, k)
    tiled = lay == "tiles"
    p = KQ.repack(t, torch.from_numpy(raw).to(cuda), (n, k), tiled=tiled)
    print(f"{NAME[t]} {lay} m={m} {n}x{k} ({LIB.plan_str(p.t, m, n, k)})", flush=True)
    w64 = torch.from_numpy(R.dequant(raw, t, k)).to(cuda).to(torch.float64)
    assert_product_dev(KQ.matmul(x, p), x64 @ w64.T, f"{NAME[t]} {lay} m={m} {n}x{k}")
