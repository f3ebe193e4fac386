"""GPU parity of decode and small batches on every weight shape of a 27B-class layer, and of rows longer than that.

The reference's engine decodes in row buckets 1/4/16/64/256 (reference src/mashbox/runtime/engine.py:424-428), and a
shape the kernel package reports covered must run (kq_covers, reference src/mashbox/ops/__init__.py:359-363). Each of
the six weight types runs M in {1, 2, 3, 4, 8, 16} over the seven projections of configs 4/5 (q 6144x5120, k/v
1024x5120, o 5120x6144, gate/up 17408x5120, down 5120x17408) and a 28672-wide down projection (5120x28672: longer than
the decode GEMV's registers hold at 1-4 rows for Q8_0 / int8, and at 3-4 rows for every type, so the weight stream runs
it).

Oracle: the weights come from the oracle's seeded generators; every output of every product is compared with the
float64 product (computed on the GPU) of the oracle's dequantization of every row, within the product bars of
tests/_check.py; the kernel's own dequantization is compared bit for bit with the oracle's on a row sample (first, last
and 60 seeded rows).
"""
import numpy as np
import pytest
import torch

from oracle import gen as G
from oracle import ref as R
from tests._check import assert_product_dev, diff_bits

import mashbox_amd.kernels as KQ
from mashbox_amd import _lib as LIB
from mashbox_amd import int8 as I8

pytestmark = pytest.mark.gpu

SHAPES = list(G.LAYER_27B.items()) + [("down28672", (5120, 28672))]
DECODE_M = [1, 2, 3, 4, 8, 16]
TYPES = [R.Q4_0, R.Q8_0, R.Q4_K, R.Q5_K, R.Q6_K, "int8"]
IDS = ["Q4_0", "Q8_0", "Q4_K", "Q5_K", "Q6_K", "int8"]


def _bf16(bits, dev):
    return torch.from_numpy(bits.astype(np.int16)).view(torch.bfloat16).to(dev)


@pytest.mark.parametrize("t", TYPES, ids=IDS)
def test_decode_batches_on_every_layer_shape(t, cuda):
    tt = LIB.INT8 if t == "int8" else t
    for si, (name, (n, k)) in enumerate(SHAPES):
        rng = np.random.default_rng([si, 0 if t == "int8" else t, 424])
        print(f"{IDS[TYPES.index(t)]} {name} {n}x{k}", flush=True)
        if t == "int8":
            q, s = G.int8_weights(rng, n, k)
            w = {"q": torch.from_numpy(q).to(cuda), "s": torch.from_numpy(s).to(cuda)}
            w64 = w["q"].to(torch.float64)
            s64 = w["s"].to(torch.float64)
        else:
            assert KQ.kq_covers(t, (n, k)), f"{name} {n}x{k} must be covered"
            raw = G.RAW[t](rng, n, k)
            planes = KQ.repack_host(t, raw, (n, k)).to(cuda)
            # the reference weights are the oracle's dequantization of every row (not the kernel's own); the kernel's
            # dequantization is checked against it bit for bit on a row sample, as a separate assertion
            w_or = R.dequant(raw, t, k)
            wd = KQ.dequant(planes)
            rows = np.unique(np.concatenate([[0, 1, n - 2, n - 1], rng.choice(n, 60, replace=False)]))
            assert diff_bits(wd[torch.from_numpy(rows).to(cuda)].cpu().numpy(), w_or[rows]) == 0
            del wd
            w64 = torch.from_numpy(w_or).to(cuda).to(torch.float64)
            del w_or
        for m in DECODE_M:
            xb = G.acts(rng, m, k)
            x = _bf16(xb, cuda)
            ref = x.to(torch.float64) @ w64.T
            kind = LIB.gemm_plan(tt, m, n, k)[0]
            if m > 4:
                assert kind != LIB.KERNEL_GEMV
            if t == "int8":
                got = []
                I8.linear(x, w, pj=lambda v: got.append(v.clone()) or v)
                assert_product_dev(got[0], ref * s64, f"int8 {name} m={m} ({LIB.KERNEL_NAMES[kind]})")
            else:
                y = KQ.matmul(x, planes)
                assert_product_dev(y, ref, f"{IDS[TYPES.index(t)]} {name} m={m} ({LIB.KERNEL_NAMES[kind]})")
        del w64
        torch.cuda.empty_cache()


@pytest.mark.parametrize("t", TYPES, ids=IDS)
def test_rows_beyond_the_gemv_registers_take_the_weight_stream(t, cuda):
    """K = 17408 at 3-4 activation rows (every type but int8 at 3), and K = 28672 Q8_0 / int8 at every decode batch,
    have no GEMV plan: the plan reports the weight-stream kernel, and the call runs (checked in full above)"""
    tt = LIB.INT8 if t == "int8" else t
    for m in (3, 4):
        kind = LIB.gemm_plan(tt, m, 5120, 17408)[0]
        if t == "int8" and m == 3:
            assert kind == LIB.KERNEL_GEMV
        else:
            assert kind == LIB.KERNEL_STREAM, (t, m, kind)
    for m in (1, 2, 3, 4):
        kind = LIB.gemm_plan(tt, m, 5120, 28672)[0]
        if t in ("int8", R.Q8_0) or m >= 3:
            assert kind == LIB.KERNEL_STREAM, (t, m, kind)
        else:
            assert kind == LIB.KERNEL_GEMV, (t, m, kind)
    assert LIB.gemm_plan(tt, 1, 17408, 5120)[0] == LIB.KERNEL_GEMV
