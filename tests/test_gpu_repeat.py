"""Run-to-run repeatability of the batched kernels whose waves hand data to each other through LDS, at the sizes of
the benchmark configs: the specialized-wave GEMM (producer waves dequantize weights into LDS for the consumer waves;
Q4_K with the even split of that work, Q6_K with the uneven one) and the K-group kernel (x staged by DMA, the K groups'
sums reduced through LDS, and, for the down projection, split-K partials exchanged through memory). Every one of these
sums in a fixed order, so repeated calls give the same bits; and the tile GEMV at one row (x staged in LDS, each
tile's rows summed over the waves through LDS), in its 8-wave and 16-wave blocks; a writer that passes a barrier before its writes land
shows as calls that differ (seen on MI355X as stale dequantized weights once the producers were sped up, until the
producers waited for their LDS writes before each barrier; and as stale x rows in a tile's final K step, from a
producer wait that counted weight loads the compiler had dropped, until the last steps issued only what they wait
for: tests/test_vmcnt.py checks those waits in the built code)."""
import pytest
import torch

import mashbox_amd.kernels as KQ
from mashbox_amd import _lib as LIB
from mashbox_amd import int8 as I8
from mashbox_amd import synth

pytestmark = pytest.mark.gpu

CASES = [(12, 2048, 6144, 5120), (14, 2048, 5120, 6144), ("int8", 64, 17408, 5120), ("int8", 64, 5120, 17408),
         ("tiles", 1, 17408, 5120), ("tiles", 1, 5120, 17408)]
IDS = ["Q4_K-2048x6144x5120", "Q6_K-2048x5120x6144", "int8-64x17408x5120", "int8-64x5120x17408",
       "Q4_K-tiles-1x17408x5120", "Q4_K-tiles-1x5120x17408"]
CALLS = 8


@pytest.mark.parametrize("t,m,n,k", CASES, ids=IDS)
def test_batched_kernels_repeat_bit_for_bit(t, m, n, k, cuda):
    x = synth.acts(m, k, seed=11, device=cuda)
    if t == "int8":
        q, s = synth.int8_weights(n, k, seed=12, device=cuda)
        planes = I8.repack(q, s)
        run = lambda: I8.linear(x, planes)
        plan = LIB.plan_str(LIB.I8T, m, n, k)
    elif t == "tiles":
        planes = KQ.repack(12, synth.q4_k_raw(n, k, seed=12, device=cuda), (n, k), tiled=True)
        run = lambda: KQ.matmul(x, planes, out_dtype=torch.bfloat16)
        plan = LIB.plan_str(planes.t, m, n, k)
    else:
        raw = {12: synth.q4_k_raw, 14: synth.q6_k_raw}[t](n, k, seed=12, device=cuda)
        planes = KQ.repack(t, raw, (n, k))
        run = lambda: KQ.matmul(x, planes, out_dtype=torch.bfloat16)
        plan = LIB.plan_str(t, m, n, k)
    print(f"case: {t} {m} x {n} x {k} ({plan}), {CALLS} calls", flush=True)
    first = run().view(torch.int16).clone()
    assert bool(torch.isfinite(first.view(torch.bfloat16)).all())
    for i in range(1, CALLS):
        y = run().view(torch.int16)
        diff = int((y != first).sum())
        assert diff == 0, f"call {i}: {diff} outputs differ from the first call ({plan}); {_where(y, first, run)}"


def _where(y, first, run):
    """where two calls' outputs differ (rows, columns, 256 x 192 tiles), and which of them one more call agrees with"""
    d = (y != first)
    rows = torch.nonzero(d.any(1)).flatten()
    cols = torch.nonzero(d.any(0)).flatten()
    tiles = torch.nonzero(d.reshape(-1, 1) if d.dim() < 2 else d).cpu()
    tset = sorted({(int(r) // 256, int(c) // 192) for r, c in tiles[:: max(1, len(tiles) // 4096)].tolist()})
    again = run().view(torch.int16)
    return (f"rows {int(rows.min())}-{int(rows.max())} ({len(rows)} distinct), columns {int(cols.min())}-"
            f"{int(cols.max())} ({len(cols)} distinct), tiles (row, column) {tset[:24]}; one more call differs from the "
            f"first in {int((again != first).sum())} outputs and from the failing call in {int((again != y).sum())}")
