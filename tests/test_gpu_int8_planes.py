"""GPU parity of the int8 linear on weights repacked at load into 16-row tiles (mashbox_amd.int8.repack, libmbq's
MBQ_I8T planes), against the reference's int8 linear (reference src/mashbox/models/qwen3_8_27b/model.py:72-82):
(x @ bf16(q).T, float32 accumulation) * s.

Oracle: the float64 product of the exact int8 weights and scales from the oracle's seeded generator (tests/_check.py
bars). Batches of 5-64 rows run the K-group kernel (mbq_kgemm.hip), which only the tiled planes have; batches past 64
rows run the same LDS-tile plans as the unpacked linear, so there the two are equal bit for bit.
"""
import numpy as np
import pytest
import torch

from oracle import gen as G
from oracle import ref as R
from tests._check import assert_product, assert_product_dev

from mashbox_amd import _lib as LIB
from mashbox_amd import int8 as I8

pytestmark = pytest.mark.gpu


def _x(rng, m, k, dev):
    xb = G.acts(rng, m, k)
    return xb, torch.from_numpy(xb.astype(np.int16)).view(torch.bfloat16).to(dev)


def _f32(x, w, **kw):
    """the float32 y * s that the int8 linear hands its pj hook, before the rounding to x's dtype"""
    got = []
    I8.linear(x, w, pj=lambda v: got.append(v.clone()) or v, **kw)
    return got[0]


@pytest.mark.parametrize("n,k", [(1, 16), (17, 48), (33, 1040), (130, 4096)])
def test_device_repack_equals_host_repack(n, k, cuda):
    rng = np.random.default_rng([n, k, 1])
    q, s = G.int8_weights(rng, n, k)
    host = I8.repack_host(q, s)
    dev = I8.repack(torch.from_numpy(q).to(cuda), torch.from_numpy(s).to(cuda))
    assert torch.equal(dev.buf.cpu(), host.buf)
    # into a buffer full of 0xAB: every byte is written (padding rows, columns and gaps zero)
    import ctypes
    dirty = torch.full((host.buf.numel(),), 0xAB, dtype=torch.uint8, device=cuda)
    qd, sd = torch.from_numpy(q).to(cuda), torch.from_numpy(s).to(cuda)
    assert LIB.lib().mbq_int8_repack_dev(ctypes.c_void_p(qd.data_ptr()), ctypes.c_void_p(sd.data_ptr()), n, k,
                                         ctypes.c_void_p(dirty.data_ptr()),
                                         ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)) == 0
    assert torch.equal(dirty.cpu(), host.buf)


@pytest.mark.parametrize("n,k", [(7, 16), (33, 48), (130, 4096), (1000, 1040)])
@pytest.mark.parametrize("m", [1, 2, 3, 4, 5, 16, 17, 64, 65, 130, 300])
def test_planes_linear_matches_reference(n, k, m, cuda):
    rng = np.random.default_rng([n, k, m])
    q, s = G.int8_weights(rng, n, k)
    xb, x = _x(rng, m, k, cuda)
    ref = (R.bf16_to_f32(xb).astype(np.float64) @ q.astype(np.float64).T) * s.astype(np.float64)
    w = {"q": torch.from_numpy(q).to(cuda), "s": torch.from_numpy(s).to(cuda)}
    p = I8.repack(w["q"], w["s"])
    y = _f32(x, p).cpu().numpy()
    assert_product(y, ref, f"int8 planes m={m} n={n} k={k} ({LIB.plan_str(LIB.I8T, m, n, k)})")
    yb = I8.linear(x, p)
    assert yb.dtype == torch.bfloat16
    assert np.array_equal(yb.view(torch.int16).cpu().numpy().view(np.uint16), R.bf16_round(y))
    if m > 64:                                                 # the same plan as the unpacked weights: same bits
        assert LIB.plan_str(LIB.I8T, m, n, k) == LIB.plan_str(LIB.INT8, m, n, k)
        assert np.array_equal(y.view(np.uint32), _f32(x, w).cpu().numpy().view(np.uint32))
    elif m > 4:
        assert LIB.gemm_plan(LIB.I8T, m, n, k)[0] == LIB.KERNEL_KGROUP


@pytest.mark.parametrize("m", [1, 4, 64, 300])
def test_planes_stack_read_in_place(m, cuda):
    """a stack of 3 weights repacked at once; layer= as an int and as a device int32 reads one in place; a device layer
    outside the stack gives NaN"""
    rng = np.random.default_rng([m, 3])
    n, k, L = 70, 320, 3
    q = np.stack([G.int8_weights(rng, n, k)[0] for _ in range(L)])
    s = np.stack([G.int8_weights(rng, n, k)[1] for _ in range(L)])
    p = I8.repack(torch.from_numpy(q).to(cuda), torch.from_numpy(s).to(cuda))
    xb, x = _x(rng, m, k, cuda)
    xf = R.bf16_to_f32(xb).astype(np.float64)
    for layer in range(L):
        ref = (xf @ q[layer].astype(np.float64).T) * s[layer]
        assert_product(_f32(x, p, layer=layer).cpu().numpy(), ref, f"layer {layer}")
        dl = torch.tensor(layer, dtype=torch.int32, device=cuda)
        got = _f32(x, p, layer=dl).cpu().numpy()
        assert_product(got, ref, f"device layer {layer}")
        assert np.array_equal(got, _f32(x, p[layer]).cpu().numpy())
    bad = _f32(x, p, layer=torch.tensor(L, dtype=torch.int32, device=cuda)).cpu().numpy()
    assert np.all(np.isnan(bad))


@pytest.fixture
def forced_plan():
    yield LIB.force_gemm_plan
    LIB.force_gemm_plan()


@pytest.mark.parametrize("bm,bn", [(256, 256), (256, 192), (256, 128), (128, 256), (128, 192), (128, 128), (128, 64),
                                   (64, 256), (64, 192), (64, 128), (64, 64)])
def test_every_tile_shape_with_and_without_split(bm, bn, forced_plan, cuda):
    rng = np.random.default_rng([bm, bn, 9])
    m, n, k = bm + bm // 2 - 3, bn + 17, 16 * 25
    q, s = G.int8_weights(rng, n, k)
    xb, x = _x(rng, m, k, cuda)
    ref = (R.bf16_to_f32(xb).astype(np.float64) @ q.astype(np.float64).T) * s
    p = I8.repack(torch.from_numpy(q).to(cuda), torch.from_numpy(s).to(cuda))
    for splits in (1, 3):
        forced_plan(LIB.KERNEL_TILES, bm, bn, splits)
        assert LIB.gemm_plan(LIB.I8T, m, n, k)[:3] == (LIB.KERNEL_TILES, bm, bn)
        assert_product(_f32(x, p).cpu().numpy(), ref, f"tile {bm}x{bn} splits {splits}")


@pytest.mark.parametrize("m", [1, 4, 5, 17, 40, 64])
@pytest.mark.parametrize("rows", [64, 128])
@pytest.mark.parametrize("k", [16 * 57, 64 * 15])
def test_weight_stream_every_shape(m, rows, k, forced_plan, cuda):
    rng = np.random.default_rng([m, rows, k])
    n = 3 * rows + 17
    q, s = G.int8_weights(rng, n, k)
    xb, x = _x(rng, m, k, cuda)
    ref = (R.bf16_to_f32(xb).astype(np.float64) @ q.astype(np.float64).T) * s
    p = I8.repack(torch.from_numpy(q).to(cuda), torch.from_numpy(s).to(cuda))
    for splits in (1, 3):
        forced_plan(LIB.KERNEL_STREAM, 16, rows, splits)
        assert_product(_f32(x, p).cpu().numpy(), ref, f"stream m={m} rows={rows} k={k} splits {splits}")


def test_full_config_4_on_planes(cuda):
    """config 4 (seed 0) with every projection repacked on the GPU: every output against the float64 product"""
    cfg = G.config(4, seed=0)
    for name, n, k, (q, s), xb in cfg["projections"]:
        print(f"config 4 planes {name} {n}x{k}", flush=True)
        x = torch.from_numpy(xb.astype(np.int16)).view(torch.bfloat16).to(cuda)
        qd, sd = torch.from_numpy(q).to(cuda), torch.from_numpy(s).to(cuda)
        p = I8.repack(qd, sd)
        y = _f32(x, p)
        ref = (x.to(torch.float64) @ qd.to(torch.float64).T) * sd.to(torch.float64)
        assert_product_dev(y, ref, f"config 4 {name} ({LIB.plan_str(LIB.I8T, 64, n, k)})")


def test_graph_replays_on_planes(forced_plan, cuda):
    """a split-K weight-stream call on planes, recorded into a HIP graph, replays bit for bit equal to the eager call
    with eager calls in between"""
    rng = np.random.default_rng(77)
    m, n, k = 64, 1024, 5120
    q, s = G.int8_weights(rng, n, k)
    xb, x = _x(rng, m, k, cuda)
    _, x2 = _x(rng, m, k, cuda)
    p = I8.repack(torch.from_numpy(q).to(cuda), torch.from_numpy(s).to(cuda))
    forced_plan(LIB.KERNEL_STREAM, 16, 64, 4)
    eager = _f32(x, p).cpu().numpy()
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        y = _f32(x, p)
    for _ in range(3):
        g.replay()
        torch.cuda.synchronize()
        assert np.array_equal(y.cpu().numpy().view(np.uint32), eager.view(np.uint32))
        _f32(x2, p)
        torch.cuda.synchronize()


# ---------------------------------------------------------------------------------------------- K-group kernel
@pytest.mark.parametrize("m", [5, 16, 17, 33, 64])
@pytest.mark.parametrize("n,k", [(1000, 16 * 57), (4500, 64 * 40), (70, 64 * 3), (7, 16)])
def test_kgroup_every_split_count(m, n, k, forced_plan, cuda):
    """the K-group kernel at every split count the planner can take (each split count fixes rows per block, row groups
    and tiles per wave), on ragged row counts (blocks whose row ranges start and end inside 16-row tiles) and ragged K
    (a last chunk partly past K), against the float64 product"""
    rng = np.random.default_rng([m, n, k, 5])
    q, s = G.int8_weights(rng, n, k)
    xb, x = _x(rng, m, k, cuda)
    ref = (R.bf16_to_f32(xb).astype(np.float64) @ q.astype(np.float64).T) * s
    p = I8.repack(torch.from_numpy(q).to(cuda), torch.from_numpy(s).to(cuda))
    kc = (k + 63) // 64
    for splits in (0, 1, 2, 3, 4, 6, 8):
        if splits > kc:
            continue
        forced_plan(LIB.KERNEL_KGROUP, 0, 0, splits)
        plan = LIB.gemm_plan(LIB.I8T, m, n, k)
        assert plan[0] == LIB.KERNEL_KGROUP and (splits == 0 or plan[3] == splits), plan
        print(f"kgroup m={m} n={n} k={k} plan {plan}", flush=True)
        y = _f32(x, p).cpu().numpy()
        assert_product(y, ref, f"kgroup m={m} n={n} k={k} plan {plan}")
        # a split K repeats bit for bit (partials added in split order, whichever block arrives last)
        assert np.array_equal(_f32(x, p).cpu().numpy().view(np.uint32), y.view(np.uint32))


def test_kgroup_plans_of_config_4():
    """the automatic plans of config 4's projections at 64 rows: the K-group kernel, with the split counts that measured
    fastest on MI355X (q, o, gate, up: 1-2; k, v, down: 4)"""
    for name, (n, k) in G.LAYER_27B.items():
        kern, _, rows, splits = LIB.gemm_plan(LIB.I8T, 64, n, k)
        assert kern == LIB.KERNEL_KGROUP, name
        assert splits in ((4,) if name in ("k", "v", "down") else (1, 2)), (name, rows, splits)


def test_kgroup_graph_replays(forced_plan, cuda):
    """a split-K K-group call recorded into a HIP graph replays bit for bit equal to the eager call, with eager calls of
    the same kernel in between"""
    rng = np.random.default_rng(78)
    m, n, k = 64, 1024, 5120
    q, s = G.int8_weights(rng, n, k)
    xb, x = _x(rng, m, k, cuda)
    _, x2 = _x(rng, m, k, cuda)
    p = I8.repack(torch.from_numpy(q).to(cuda), torch.from_numpy(s).to(cuda))
    forced_plan(LIB.KERNEL_KGROUP, 0, 0, 4)
    eager = _f32(x, p).cpu().numpy()
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        y = _f32(x, p)
    for _ in range(3):
        g.replay()
        torch.cuda.synchronize()
        assert np.array_equal(y.cpu().numpy().view(np.uint32), eager.view(np.uint32))
        _f32(x2, p)
        torch.cuda.synchronize()
