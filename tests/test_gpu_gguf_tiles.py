"""GPU parity of every GGUF type's weights (Q4_K, Q8_0, Q6_K, Q5_K, Q4_0) repacked at load into 16-row tiles (kernels.repack(..., tiled=True),
libmbq's MBQ_Q4KT, MBQ_Q8T, MBQ_Q6KT and MBQ_Q5KT planes) against the reference's dequantization (reference
src/mashbox/ops/reference.py:132-149, :101-103, :164-173, :150-159) and its dequantize-then-matmul (reference src/mashbox/ops/__init__.py:594-632).

Oracle: oracle.ref's dequantization of the same blocks (bit for bit for dequant, take_rows and the repack) and the
float64 product of those weights (tests/_check.py bars). One row runs the tile GEMV (mbq_tgemv.hip) and 2-64 rows the
K-group kernel (mbq_kgemm.hip), which read only tiled planes; batches past 64 rows run the same LDS-tile plans as
row-major planes, so there the two layouts give the same bits.
"""
import ctypes

import numpy as np
import pytest
import torch

from oracle import gen as G
from oracle import ref as R
from tests._check import assert_product, assert_product_dev, diff_bits

from mashbox_amd import _lib as LIB
from mashbox_amd import kernels as KQ

pytestmark = pytest.mark.gpu
TYPES = [R.Q4_K, R.Q8_0, R.Q6_K, R.Q5_K, R.Q4_0]
NAME = {R.Q4_K: "Q4_K", R.Q8_0: "Q8_0", R.Q6_K: "Q6_K", R.Q5_K: "Q5_K", R.Q4_0: "Q4_0"}


def _x(rng, m, k, dev):
    xb = G.acts(rng, m, k)
    return xb, torch.from_numpy(xb.astype(np.int16)).view(torch.bfloat16).to(dev)


@pytest.fixture
def forced_plan():
    yield LIB.force_gemm_plan
    LIB.force_gemm_plan()


@pytest.mark.parametrize("t", TYPES, ids=NAME.get)
@pytest.mark.parametrize("n,k", [(1, 256), (17, 512), (100, 768), (130, 4096)])
def test_device_repack_equals_host_repack(t, n, k, cuda):
    """the GPU repack writes the host repack's bytes, every byte (into a buffer full of 0xAB), the padding rows of the
    last tile included"""
    rng = np.random.default_rng([n, k, 120])
    raw = G.RAW[t](rng, n, k)
    host = KQ.repack_host(t, raw, (n, k), tiled=True)
    dev = KQ.repack(t, torch.from_numpy(raw).to(cuda), (n, k), tiled=True)
    assert dev.t == KQ.TILED[t] and torch.equal(dev.buf.cpu(), host.buf)
    dirty = torch.full((host.buf.numel(),), 0xAB, dtype=torch.uint8, device=cuda)
    rd = torch.from_numpy(raw).to(cuda)
    assert LIB.lib().mbq_repack_dev(KQ.TILED[t], ctypes.c_void_p(rd.data_ptr()), n, k, ctypes.c_void_p(dirty.data_ptr()),
                                    ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)) == 0
    assert torch.equal(dirty.cpu(), host.buf)


@pytest.mark.parametrize("t", TYPES, ids=NAME.get)
@pytest.mark.parametrize("n,k", [(1, 256), (33, 512), (130, 2304)])
def test_dequant_and_rows_bit_exact(t, n, k, cuda):
    """dequant and take_rows of tiled planes: bit for bit the oracle's dequantization (random bytes: NaN and infinite
    scales included)"""
    rng = np.random.default_rng([n, k, 121])
    raw = rng.integers(0, 256, (n, R.row_bytes(t, k)), dtype=np.uint8)
    p = KQ.repack_host(t, raw, (n, k), tiled=True).to(cuda)
    want = R.dequant(raw, t, k)
    assert diff_bits(KQ.dequant(p).cpu().numpy(), want) == 0
    ids = rng.integers(-n, n, 9)
    assert diff_bits(KQ.take_rows(p, torch.from_numpy(ids)).cpu().numpy(), want[ids]) == 0


@pytest.mark.parametrize("t", TYPES, ids=NAME.get)
@pytest.mark.parametrize("n,k", [(33, 256), (100, 512), (1000, 2304), (4500, 1024)])
@pytest.mark.parametrize("m", [1, 2, 3, 4, 5, 8, 16, 17, 32, 33, 48, 64, 65, 130])
def test_matmul_matches_reference(t, n, k, m, cuda):
    _matmul_case(t, n, k, m, cuda)


@pytest.mark.parametrize("t", [R.Q8_0, R.Q4_0], ids=NAME.get)
@pytest.mark.parametrize("n,k", [(33, 96), (100, 1056), (7, 32)])
@pytest.mark.parametrize("m", [1, 4, 16, 33, 64, 65, 130])
def test_ragged_k(t, n, k, m, cuda):
    """Q8_0 and Q4_0 rows whose blocks do not fill the tiles' last chunk (64 values for Q8_0, 128 for Q4_0): its
    remaining blocks are padding (zero quants, zero scale)"""
    _matmul_case(t, n, k, m, cuda)


def _matmul_case(t, n, k, m, cuda):
    rng = np.random.default_rng([n, k, m, 122])
    raw = G.RAW[t](rng, n, k)
    xb, x = _x(rng, m, k, cuda)
    ref = R.bf16_to_f32(xb).astype(np.float64) @ R.dequant(raw, t, k).astype(np.float64).T
    p = KQ.repack_host(t, raw, (n, k), tiled=True).to(cuda)
    plan = LIB.plan_str(KQ.TILED[t], m, n, k)
    print(f"{NAME[t]} tiles m={m} n={n} k={k} {plan}", flush=True)
    y = KQ.matmul(x, p).cpu().numpy()
    assert_product(y, ref, f"{NAME[t]} tiles m={m} n={n} k={k} ({plan})")
    yb = KQ.matmul(x, p, out_dtype=torch.bfloat16)
    assert np.array_equal(yb.view(torch.int16).cpu().numpy().view(np.uint16), R.bf16_round(y))
    if m == 1:
        assert LIB.gemm_plan(KQ.TILED[t], m, n, k)[0] == LIB.KERNEL_GEMV
    elif m <= 64:
        assert LIB.gemm_plan(KQ.TILED[t], m, n, k)[0] == LIB.KERNEL_KGROUP
    else:                                                       # the row-major planes' plan: the same bits
        assert plan == LIB.plan_str(t, m, n, k)
        rm = KQ.repack_host(t, raw, (n, k)).to(cuda)
        assert np.array_equal(y.view(np.uint32), KQ.matmul(x, rm).cpu().numpy().view(np.uint32))


@pytest.mark.parametrize("t", TYPES, ids=NAME.get)
@pytest.mark.parametrize("m", [1, 4, 16, 17, 33, 64])
@pytest.mark.parametrize("n,k", [(1000, 256 * 9), (4500, 1024), (70, 768)])
def test_kgroup_every_split_count(t, m, n, k, forced_plan, cuda):
    """the K-group kernel on tiled planes at every split count the planner can take (each fixes rows per block, row
    groups and tiles per wave), on row counts whose block ranges start and end inside 16-row tiles and K ranges whose
    splits end inside super-blocks (a chunk is half a super-block), against the float64 product; a split K repeats bit
    for bit"""
    rng = np.random.default_rng([m, n, k, 123])
    raw = G.RAW[t](rng, n, k)
    xb, x = _x(rng, m, k, cuda)
    ref = R.bf16_to_f32(xb).astype(np.float64) @ R.dequant(raw, t, k).astype(np.float64).T
    p = KQ.repack_host(t, raw, (n, k), tiled=True).to(cuda)
    for splits in (0, 1, 2, 3, 4, 6, 8):
        if splits > k // 128:
            continue
        forced_plan(LIB.KERNEL_KGROUP, 0, 0, splits)
        try:
            plan = LIB.gemm_plan(KQ.TILED[t], m, n, k)
        except LIB.MbqError as e:
            # a forced split count whose row ranges need more tiles per wave than the kernel holds (Q4_K at 33-64 rows:
            # 5) has no plan; the call is refused the same way, with nothing launched. The automatic plan always runs.
            assert splits > 0 and "no plan" in str(e), e
            with pytest.raises(LIB.MbqError):
                KQ.matmul(x, p)
            continue
        plan = LIB.gemm_plan(KQ.TILED[t], m, n, k)
        assert plan[0] == LIB.KERNEL_KGROUP and (splits == 0 or plan[3] == splits), plan
        print(f"{NAME[t]} tiles kgroup m={m} n={n} k={k} plan {plan}", flush=True)
        y = KQ.matmul(x, p).cpu().numpy()
        assert_product(y, ref, f"{NAME[t]} tiles kgroup m={m} n={n} k={k} plan {plan}")
        assert np.array_equal(KQ.matmul(x, p).cpu().numpy().view(np.uint32), y.view(np.uint32))


@pytest.mark.parametrize("t", TYPES, ids=NAME.get)
def test_stream_plan_refused(t, forced_plan, cuda):
    """the weight-stream kernel reads row-major planes only: a forced stream plan on tiled planes is an error, not a
    launch"""
    rng = np.random.default_rng(124)
    raw = G.RAW[t](rng, 64, 512)
    p = KQ.repack_host(t, raw, (64, 512), tiled=True).to(cuda)
    _, x = _x(rng, 8, 512, cuda)
    forced_plan(LIB.KERNEL_STREAM, 16, 64, 1)
    with pytest.raises(LIB.MbqError):
        KQ.matmul(x, p)


@pytest.mark.parametrize("t", TYPES, ids=NAME.get)
@pytest.mark.parametrize("m", [1, 4, 64, 300])
def test_stack_read_in_place(t, m, cuda):
    """a stack of 3 weights repacked at once; layer= as an int and as a device int32 reads one in place; a device layer
    outside the stack gives NaN"""
    rng = np.random.default_rng([m, 125])
    n, k, L = 70, 768, 3
    st = np.stack([G.RAW[t](rng, n, k) for _ in range(L)])
    p = KQ.repack(t, torch.from_numpy(st).to(cuda), (n, k), tiled=True)
    xb, x = _x(rng, m, k, cuda)
    xf = R.bf16_to_f32(xb).astype(np.float64)
    for layer in range(L):
        ref = xf @ R.dequant(st[layer], t, k).astype(np.float64).T
        assert_product(KQ.matmul(x, p, layer=layer).cpu().numpy(), ref, f"layer {layer}")
        got = KQ.matmul(x, p, layer=torch.tensor(layer, dtype=torch.int32, device=cuda)).cpu().numpy()
        assert_product(got, ref, f"device layer {layer}")
        assert np.array_equal(got.view(np.uint32), KQ.matmul(x, p[layer]).cpu().numpy().view(np.uint32))
    bad = KQ.matmul(x, p, layer=torch.tensor(L, dtype=torch.int32, device=cuda)).cpu().numpy()
    assert np.all(np.isnan(bad))


@pytest.mark.parametrize("t", TYPES, ids=NAME.get)
@pytest.mark.parametrize("m", [1, 4, 16])
def test_27b_layer_at_decode_buckets(t, m, cuda):
    """the 7 projections of a 27B-class layer at the engine's row buckets 1, 4 and 16 (reference
    src/mashbox/runtime/engine.py:424-428; one row: the tile GEMV, 4 and 16: the K-group kernel): every output against
    the float64 product (on the GPU) of the oracle's dequantization"""
    rng = np.random.default_rng([m, 126])
    for name, (n, k) in G.LAYER_27B.items():
        raw = G.RAW[t](rng, n, k)
        xb, x = _x(rng, m, k, cuda)
        p = KQ.repack(t, torch.from_numpy(raw).to(cuda), (n, k), tiled=True)
        print(f"{NAME[t]} tiles 27B {name} m={m} ({LIB.plan_str(KQ.TILED[t], m, n, k)})", flush=True)
        y = KQ.matmul(x, p)
        w64 = torch.from_numpy(R.dequant(raw, t, k)).to(cuda).to(torch.float64)
        assert_product_dev(y, x.to(torch.float64) @ w64.T, f"27B {name} m={m} ({LIB.plan_str(KQ.TILED[t], m, n, k)})")
        del w64, y
        torch.cuda.empty_cache()


@pytest.mark.parametrize("t", TYPES, ids=NAME.get)
def test_noalloc_equals_matmul(t, forced_plan, cuda):
    """mbq_matmul_noalloc on tiled planes (split-K partials in the static scratch) gives mbq_matmul's bits, on two calls
    in a row, the second smaller"""
    rng = np.random.default_rng(127)
    n, k = 1024, 5120
    raw = G.RAW[t](rng, n, k)
    p = KQ.repack_host(t, raw, (n, k), tiled=True).to(cuda)
    forced_plan(LIB.KERNEL_KGROUP, 0, 0, 4)
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    for m in (16, 5):
        _, x = _x(rng, m, k, cuda)
        want = KQ.matmul(x, p)
        got = torch.empty_like(want)
        assert LIB.lib().mbq_matmul_noalloc(KQ.TILED[t], ctypes.c_void_p(p.buf.data_ptr()), 0, None, 1,
                                            ctypes.c_void_p(x.data_ptr()), m, n, k, ctypes.c_void_p(got.data_ptr()),
                                            LIB.OUT_F32, stream) == 0
        assert torch.equal(got.view(torch.int32), want.view(torch.int32))


@pytest.mark.parametrize("t", TYPES, ids=NAME.get)
def test_kgroup_graph_replays(t, forced_plan, cuda):
    """a split-K K-group call on tiled planes recorded into a HIP graph replays bit for bit equal to the eager call,
    with eager calls of the same kernel in between"""
    rng = np.random.default_rng(128)
    m, n, k = 16, 1024, 5120
    raw = G.RAW[t](rng, n, k)
    p = KQ.repack_host(t, raw, (n, k), tiled=True).to(cuda)
    _, x = _x(rng, m, k, cuda)
    _, x2 = _x(rng, m, k, cuda)
    forced_plan(LIB.KERNEL_KGROUP, 0, 0, 4)
    eager = KQ.matmul(x, p).cpu().numpy()
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        y = KQ.matmul(x, p)
    for _ in range(3):
        g.replay()
        torch.cuda.synchronize()
        assert np.array_equal(y.cpu().numpy().view(np.uint32), eager.view(np.uint32))
        KQ.matmul(x2, p)
        torch.cuda.synchronize()


@pytest.mark.parametrize("t", TYPES, ids=NAME.get)
def test_ops_prepare_loads_tiles(t, monkeypatch, cuda):
    """by default the ops layer loads every GGUF type's weights (one and a stack) as tiles: qmatmul at 1, 4 and 300
    rows, layer= in place and dequant against the oracle; device_nbytes counts the tiled planes"""
    from mashbox_amd import ops
    monkeypatch.delenv("MBQ_LAYOUT", raising=False)
    ops.load_kernels()
    rng = np.random.default_rng(129)
    n, k, L = 100, 512, 2
    st = np.stack([G.RAW[t](rng, n, k) for _ in range(L)])
    h = ops.prepare(st[0], t, (n, k))
    hs = ops.prepare(st, t, (n, k))
    assert isinstance(h, ops.Packed) and h.packed.t == KQ.TILED[t] and hs.packed.t == KQ.TILED[t]
    assert ops.device_nbytes(t, (L, n, k), st.nbytes) == L * KQ.plane_bytes(KQ.TILED[t], (n, k))
    w = [R.dequant(st[i], t, k) for i in range(L)]
    assert diff_bits(ops.dequant(h).cpu().numpy(), w[0]) == 0
    for m in (1, 4, 300):
        xb, x = _x(rng, m, k, cuda)
        xf = R.bf16_to_f32(xb).astype(np.float64)
        assert_product(ops.qmatmul(x.float(), h).float().cpu().numpy(), xf @ w[0].astype(np.float64).T, f"prepare m={m}")
        for i in range(L):
            y = ops.qmatmul(x.float(), ops.At(hs.packed, i, t, (n, k))).float().cpu().numpy()
            assert_product(y, xf @ w[i].astype(np.float64).T, f"prepare stack layer {i} m={m}")


@pytest.mark.parametrize("t", TYPES, ids=NAME.get)
def test_default_prepare_at_decode_buckets(t, monkeypatch, cuda):
    """the ops layer's default prepare (no environment switch) serves a decoding server's row buckets 1, 4 and 16
    (reference src/mashbox/runtime/engine.py:424-428) from one load: every output against the float64 product of the
    oracle's dequantization, for one weight and for a layer of a stack read in place; layout "both" holds the
    row-major planes beside the tiles and runs one row on them (the decode GEMV's bits) and 4 and 16 rows on the tiles
    (the K-group kernel's bits)"""
    from mashbox_amd import ops
    monkeypatch.delenv("MBQ_LAYOUT", raising=False)
    ops.load_kernels()
    rng = np.random.default_rng([t, 130])
    n, k, L = 1000, 2048, 2
    st = np.stack([G.RAW[t](rng, n, k) for _ in range(L)])
    h = ops.prepare(st[1], t, (n, k))
    hs = ops.prepare(st, t, (n, k))
    assert h.packed.t == KQ.TILED[t] and h.packed.alt is None
    w64 = torch.from_numpy(R.dequant(st[1], t, k)).to(cuda).to(torch.float64)
    monkeypatch.setenv("MBQ_LAYOUT", "both")
    hb = ops.prepare(st[1], t, (n, k))
    assert hb.packed.t == KQ.TILED[t] and hb.packed.alt is not None and hb.packed.alt.t == t
    assert ops.device_nbytes(t, (n, k), st[1].nbytes) == KQ.plane_bytes(KQ.TILED[t], (n, k)) + KQ.plane_bytes(t, (n, k))
    rm = KQ.repack_host(t, st[1], (n, k)).to(cuda)
    for m in (1, 4, 16):
        xb, x = _x(rng, m, k, cuda)
        ref = x.to(torch.float64) @ w64.T
        print(f"{NAME[t]} default prepare m={m} ({LIB.plan_str(KQ.TILED[t], m, n, k)})", flush=True)
        y = ops.qmatmul(x, h)
        assert y.dtype == torch.bfloat16
        assert_product_dev(y, ref, f"{NAME[t]} default m={m}")
        ya = ops.qmatmul(x, ops.At(hs.packed, 1, t, (n, k)))
        assert torch.equal(ya.view(torch.int16), y.view(torch.int16)), f"{NAME[t]} stack layer m={m}"
        yb = ops.qmatmul(x, hb)
        want = KQ.matmul(x, rm if m == 1 else h.packed, out_dtype=torch.bfloat16)
        assert torch.equal(yb.view(torch.int16), want.view(torch.int16)), f"{NAME[t]} both m={m}"


@pytest.mark.parametrize("t", [R.Q4_K, R.Q8_0, R.Q6_K], ids=NAME.get)
def test_tile_gemv_long_rows(t, cuda):
    """one row of 28672 values (x staged in LDS in two batches; the 16-wave blocks of a 5120-row weight) and a 70-row
    weight whose single block holds a partial tile: every output against the float64 product of the oracle's
    dequantization, in float32 and bfloat16 (the bfloat16 output is the float32 one rounded)"""
    rng = np.random.default_rng([t, 131])
    for n, k in ((5120, 28672), (70, 28672)):
        assert LIB.gemm_plan(KQ.TILED[t], 1, n, k)[0] == LIB.KERNEL_GEMV
        raw = G.RAW[t](rng, n, k)
        xb, x = _x(rng, 1, k, cuda)
        p = KQ.repack(t, torch.from_numpy(raw).to(cuda), (n, k), tiled=True)
        print(f"{NAME[t]} tile GEMV {n}x{k}", flush=True)
        y = KQ.matmul(x, p)
        w64 = torch.from_numpy(R.dequant(raw, t, k)).to(cuda).to(torch.float64)
        assert_product_dev(y, x.to(torch.float64) @ w64.T, f"{NAME[t]} tile GEMV {n}x{k}")
        yb = KQ.matmul(x, p, out_dtype=torch.bfloat16)
        assert np.array_equal(yb.view(torch.int16).cpu().numpy().view(np.uint16), R.bf16_round(y.cpu().numpy()))
        del w64
        torch.cuda.empty_cache()


def test_every_covered_shape_has_a_plan(cuda):
    """every weight that mbq_covers accepts has a plan at every batch size, on row-major planes, tiled planes and int8
    (a plan query launches nothing): tall weights (more rows per CU than a wave's tiles hold) take several rounds of
    K-group blocks, and 1-4 rows of K beyond what x in registers holds take x through LDS"""
    types = [R.Q4_0, R.Q8_0, R.Q4_K, R.Q5_K, R.Q6_K] + [KQ.TILED[t] for t in TYPES] + [LIB.INT8, LIB.I8T]
    quant_k = {R.Q4_K, R.Q5_K, R.Q6_K, KQ.TILED[R.Q4_K], KQ.TILED[R.Q5_K], KQ.TILED[R.Q6_K]}
    ns = (1, 16, 70, 1024, 5120, 17408, 24576, 28672, 34816, 53248, 151936)
    ks = (256, 2560, 5120, 8192, 17408, 28672, 41216, 53248)
    ms = (1, 2, 3, 4, 5, 8, 9, 16, 17, 32, 33, 48, 64, 65, 2048)
    checked = 0
    for t in types:
        for n in ns:
            for k in ks:
                if t in quant_k and k % 256:
                    continue
                if not LIB.lib().mbq_covers(int(t), n, k):
                    continue
                for m in ms:
                    try:
                        LIB.gemm_plan(t, m, n, k)
                    except LIB.MbqError as e:
                        pytest.fail(f"type {t} m={m} n={n} k={k}: {e}")
                    checked += 1
    print(f"{checked} covered (type, m, n, k) have a plan", flush=True)
    assert checked > 10000


@pytest.mark.parametrize("t,n,k,ms", [
    (R.Q4_K, 34816, 512, (2, 4, 8, 16, 64)),       # gate|up stacked: two rounds of K-group blocks at 2-8 rows
    (R.Q5_K, 34816, 512, (4,)),
    (R.Q8_0, 34816, 512, (4, 64)),
    (R.Q6_K, 151936, 256, (4, 16, 64)),            # a vocabulary head's rows: four to seven rounds
    (R.Q4_K, 12416, 5376, (4,)),                   # two K splits over two rounds
    (R.Q4_K, 300, 41216, (2, 4)),                  # K past x in registers: the diagonal x tiles through LDS
    (R.Q4_0, 300, 41216, (3,)),
], ids=lambda v: NAME.get(v) if isinstance(v, int) and v in NAME else str(v))
def test_tall_and_long_weights(t, n, k, ms, cuda):
    """weights the K-group kernel runs in several rounds of blocks, or with x staged in LDS at 1-4 rows: every output
    against the float64 product (on the GPU) of the oracle's dequantization, in float32 and bfloat16 (the float32
    result rounded), and a second call repeats bit for bit"""
    rng = np.random.default_rng([t, n, k, 132])
    raw = G.RAW[t](rng, n, k)
    p = KQ.repack(t, torch.from_numpy(raw).to(cuda), (n, k), tiled=True)
    w64 = torch.from_numpy(R.dequant(raw, t, k)).to(cuda).to(torch.float64)
    for m in ms:
        plan = LIB.gemm_plan(KQ.TILED[t], m, n, k)
        assert plan[0] == LIB.KERNEL_KGROUP, plan
        print(f"{NAME[t]} tiles m={m} {n}x{k} ({LIB.plan_str(KQ.TILED[t], m, n, k)})", flush=True)
        xb, x = _x(rng, m, k, cuda)
        y = KQ.matmul(x, p)
        assert_product_dev(y, x.to(torch.float64) @ w64.T, f"{NAME[t]} tiles m={m} {n}x{k}")
        yb = KQ.matmul(x, p, out_dtype=torch.bfloat16)
        assert np.array_equal(yb.view(torch.int16).cpu().numpy().view(np.uint16), R.bf16_round(y.cpu().numpy()))
        assert torch.equal(KQ.matmul(x, p).view(torch.int32), y.view(torch.int32))
        # the allocation-free entry point runs the same plan (split partials in its static scratch): the same bits
        got = torch.empty_like(y)
        assert LIB.lib().mbq_matmul_noalloc(KQ.TILED[t], ctypes.c_void_p(p.buf.data_ptr()), 0, None, 1,
                                            ctypes.c_void_p(x.data_ptr()), m, n, k, ctypes.c_void_p(got.data_ptr()),
                                            LIB.OUT_F32, ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)) == 0
        assert torch.equal(got.view(torch.int32), y.view(torch.int32))
    del w64
    torch.cuda.empty_cache()
