"""GPU parity: the gfx950 kernels of libmbq.so against the CPU oracle (oracle/ref.py) on the same seeded inputs.

Mirrors the reference's own bars:
  dequant: bit for bit, NaN where the reference has NaN, on random bytes with all-zero and all-0xFF blocks
           (reference tests/cpu/test_gguf_dequant.py:17-45; contract rule src/mashbox/ops/__init__.py:691-705)
  matmul:  NMSE <= 2e-5 against the float64 product of the exact weights (reference tests/contracts/test_ops.py:28-31)
           and max |y - ref| / max |ref| <= 1e-2; weight rows 1..130, K 1..16 blocks, activation rows 1..130,
           leading axes, empty batches (reference tests/cpu/test_moe_bundle_dense.py:108-128)
  int8:    the same product bars for reference src/mashbox/models/qwen3_8_27b/model.py:72-82
Full-size BASELINE configs: every output of configs 1-5 compared whole.
"""
import numpy as np
import pytest
import torch

from oracle import gen as G
from oracle import ref as R
from tests._check import assert_product, assert_product_dev, diff_bits

import mashbox_amd.kernels as KQ
from mashbox_amd import int8 as I8

pytestmark = pytest.mark.gpu

TYPES = [R.Q4_0, R.Q8_0, R.Q4_K, R.Q5_K, R.Q6_K]
NAME = {R.Q4_0: "Q4_0", R.Q8_0: "Q8_0", R.Q4_K: "Q4_K", R.Q5_K: "Q5_K", R.Q6_K: "Q6_K"}
GEMM_TYPES = [R.Q4_0, R.Q8_0, R.Q4_K, R.Q5_K, R.Q6_K, "int8"]
GEMM_IDS = ["Q4_0", "Q8_0", "Q4_K", "Q5_K", "Q6_K", "int8"]
KQUANT = (R.Q4_K, R.Q5_K, R.Q6_K)                     # rows of whole 256-value super-blocks
UNIT32 = (R.Q4_0,) + KQUANT                           # GEMV units of 32 values


def _bf16_tensor(bits: np.ndarray, dev) -> torch.Tensor:
    return torch.from_numpy(bits.astype(np.int16)).view(torch.bfloat16).to(dev)


def _random_blocks(t, rows, kb, rng):
    bs = R.TYPES[t][1]
    cols = bs * kb
    raw = rng.integers(0, 256, size=(rows, R.row_bytes(t, cols)), dtype=np.uint8)
    raw[0] = 0
    raw[1] = 0xFF
    return raw, cols


@pytest.mark.parametrize("t", TYPES, ids=NAME.get)
@pytest.mark.parametrize("kb", [1, 2, 16])
def test_dequant_bit_exact_on_random_bytes(t, kb, cuda):
    rng = np.random.default_rng(1000 + t + kb)
    raw, cols = _random_blocks(t, 6, kb, rng)
    planes = KQ.repack_host(t, raw, (6, cols)).to(cuda)
    got = KQ.dequant(planes).cpu().numpy()
    assert diff_bits(got, R.dequant(raw, t, cols)) == 0


@pytest.mark.parametrize("t", TYPES, ids=NAME.get)
def test_dequant_leading_axes(t, cuda):
    """a stack (L, rows, row_bytes) dequantizes as one tensor at a time (test_gguf_dequant.py:48-56)"""
    rng = np.random.default_rng(2000 + t)
    raw, cols = _random_blocks(t, 6, 2, rng)
    st = np.stack([raw, raw[::-1]])
    planes = KQ.repack_host(t, st, (6, cols)).to(cuda)
    got = KQ.dequant(planes).cpu().numpy()
    for i in range(2):
        assert diff_bits(got[i], R.dequant(st[i], t, cols)) == 0
        assert diff_bits(KQ.dequant(planes, layer=i).cpu().numpy(), R.dequant(st[i], t, cols)) == 0


@pytest.mark.parametrize("t", TYPES, ids=NAME.get)
def test_device_repack_equals_host_repack(t, cuda):
    rng = np.random.default_rng(3000 + t)
    raw, cols = _random_blocks(t, 37, 3, rng)
    host = KQ.repack_host(t, raw, (37, cols))
    dev = KQ.repack(t, torch.from_numpy(raw).to(cuda), (37, cols))
    assert torch.equal(host.buf, dev.buf.cpu())


@pytest.mark.parametrize("t", TYPES, ids=NAME.get)
def test_device_repack_zeroes_the_padding_of_a_dirty_buffer(t, cuda):
    """mbq_repack_dev into a buffer full of 0xAB: the planes and their alignment padding equal the host repack's bytes
    (the padding is cleared by a fill kernel, so a captured repack replays the same)"""
    import ctypes
    from mashbox_amd import _lib as L
    rng = np.random.default_rng(3100 + t)
    raw, cols = _random_blocks(t, 13, 3, rng)
    host = KQ.repack_host(t, raw, (13, cols)).buf
    planes = torch.full((host.numel(),), 0xAB, dtype=torch.uint8, device=cuda)
    raw_d = torch.from_numpy(raw).to(cuda)
    rc = L.lib().mbq_repack_dev(t, ctypes.c_void_p(raw_d.data_ptr()), 13, cols, ctypes.c_void_p(planes.data_ptr()),
                                ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
    assert rc == 0
    assert torch.equal(planes.cpu(), host)


MM_SHAPES = [(1, 1), (9, 2), (37, 3), (130, 4)]        # (weight rows N, K in blocks)
MM_ROWS = [1, 2, 3, 4, 5, 16, 64, 130]


@pytest.mark.parametrize("t", TYPES, ids=NAME.get)
@pytest.mark.parametrize("n,kb", MM_SHAPES)
@pytest.mark.parametrize("m", MM_ROWS)
def test_matmul_matches_exact_product(t, n, kb, m, cuda):
    rng = np.random.default_rng([t, n, kb, m])
    k = R.TYPES[t][1] * kb
    raw = G.RAW[t](rng, n, k)
    xb = G.acts(rng, m, k)
    planes = KQ.repack_host(t, raw, (n, k)).to(cuda)
    x = _bf16_tensor(xb, cuda)
    y = KQ.matmul(x, planes).cpu().numpy()
    assert y.dtype == np.float32 and y.shape == (m, n)
    w = R.dequant(raw, t, k).astype(np.float64)
    ref = R.bf16_to_f32(xb).astype(np.float64) @ w.T
    assert_product(y, ref, f"{NAME[t]} m={m} n={n} k={k}")
    yb = KQ.matmul(x, planes, out_dtype=torch.bfloat16)
    assert yb.dtype == torch.bfloat16
    # the bf16 output is the f32 output rounded to nearest even (ops casts the f32 result to x.dtype)
    assert np.array_equal(yb.view(torch.int16).cpu().numpy().view(np.uint16), R.bf16_round(y))


@pytest.mark.parametrize("t", TYPES, ids=NAME.get)
@pytest.mark.parametrize("lead", [(2, 3), (1, 1, 5), (24,)])
def test_matmul_leading_axes(t, lead, cuda):
    rng = np.random.default_rng([t, len(lead)])
    n, k = 21, R.TYPES[t][1] * 2
    raw = G.RAW[t](rng, n, k)
    xb = G.acts(rng, int(np.prod(lead)), k)
    planes = KQ.repack_host(t, raw, (n, k)).to(cuda)
    y = KQ.matmul(_bf16_tensor(xb, cuda).reshape(lead + (k,)), planes)
    assert tuple(y.shape) == lead + (n,)
    ref = R.bf16_to_f32(xb).astype(np.float64) @ R.dequant(raw, t, k).astype(np.float64).T
    assert_product(y.reshape(-1, n).cpu().numpy(), ref)


@pytest.mark.parametrize("lead", [(0,), (2, 0)])
def test_empty_batch_gives_an_empty_result(lead, cuda):
    n, k = 8, 256
    raw = G.q4_k_raw(np.random.default_rng(0), n, k)
    planes = KQ.repack_host(R.Q4_K, raw, (n, k)).to(cuda)
    y = KQ.matmul(torch.zeros(lead + (k,), dtype=torch.bfloat16, device=cuda), planes)
    assert tuple(y.shape) == lead + (n,) and y.dtype == torch.float32


@pytest.mark.parametrize("t", TYPES, ids=NAME.get)
@pytest.mark.parametrize("m", [1, 4, 64])
def test_layer_reads_one_weight_of_a_stack_in_place(t, m, cuda):
    rng = np.random.default_rng([t, m, 7])
    n, k, L = 33, R.TYPES[t][1] * 2, 3
    st = np.stack([G.RAW[t](rng, n, k) for _ in range(L)])
    xb = G.acts(rng, m, k)
    planes = KQ.repack_host(t, st, (n, k)).to(cuda)
    x = _bf16_tensor(xb, cuda)
    xf = R.bf16_to_f32(xb).astype(np.float64)
    for layer in range(L):
        ref = xf @ R.dequant(st[layer], t, k).astype(np.float64).T
        assert_product(KQ.matmul(x, planes, layer=layer).cpu().numpy(), ref, f"host layer {layer}")
        dl = torch.tensor(layer, dtype=torch.int32, device=cuda)
        got = KQ.matmul(x, planes, layer=dl).cpu().numpy()
        assert_product(got, ref, f"device layer {layer}")
        assert np.array_equal(got, KQ.matmul(x, planes[layer]).cpu().numpy())
    bad = KQ.matmul(x, planes, layer=torch.tensor(L, dtype=torch.int32, device=cuda)).cpu().numpy()
    assert np.all(np.isnan(bad)), "a device layer outside the stack must give NaN, never an out-of-range read"


@pytest.mark.parametrize("m", [1, 2, 3, 4, 5, 64, 130])
@pytest.mark.parametrize("n,k", [(7, 16), (33, 48), (130, 4096)])
def test_int8_linear_matches_reference(m, n, k, cuda):
    rng = np.random.default_rng([m, n, k])
    xb = G.acts(rng, m, k)
    q, s = G.int8_weights(rng, n, k)
    w = {"q": torch.from_numpy(q).to(cuda), "s": torch.from_numpy(s).to(cuda)}
    x = _bf16_tensor(xb, cuda)
    ref = (R.bf16_to_f32(xb).astype(np.float64) @ q.astype(np.float64).T) * s.astype(np.float64)
    yf = I8.linear(x, w, pj=lambda v: v).float().cpu().numpy()
    assert_product(yf, ref, f"int8 m={m} n={n} k={k}")
    y = I8.linear(x, w)
    assert y.dtype == torch.bfloat16 and tuple(y.shape) == (m, n)
    assert_product(y.float().cpu().numpy(), ref)
    # the oracle's float32 restatement rounds the same way within the bar
    assert_product(R.int8_linear(R.bf16_to_f32(xb), q, s), ref)


# --------------------------------------------------------------------------------- full-size BASELINE configs
@pytest.mark.parametrize("idx", [1, 2, 3])
def test_decode_gemv_full_config(idx, cuda):
    cfg = G.config(idx, seed=0)
    (_, n, k, wts, xb), = cfg["projections"]
    x = _bf16_tensor(xb, cuda)
    xf = R.bf16_to_f32(xb).astype(np.float64)
    if cfg["t"] == "int8":
        q, s = wts
        y = I8.linear(x, {"q": torch.from_numpy(q).to(cuda), "s": torch.from_numpy(s).to(cuda)}, pj=lambda v: v)
        ref = (xf @ q.astype(np.float64).T) * s
    else:
        planes = KQ.repack_host(cfg["t"], wts, (n, k)).to(cuda)
        got_w = KQ.dequant(planes).cpu().numpy()
        w = R.dequant(wts, cfg["t"], k)
        assert diff_bits(got_w, w) == 0
        y = KQ.matmul(x, planes)
        ref = xf @ w.astype(np.float64).T
    assert_product(y.float().cpu().numpy(), ref, f"config {idx}")


@pytest.mark.parametrize("idx", [4, 5])
def test_batched_gemm_full_config(idx, cuda):
    """full-size configs 4 and 5 (seed 0): every output of every projection, the last M and N tiles included, against
    the float64 product (on the GPU) of the oracle's exact weights: int8 q * s, or the oracle's dequantization of the
    Q4_K blocks; every output finite (reference tests/contracts/test_ops.py:19-35,51)"""
    cfg = G.config(idx, seed=0)
    for name, n, k, wts, xb in cfg["projections"]:
        print(f"config {idx} {name} {xb.shape[0]}x{n}x{k}", flush=True)
        x = _bf16_tensor(xb, cuda)
        x64 = x.to(torch.float64)
        if cfg["t"] == "int8":
            q, s = wts
            w = {"q": torch.from_numpy(q).to(cuda), "s": torch.from_numpy(s).to(cuda)}
            got = []
            I8.linear(x, w, pj=lambda v: got.append(v.clone()) or v)
            y = got[0]
            ref = (x64 @ w["q"].to(torch.float64).T) * w["s"].to(torch.float64)
        else:
            planes = KQ.repack_host(cfg["t"], wts, (n, k)).to(cuda)
            y = KQ.matmul(x, planes)
            w64 = torch.from_numpy(R.dequant(wts, cfg["t"], k)).to(cuda).to(torch.float64)
            ref = x64 @ w64.T
            del w64
        assert_product_dev(y, ref, f"config {idx} {name} ({LIB.plan_str(-8 if cfg['t'] == 'int8' else cfg['t'], xb.shape[0], n, k)})")
        del y, ref
        torch.cuda.empty_cache()


@pytest.mark.parametrize("t", UNIT32, ids=NAME.get)
@pytest.mark.parametrize("m", [3, 4])
def test_gemv_row_parts_past_the_row_end(t, m, cuda):
    """K = 8448 (264 units of 32 values) at 3-4 activation rows: the GEMV cuts a K-quant row into 8 parts of 40 units
    (Q4_0: 33), so the last part starts past the row's end and holds nothing; the block's sum over the parts must leave
    it out"""
    rng = np.random.default_rng([t, m, 8448])
    n, k = 70, 8448
    raw = G.RAW[t](rng, n, k)
    xb = G.acts(rng, m, k)
    planes = KQ.repack_host(t, raw, (n, k)).to(cuda)
    y = KQ.matmul(_bf16_tensor(xb, cuda), planes).cpu().numpy()
    ref = R.bf16_to_f32(xb).astype(np.float64) @ R.dequant(raw, t, k).astype(np.float64).T
    assert_product(y, ref, f"{NAME[t]} m={m} k={k}")


@pytest.mark.parametrize("t", GEMM_TYPES, ids=GEMM_IDS)
@pytest.mark.parametrize("n", [1, 3, 4, 5, 130, 1027])
def test_gemv_rows_of_80_units_packed_four_to_an_item(t, n, cuda):
    """one activation row over rows of 80 units (2560 K-quant values, 1280 Q8_0 / int8 values): the GEMV packs 4 rows
    into an item of 5 chunks; row counts that are not multiples of 4 leave a partial last group; a stack read at a
    device layer (and one outside the stack: NaN) takes the same path"""
    rng = np.random.default_rng([n, 80, 0 if t == "int8" else t])
    k = 1280 if t in ("int8", R.Q8_0) else 2560
    xb = G.acts(rng, 1, k)
    x = _bf16_tensor(xb, cuda)
    xf = R.bf16_to_f32(xb).astype(np.float64)
    if t == "int8":
        q, sc = G.int8_weights(rng, n, k)
        y = _int8_f32(x, {"q": torch.from_numpy(q).to(cuda), "s": torch.from_numpy(sc).to(cuda)})
        assert_product(y, (xf @ q.astype(np.float64).T) * sc, f"int8 n={n}")
        return
    st = np.stack([G.RAW[t](rng, n, k) for _ in range(2)])
    planes = KQ.repack_host(t, st, (n, k)).to(cuda)
    for layer in range(2):
        ref = xf @ R.dequant(st[layer], t, k).astype(np.float64).T
        assert_product(KQ.matmul(x, planes, layer=layer).cpu().numpy(), ref, f"{NAME[t]} n={n} layer {layer}")
        dl = torch.tensor(layer, dtype=torch.int32, device=cuda)
        assert_product(KQ.matmul(x, planes, layer=dl).cpu().numpy(), ref, f"{NAME[t]} n={n} device layer {layer}")
    bad = KQ.matmul(x, planes, layer=torch.tensor(2, dtype=torch.int32, device=cuda)).cpu().numpy()
    assert np.all(np.isnan(bad))


@pytest.mark.parametrize("t", GEMM_TYPES, ids=GEMM_IDS)
@pytest.mark.parametrize("m", [16, 17, 64])
def test_small_batches_over_tall_weights(t, m, cuda):
    """17-64 activation rows over a weight of at least 64 rows per CU take the LDS-tile kernel's 64 x 128 tiles,
    16 rows the weight stream; both give the exact product (a sample of 512 weight rows compared)"""
    n = 64 * torch.cuda.get_device_properties(0).multi_processor_count + 37
    k = 512 if t != "int8" else 272
    tt = -8 if t == "int8" else t
    kind, bm, bn, _ = LIB.gemm_plan(tt, m, n, k)
    assert (kind, bm, bn) == ((LIB.KERNEL_STREAM, 16, 128) if m == 16 else (LIB.KERNEL_TILES, 64, 128))
    rng = np.random.default_rng([m, n, 0 if t == "int8" else t])
    run, ref = _direct_case(t, m, n, k, rng, cuda)
    ns = np.sort(rng.choice(n, 512, replace=False))
    assert_product(run()[:, ns], ref[:, ns], f"{t} m={m} n={n}")


@pytest.mark.parametrize("t", UNIT32, ids=NAME.get)
@pytest.mark.parametrize("n", [1, 7, 300])
def test_gemv_rows_in_three_parts(t, n, cuda):
    """K = 17408 (544 units) at one activation row cuts a row into 3 parts of 184, 184 and 176 units, taken by 3, 3
    and 2 of a block's 8 waves; the block adds the parts through LDS"""
    rng = np.random.default_rng([t, n, 17408])
    k = 17408
    raw = G.RAW[t](rng, n, k)
    xb = G.acts(rng, 1, k)
    planes = KQ.repack_host(t, raw, (n, k)).to(cuda)
    y = KQ.matmul(_bf16_tensor(xb, cuda), planes).cpu().numpy()
    ref = R.bf16_to_f32(xb).astype(np.float64) @ R.dequant(raw, t, k).astype(np.float64).T
    assert_product(y, ref, f"{NAME[t]} n={n}")


def test_q6_k_output_head_full_size_sampled(cuda):
    """the reference's published Q6_K shape (an output head of 151936 x 2560, one activation row; reference
    CORE-CHANGES.md:73): repacked on the GPU from the file's blocks, run whole by the decode GEMV, and a seeded sample of
    2048 rows compared with the exact product; two and four activation rows the same way"""
    n, k = 151936, 2560
    rng = np.random.default_rng(14)
    raw = G.q6_k_raw(rng, n, k)
    planes = KQ.repack(R.Q6_K, torch.from_numpy(raw).to(cuda), (n, k))
    ns = np.sort(rng.choice(n, 2048, replace=False))
    w = R.dequant(raw[ns], R.Q6_K, k).astype(np.float64)
    assert diff_bits(KQ.dequant(planes).cpu().numpy()[ns], w.astype(np.float32)) == 0
    for m in (1, 2, 4):
        xb = G.acts(rng, m, k)
        y = KQ.matmul(_bf16_tensor(xb, cuda), planes).cpu().numpy()
        assert np.all(np.isfinite(y))
        assert_product(y[:, ns], R.bf16_to_f32(xb).astype(np.float64) @ w.T, f"Q6_K head m={m}")


def test_q4_0_config_2_shape_full_size_sampled(cuda):
    """Q4_0 at config 2's weight shape (17408 x 5120), repacked on the GPU from the file's blocks; dequant of a seeded
    sample of 1024 rows bit for bit, and the decode GEMV (1 row), the weight stream (16 rows) and the LDS tiles (64
    rows over a weight this tall, and 300 rows) on the same sample within the product bars"""
    n, k = 17408, 5120
    rng = np.random.default_rng(2)
    raw = G.q4_0_raw(rng, n, k)
    planes = KQ.repack(R.Q4_0, torch.from_numpy(raw).to(cuda), (n, k))
    ns = np.sort(rng.choice(n, 1024, replace=False))
    w = R.dequant(raw[ns], R.Q4_0, k)
    assert diff_bits(KQ.dequant(planes).cpu().numpy()[ns], w) == 0
    for m, kind in ((1, LIB.KERNEL_GEMV), (16, LIB.KERNEL_STREAM), (64, LIB.KERNEL_TILES), (300, LIB.KERNEL_TILES)):
        assert LIB.gemm_plan(R.Q4_0, m, n, k)[0] == kind
        xb = G.acts(rng, m, k)
        y = KQ.matmul(_bf16_tensor(xb, cuda), planes).cpu().numpy()
        assert np.all(np.isfinite(y))
        assert_product(y[:, ns], R.bf16_to_f32(xb).astype(np.float64) @ w.astype(np.float64).T, f"Q4_0 m={m}")


# ------------------------------------------------------------------------------------------------ golden fixtures
import os  # noqa: E402

_GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def _kernel_fixtures():
    """the committed fixtures of the kernel types (the exact path's other types: tests/test_gpu_raw_types.py)"""
    out = []
    for f in sorted(f for f in os.listdir(_GOLDEN) if f.endswith(".npz")):
        if int(np.load(os.path.join(_GOLDEN, f), allow_pickle=False)["t"]) in R.KERNEL_TYPES:
            out.append(f)
    return out


@pytest.mark.parametrize("name", _kernel_fixtures())
def test_golden_fixture(name, cuda):
    """committed fixtures (random bytes with zero / 0xFF rows; real llama-quantize blocks of the reference's fixture
    models): dequant bit for bit, and the product within the bars"""
    z = np.load(os.path.join(_GOLDEN, name), allow_pickle=False)
    t, cols, raw = int(z["t"]), int(z["cols"]), z["raw"]
    rows = raw.shape[0]
    planes = KQ.repack_host(t, raw, (rows, cols)).to(cuda)
    assert diff_bits(KQ.dequant(planes).cpu().numpy(), z["w"]) == 0
    dev_planes = KQ.repack(t, torch.from_numpy(raw).to(cuda), (rows, cols))
    assert torch.equal(dev_planes.buf, planes.buf)
    if "x" in z.files:
        for m in (1, 3):
            y = KQ.matmul(_bf16_tensor(z["x"][:m], cuda), planes).cpu().numpy()
            assert_product(y, z["y64"][:m], name)


# ------------------------------------------------------------------------------------ every GEMM tile shape, split-K
from mashbox_amd import _lib as LIB  # noqa: E402

GEMM_TILES = [(256, 256), (256, 192), (256, 128), (128, 256), (128, 192), (128, 128), (128, 64), (64, 256), (64, 192),
              (64, 128), (64, 64)]


def _int8_f32(x, w):
    """the float32 y * s that the int8 linear hands its pj hook, before the rounding to x's dtype"""
    got = []
    I8.linear(x, w, pj=lambda v: got.append(v.clone()) or v)
    return got[0].cpu().numpy()


@pytest.fixture
def forced_plan():
    yield LIB.force_gemm_plan
    LIB.force_gemm_plan()


@pytest.mark.parametrize("t", GEMM_TYPES, ids=GEMM_IDS)
@pytest.mark.parametrize("bm,bn", GEMM_TILES)
def test_every_gemm_tile_shape_with_and_without_split(t, bm, bn, forced_plan, cuda):
    """partial tiles on both edges, K over several steps (a Q8_0 / int8 K that is not a multiple of the 64-value step
    included, Q4_0 the same), split-K into 3 ranges against 1"""
    rng = np.random.default_rng([bm, bn, 0 if t == "int8" else t])
    m, n = bm + bm // 2 - 3, bn + 17
    k = {R.Q4_0: 32 * 13, R.Q8_0: 32 * 13, R.Q4_K: 256 * 3, R.Q5_K: 256 * 3, R.Q6_K: 256 * 3, "int8": 16 * 25}[t]
    xb = G.acts(rng, m, k)
    x = _bf16_tensor(xb, cuda)
    xf = R.bf16_to_f32(xb).astype(np.float64)
    if t == "int8":
        q, s = G.int8_weights(rng, n, k)
        w = {"q": torch.from_numpy(q).to(cuda), "s": torch.from_numpy(s).to(cuda)}
        run = lambda: _int8_f32(x, w)
        ref = (xf @ q.astype(np.float64).T) * s
    else:
        raw = G.RAW[t](rng, n, k)
        planes = KQ.repack_host(t, raw, (n, k)).to(cuda)
        run = lambda: KQ.matmul(x, planes).cpu().numpy()
        ref = xf @ R.dequant(raw, t, k).astype(np.float64).T
    outs = []
    for splits in (1, 3):
        forced_plan(LIB.KERNEL_TILES, bm, bn, splits)
        assert LIB.gemm_plan(-8 if t == "int8" else t, m, n, k)[:3] == (LIB.KERNEL_TILES, bm, bn)
        y = run()
        assert_product(y, ref, f"{t} tile {bm}x{bn} splits {splits}")
        outs.append(y)
    # a split sums float32 partials in another order: close to, not bitwise equal to, one range
    assert np.max(np.abs(outs[0] - outs[1])) <= 1e-4 * np.max(np.abs(ref))


@pytest.mark.parametrize("t", TYPES, ids=NAME.get)
def test_specialized_gemm_bf16_output_tile_edges(t, forced_plan, cuda):
    """the 256 x 192 tile without a split (the specialized-wave kernel) with bfloat16 output, whose tile leaves through
    LDS in 16-byte chunks when N % 8 == 0: partial tiles on both edges (381 activation rows, 200 weight rows), against
    the oracle, and bit for bit the same kernel's float32 output rounded to nearest even"""
    rng = np.random.default_rng([t, 381, 200])
    m, n, k = 381, 200, R.TYPES[t][1] * (24 if t in (R.Q4_0, R.Q8_0) else 3)
    raw = G.RAW[t](rng, n, k)
    xb = G.acts(rng, m, k)
    planes = KQ.repack_host(t, raw, (n, k)).to(cuda)
    x = _bf16_tensor(xb, cuda)
    forced_plan(LIB.KERNEL_TILES, 256, 192, 1)
    assert LIB.gemm_plan(t, m, n, k)[:4] == (LIB.KERNEL_TILES, 256, 192, 1)
    print(f"case: {NAME[t]} {m} x {n} x {k}, tile 256 x 192, bf16 and f32 outputs", flush=True)
    y = KQ.matmul(x, planes).cpu().numpy()
    yb = KQ.matmul(x, planes, out_dtype=torch.bfloat16)
    ref = R.bf16_to_f32(xb).astype(np.float64) @ R.dequant(raw, t, k).astype(np.float64).T
    assert_product(y, ref, f"{NAME[t]} tile 256x192 f32")
    assert np.array_equal(yb.view(torch.int16).cpu().numpy().view(np.uint16), R.bf16_round(y))


def _direct_case(t, m, n, k, rng, cuda):
    xb = G.acts(rng, m, k)
    x = _bf16_tensor(xb, cuda)
    xf = R.bf16_to_f32(xb).astype(np.float64)
    if t == "int8":
        q, s = G.int8_weights(rng, n, k)
        w = {"q": torch.from_numpy(q).to(cuda), "s": torch.from_numpy(s).to(cuda)}
        return (lambda: _int8_f32(x, w)), (xf @ q.astype(np.float64).T) * s
    raw = G.RAW[t](rng, n, k)
    planes = KQ.repack_host(t, raw, (n, k)).to(cuda)
    return (lambda: KQ.matmul(x, planes).cpu().numpy()), xf @ R.dequant(raw, t, k).astype(np.float64).T


@pytest.mark.parametrize("t", GEMM_TYPES, ids=GEMM_IDS)
def test_kernel_choice_by_batch_and_forced_auto_shapes(t, forced_plan, cuda):
    """automatic plans: GEMV to 4 rows, weight-stream to 64, LDS tiles beyond; a forced LDS-tile plan with bm = bn = 0
    takes that kernel's own tile choice and gives the right product"""
    n, k = 1000, 1024
    tt = -8 if t == "int8" else t
    assert LIB.gemm_plan(tt, 4, n, k)[0] == LIB.KERNEL_GEMV
    assert LIB.gemm_plan(tt, 64, n, k)[0] == LIB.KERNEL_STREAM
    assert LIB.gemm_plan(tt, 65, n, k)[0] == LIB.KERNEL_TILES
    assert LIB.gemm_plan(tt, 2048, n, k)[0] == LIB.KERNEL_TILES
    m = 300
    run, ref = _direct_case(t, m, n, k, np.random.default_rng(5), cuda)
    for kind in (LIB.KERNEL_TILES,):
        forced_plan(kind, 0, 0, 0)
        kn, bm, bn, _ = LIB.gemm_plan(tt, m, n, k)
        assert kn == kind and bm > 0 and bn > 0
        assert_product(run(), ref, f"{t} kernel {kind} {bm}x{bn}")


@pytest.mark.parametrize("t", GEMM_TYPES, ids=GEMM_IDS)
@pytest.mark.parametrize("m", [5, 17, 40, 64])
@pytest.mark.parametrize("rows", [64, 128])
@pytest.mark.parametrize("kfull", [False, True], ids=["k_ragged", "k_full"])
def test_weight_stream_gemm_every_shape(t, m, rows, kfull, forced_plan, cuda):
    """the weight-stream kernel (4 < M <= 64): 1-4 tiles of 16 activation rows, 64 and 128 weight rows per block,
    ragged weight rows, a K that is or is not a multiple of the kernel's iteration (64 values; 128 for Q4_0 and the
    K-quants, whose K is always whole), K split into 3 ranges (a split with fewer iterations than waves included) against 1"""
    rng = np.random.default_rng([m, rows, int(kfull), 0 if t == "int8" else t])
    n = 3 * rows + 17
    k = {R.Q4_0: (32 * 27, 128 * 7), R.Q8_0: (32 * 27, 64 * 13), R.Q4_K: (256 * 5, 256 * 6), R.Q5_K: (256 * 5, 256 * 6), R.Q6_K: (256 * 5, 256 * 6),
         "int8": (16 * 57, 64 * 15)}[t][int(kfull)]
    xb = G.acts(rng, m, k)
    x = _bf16_tensor(xb, cuda)
    xf = R.bf16_to_f32(xb).astype(np.float64)
    if t == "int8":
        q, s = G.int8_weights(rng, n, k)
        w = {"q": torch.from_numpy(q).to(cuda), "s": torch.from_numpy(s).to(cuda)}
        run = lambda: _int8_f32(x, w)
        ref = (xf @ q.astype(np.float64).T) * s
    else:
        raw = G.RAW[t](rng, n, k)
        planes = KQ.repack_host(t, raw, (n, k)).to(cuda)
        run = lambda: KQ.matmul(x, planes).cpu().numpy()
        ref = xf @ R.dequant(raw, t, k).astype(np.float64).T
    outs = []
    for splits in (1, 3):
        forced_plan(LIB.KERNEL_STREAM, 16, rows, splits)
        kn, bm, bn, sp = LIB.gemm_plan(-8 if t == "int8" else t, m, n, k)
        assert (kn, bm, bn) == (LIB.KERNEL_STREAM, 16, rows) and 1 <= sp <= splits
        y = run()
        assert_product(y, ref, f"{t} m={m} rows {rows} k={k} splits {splits}")
        outs.append(y)
    assert np.max(np.abs(outs[0] - outs[1])) <= 1e-4 * np.max(np.abs(ref))


@pytest.mark.parametrize("t", GEMM_TYPES, ids=GEMM_IDS)
@pytest.mark.parametrize("m,plan", [(64, (1, 16, 64, 4)), (130, (2, 64, 128, 3))], ids=["weight_stream", "lds_tiles"])
def test_split_k_repeats_bit_for_bit(t, m, plan, forced_plan, cuda):
    """a K split into ranges repeats bit for bit over calls (the arrival counters reset themselves), whichever split
    arrives last: both GEMM kernels"""
    rng = np.random.default_rng(77)
    n, k = 1024, 5120
    xb = G.acts(rng, m, k)
    x = _bf16_tensor(xb, cuda)
    tt = -8 if t == "int8" else t
    forced_plan(*plan)
    assert LIB.gemm_plan(tt, m, n, k) == plan
    if t == "int8":
        q, s = G.int8_weights(rng, n, k)
        w = {"q": torch.from_numpy(q).to(cuda), "s": torch.from_numpy(s).to(cuda)}
        run = lambda: _int8_f32(x, w)
        ref = (R.bf16_to_f32(xb).astype(np.float64) @ q.astype(np.float64).T) * s
    else:
        raw = G.RAW[t](rng, n, k)
        planes = KQ.repack_host(t, raw, (n, k)).to(cuda)
        run = lambda: KQ.matmul(x, planes).cpu().numpy()
        ref = R.bf16_to_f32(xb).astype(np.float64) @ R.dequant(raw, t, k).astype(np.float64).T
    first = run()
    assert_product(first, ref)
    for _ in range(4):
        assert np.array_equal(run().view(np.uint32), first.view(np.uint32))


# ----------------------------------------------------------------------------------------------- HIP graph replays
GRAPH_CASES = [  # (type, activation rows, weight rows, K, forced plan or None, stack of layers read at a device index)
    (R.Q4_K, 1, 700, 2048, None, False),                       # decode GEMV
    (R.Q8_0, 3, 700, 1024, None, True),                         # GEMV, device layer of a stack
    ("int8", 64, 1024, 5120, (1, 16, 64, 4), False),           # weight stream, 4 K ranges (arrival counters)
    (R.Q4_0, 130, 640, 2048, (2, 64, 128, 3), False),           # LDS tiles, 3 K ranges
    (R.Q6_K, 300, 512, 1024, None, True),                       # LDS tiles, device layer
]


@pytest.mark.parametrize("case", GRAPH_CASES, ids=lambda c: f"{c[0] if c[0] == 'int8' else NAME[c[0]]}-m{c[1]}")
def test_graph_replays_match_the_eager_result(case, forced_plan, cuda):
    """calls recorded into a HIP graph (torch.cuda.graph) replay bit for bit equal to the eager call, on every replay,
    with eager calls of the same kernels between the replays (the K-split counters reset themselves, and the library
    records no memset node)"""
    t, m, n, k, plan, stacked = case
    rng = np.random.default_rng([m, n, k])
    xb = G.acts(rng, m, k)
    x = _bf16_tensor(xb, cuda)
    x_other = _bf16_tensor(G.acts(rng, m, k), cuda)
    if plan is not None:
        forced_plan(*plan)
    if t == "int8":
        q, s = G.int8_weights(rng, n, k)
        w = {"q": torch.from_numpy(q).to(cuda), "s": torch.from_numpy(s).to(cuda)}
        run = lambda xx: I8.linear(xx, w, pj=lambda v: v)
        ref = (R.bf16_to_f32(xb).astype(np.float64) @ q.astype(np.float64).T) * s
    else:
        layers = 3 if stacked else 1
        st = np.stack([G.RAW[t](rng, n, k) for _ in range(layers)])
        planes = KQ.repack_host(t, st if stacked else st[0], (n, k)).to(cuda)
        li = torch.tensor(layers - 1, dtype=torch.int32, device=cuda)
        run = (lambda xx: KQ.matmul(xx, planes, layer=li)) if stacked else (lambda xx: KQ.matmul(xx, planes))
        ref = R.bf16_to_f32(xb).astype(np.float64) @ R.dequant(st[-1], t, k).astype(np.float64).T
    eager = run(x).float().cpu().numpy()
    assert_product(eager, ref)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        y = run(x)
    for _ in range(3):
        g.replay()
        torch.cuda.synchronize()
        assert np.array_equal(y.float().cpu().numpy().view(np.uint32), eager.view(np.uint32))
        run(x_other)                                              # eager work between the replays
        torch.cuda.synchronize()
    del g
