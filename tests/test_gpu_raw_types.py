"""The exact path's other ggml types on the GPU: F32, F16, BF16, Q4_1, Q5_0, Q5_1, Q2_K, Q3_K, IQ4_NL, IQ4_XS, TQ1_0,
TQ2_0, MXFP4 and NVFP4 have no kernel planes; the reference runs them on its exact path (dequant + float32 product:
src/mashbox/ops/__init__.py:574-576, 624-632, with src/mashbox/ops/reference.py's per-type rebuilds), and so does this
build through mbq_dequant_raw.

Bars, as the kernel types' (tests/test_gpu_parity.py):
  dequant: bit for bit against the oracle (oracle/ref.py, pinned by tests/test_oracle_types.py), NaN where it has NaN,
           on random bytes with all-zero and all-0xFF blocks (reference tests/cpu/test_gguf_dequant.py:17-45) and on
           the real llama-quantize blocks of tests/golden;
  product: ops.qmatmul on the prepared weight within the float32 bars of tests/_check.py against the float64 product
           of the oracle's weights.
"""
import numpy as np
import pytest
import torch

from oracle import ref as R
from tests._check import assert_product_dev, diff_bits
from tests.test_oracle import GOLDEN

import mashbox_amd.ops as OPS

NAME = {t: R.TYPES[t][0] for t in R.TYPES}
FLOATS = (R.F32, R.F16, R.BF16)


def _cols(t, kb):
    bs = R.TYPES[t][1]
    return bs * kb if bs > 1 else 37 * kb


def _raw(t, rows, kb, seed):
    rng = np.random.default_rng(seed)
    cols = _cols(t, kb)
    raw = rng.integers(0, 256, size=(rows, R.row_bytes(t, cols)), dtype=np.uint8)
    raw[0], raw[1] = 0, 0xFF
    return raw, cols


@pytest.mark.gpu
@pytest.mark.parametrize("t", R.EXACT_ONLY, ids=NAME.get)
@pytest.mark.parametrize("kb", [1, 2, 16])
def test_raw_dequant_bit_exact(t, kb, cuda):
    raw, cols = _raw(t, 6, kb, 5000 + 10 * t + kb)
    got = OPS._raw_dequant(torch.from_numpy(raw).to(cuda), t, 6, cols).cpu().numpy()
    assert diff_bits(got, R.dequant(raw, t, cols)) == 0


@pytest.mark.gpu
@pytest.mark.parametrize("t", FLOATS, ids=NAME.get)
@pytest.mark.parametrize("rows,cols", [(1, 1), (3, 37), (5, 1001), (2, 4)])
def test_float_types_any_row_length(t, rows, cols, cuda):
    """one value per block: rows x cols not a multiple of the kernel's 4-value step"""
    rng = np.random.default_rng(rows * cols + t)
    raw = rng.integers(0, 256, size=(rows, R.row_bytes(t, cols)), dtype=np.uint8)
    got = OPS._raw_dequant(torch.from_numpy(raw).to(cuda), t, rows, cols).cpu().numpy()
    assert diff_bits(got, R.dequant(raw, t, cols)) == 0


@pytest.mark.gpu
def test_mxfp4_and_nvfp4_every_scale(cuda):
    """every E8M0 exponent (subnormal results, overflow to inf) and every E4M3 scale byte, each with all 16 codes"""
    codes = np.array([0x10, 0x32, 0x54, 0x76, 0x98, 0xBA, 0xDC, 0xFE], np.uint8)
    mx = np.zeros((256, 17), np.uint8)
    mx[:, 0] = np.arange(256)
    mx[:, 1:9] = codes
    nv = np.zeros((64, 36), np.uint8)
    nv[:, :4] = np.arange(256, dtype=np.uint8).reshape(64, 4)
    nv[:, 4:] = np.tile(codes, 4)
    for t, raw, cols in ((R.MXFP4, mx, 32), (R.NVFP4, nv, 64)):
        got = OPS._raw_dequant(torch.from_numpy(raw).to(cuda), t, raw.shape[0], cols).cpu().numpy()
        assert diff_bits(got, R.dequant(raw, t, cols)) == 0, NAME[t]


def _golden_exact():
    import os
    out = []
    if os.path.isdir(GOLDEN):
        for f in sorted(os.listdir(GOLDEN)):
            if f.endswith(".npz"):
                z = np.load(os.path.join(GOLDEN, f), allow_pickle=False)
                if int(z["t"]) in R.EXACT_ONLY:
                    out.append(f)
    return out


@pytest.mark.gpu
@pytest.mark.parametrize("name", _golden_exact())
def test_golden_blocks_dequant_and_product(name, cuda):
    """the committed fixtures of the exact path's types: dequant bit for bit; for the real llama-quantize slices also
    ops.prepare -> Raw -> ops.qmatmul against the float64 product the fixture holds"""
    import os
    z = np.load(os.path.join(GOLDEN, name), allow_pickle=False)
    t, cols, raw = int(z["t"]), int(z["cols"]), z["raw"]
    rows = raw.shape[0]
    got = OPS._raw_dequant(torch.from_numpy(raw).to(cuda), t, rows, cols).cpu().numpy()
    assert diff_bits(got, z["w"]) == 0
    if "x" in z.files:
        h = OPS.prepare(raw, t, (rows, cols))
        assert isinstance(h, OPS.Raw) and OPS.weight_path(t, (rows, cols)) == "exact"
        x = torch.from_numpy(z["x"].astype(np.int16)).view(torch.bfloat16).to(cuda)
        y = OPS.qmatmul(x, h)
        assert y.dtype == torch.bfloat16 and tuple(y.shape) == (x.shape[0], rows)
        assert_product_dev(y.float(), torch.from_numpy(z["y64"]).to(cuda), name)


@pytest.mark.gpu
@pytest.mark.parametrize("t", R.EXACT_ONLY, ids=NAME.get)
def test_qmatmul_exact_path(t, cuda):
    """a (rows, cols) weight of every exact-only type through ops.prepare / ops.qmatmul, leading activation axes kept,
    against the float64 product of the oracle's weights; finite scales so that the product is finite"""
    from tests.test_oracle_types import random_blocks
    bs, ts = R.TYPES[t][1], R.TYPES[t][2]
    rows = 45
    if t in FLOATS:
        cols = 300
        rng = np.random.default_rng(t)
        w = (rng.standard_normal((rows, cols)) * 0.05).astype(np.float32)
        raw = (w.view(np.uint8) if t == R.F32 else
               w.astype(np.float16).view(np.uint8) if t == R.F16 else
               (R.bf16_round(w)).view(np.uint8)).reshape(rows, -1)
    else:
        kb = max(1, 512 // bs)
        cols = bs * kb
        blocks = random_blocks(t, rows * kb, 6000 + t)
        if t == R.MXFP4:
            blocks[:, 0] = np.random.default_rng(t).integers(110, 130, blocks.shape[0])      # exponents of weights
        raw = blocks.reshape(rows, kb * ts)
    h = OPS.prepare(raw, t, (rows, cols))
    assert isinstance(h, OPS.Raw)
    w64 = torch.from_numpy(R.dequant(raw, t, cols)).to(cuda).double()
    rng = np.random.default_rng(7 + t)
    x = torch.from_numpy(rng.standard_normal((2, 3, cols)).astype(np.float32)).to(cuda).to(torch.bfloat16)
    y = OPS.qmatmul(x, h)
    assert tuple(y.shape) == (2, 3, rows) and y.dtype == torch.bfloat16
    assert_product_dev(y.float(), x.double() @ w64.T, NAME[t])


@pytest.mark.gpu
@pytest.mark.parametrize("t", [R.Q3_K, R.IQ4_XS, R.BF16, R.NVFP4], ids=NAME.get)
def test_take_rows_exact_path(t, cuda):
    """an embedding lookup on a Raw weight rebuilds only the looked-up rows, bit for bit the rows of the whole
    dequantization (negative ids count from the end); no ids give an empty result"""
    raw, cols = _raw(t, 20, 2, 7000 + t)
    h = OPS.prepare(raw, t, (20, cols))
    want = R.dequant(raw, t, cols)
    ids = torch.tensor([[3, -1], [0, 19]], device=cuda)
    got = OPS.take_rows(h, ids).cpu().numpy()
    assert diff_bits(got, want[[[3, 19], [0, 19]]]) == 0
    assert tuple(OPS.take_rows(h, torch.zeros(0, dtype=torch.long, device=cuda)).shape) == (0, cols)


def test_prepare_refuses_code_book_types():
    """the seven types whose values come from gguf-py's code books are refused at load, with the reason"""
    for t in OPS.CODEBOOK_TYPES:
        with pytest.raises(NotImplementedError, match="code books"):
            OPS.prepare(np.zeros((1, 66), np.uint8), t, (1, 256))
    assert set(OPS.TYPES) == set(R.TYPES)
    for t in R.EXACT_ONLY:
        assert OPS.row_bytes(t, _cols(t, 3)) == R.row_bytes(t, _cols(t, 3))


@pytest.mark.gpu
def test_mixed_role_of_a_kernel_type_and_an_exact_type(cuda):
    """a role whose layers mix a kernel type and an exact-only type (as Q3_K_M files mix Q3_K and Q4_K per layer,
    reference src/mashbox/ops/__init__.py:216-270): stack_mixed, scan_split / scan_join and qmatmul give each layer's
    product, the Q3_K stack dequantizes with its leading axis, against the oracle"""
    from oracle import gen as G
    from tests.test_oracle_types import random_blocks
    rows, cols = 48, 512
    layers = []
    for l, t in enumerate([R.Q4_K, R.Q3_K, R.Q4_K, R.Q3_K]):
        raw = (G.RAW[t](np.random.default_rng(l), rows, cols) if t == R.Q4_K else
               random_blocks(t, rows * (cols // 256), 900 + l).reshape(rows, -1))
        layers.append((raw, t))
    OPS.load_kernels()
    try:
        h = OPS.stack_mixed(layers, (rows, cols))
        assert isinstance(h, OPS.Mixed) and tuple(h.types) == (R.Q4_K, R.Q3_K)
        assert isinstance(h.stacks[1], OPS.Raw)
        st = OPS.dequant(h.stacks[1]).cpu().numpy()
        assert st.shape == (2, rows, cols)
        for s, l in enumerate((1, 3)):
            assert diff_bits(st[s], R.dequant(layers[l][0], R.Q3_K, cols)) == 0
        held, xs = OPS.scan_split({"w": h})
        rng = np.random.default_rng(11)
        x = torch.from_numpy(rng.standard_normal((3, cols)).astype(np.float32)).to(cuda).to(torch.bfloat16)
        for l, (raw, t) in enumerate(layers):
            w = OPS.scan_join(held, xs, torch.tensor(l, dtype=torch.int32, device=cuda))["w"]
            y = OPS.qmatmul(x, w)
            ref = x.double() @ torch.from_numpy(R.dequant(raw, t, cols)).to(cuda).double().T
            assert_product_dev(y.float(), ref, f"layer {l} {NAME[t]}")
    finally:
        OPS.load_kernels(module="off")


# ---------------------------------------------------------------------------------------- fused raw GEMV (1-8 rows)
def _weights(t, n, k, seed):
    """(n, k) weights of type t as file blocks with finite values: random blocks with finite fp16 scales (MXFP4: the
    exponents of weights), or normal values for the float types"""
    from tests.test_oracle_types import random_blocks
    bs, ts = R.TYPES[t][1], R.TYPES[t][2]
    if t in FLOATS:
        w = (np.random.default_rng(seed).standard_normal((n, k)) * 0.05).astype(np.float32)
        return (w.view(np.uint8) if t == R.F32 else w.astype(np.float16).view(np.uint8) if t == R.F16 else
                R.bf16_round(w).view(np.uint8)).reshape(n, -1)
    blocks = random_blocks(t, n * (k // bs), seed)
    if t == R.MXFP4:
        blocks[:, 0] = np.random.default_rng(seed).integers(110, 130, blocks.shape[0])
    return blocks.reshape(n, (k // bs) * ts)


def _matmul_raw(t, raw_dev, x, n, k, out_bf16):
    import ctypes
    from mashbox_amd import _lib as LIB
    m = x.shape[0]
    y = torch.empty((m, n), dtype=torch.bfloat16 if out_bf16 else torch.float32, device=x.device)
    LIB.check(LIB.lib().mbq_matmul_raw(t, ctypes.c_void_p(raw_dev.data_ptr()), ctypes.c_void_p(x.data_ptr()), m, n, k,
                                       ctypes.c_void_p(y.data_ptr()), 1 if out_bf16 else 0,
                                       ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)), "matmul_raw")
    return y


@pytest.mark.gpu
@pytest.mark.parametrize("t", R.EXACT_ONLY, ids=NAME.get)
@pytest.mark.parametrize("m,n,k", [(1, 77, 256), (3, 200, 4096), (8, 33, 512), (5, 130, 2304), (2, 65, 8448)])
def test_matmul_raw_against_the_exact_product(t, m, n, k, cuda):
    """mbq_matmul_raw against the float64 product of the oracle's weights (16, 32 and 64 lanes per row, two units in
    flight at K = 8448, rows past a block and partial lane rounds); its bfloat16 output is its float32 output rounded to
    nearest even, bit for bit; a second call repeats the bits"""
    raw = _weights(t, n, k, 8000 + 7 * t + m)
    raw_dev = torch.from_numpy(raw).to(cuda)
    rng = np.random.default_rng(m * n + k)
    x = torch.from_numpy(rng.standard_normal((m, k)).astype(np.float32)).to(cuda).to(torch.bfloat16)
    y32 = _matmul_raw(t, raw_dev, x, n, k, False)
    ref = x.double() @ torch.from_numpy(R.dequant(raw, t, k)).to(cuda).double().T
    assert_product_dev(y32, ref, f"{NAME[t]} m={m} {n}x{k}")
    yb = _matmul_raw(t, raw_dev, x, n, k, True)
    assert np.array_equal(yb.view(torch.int16).cpu().numpy().view(np.uint16), R.bf16_round(y32.cpu().numpy()))
    assert torch.equal(_matmul_raw(t, raw_dev, x, n, k, False).view(torch.int32), y32.view(torch.int32))


@pytest.mark.gpu
@pytest.mark.parametrize("t", [R.Q2_K, R.IQ4_XS, R.F16], ids=NAME.get)
def test_qmatmul_routes_decode_rows_to_the_fused_product(t, cuda):
    """ops.qmatmul on a Raw weight: a bfloat16 x of 1-8 rows takes mbq_matmul_raw (the same bits as a direct call),
    9 rows and float32 x the rebuild and a GEMM; all within the bars"""
    n, k = 96, 1024
    raw = _weights(t, n, k, 9100 + t)
    h = OPS.prepare(raw, t, (n, k))
    w64 = torch.from_numpy(R.dequant(raw, t, k)).to(cuda).double()
    rng = np.random.default_rng(t)
    for m in (1, 8, 9):
        x = torch.from_numpy(rng.standard_normal((m, k)).astype(np.float32)).to(cuda).to(torch.bfloat16)
        y = OPS.qmatmul(x, h)
        assert_product_dev(y.float(), x.double() @ w64.T, f"{NAME[t]} m={m}")
        if m <= OPS.RAW_GEMV_MAX_M:
            direct = _matmul_raw(t, h.raw.reshape(n, -1).contiguous(), x, n, k, True)
            assert torch.equal(y.view(torch.int16), direct.view(torch.int16))
    x32 = torch.from_numpy(rng.standard_normal((2, k)).astype(np.float32)).to(cuda)
    y32 = OPS.qmatmul(x32, h)
    assert y32.dtype == torch.float32
    assert_product_dev(y32, x32.double() @ w64.T, f"{NAME[t]} float32 x")


def test_matmul_raw_argument_checks():
    """refused before any launch: the kernel types (they have planes), more than 8 rows, K not a multiple of 32 or of
    the block, a non-ggml type; M = 0 launches nothing"""
    from mashbox_amd import _lib as LIB
    lib = LIB.lib()
    assert lib.mbq_matmul_raw(R.Q4_K, None, None, 1, 8, 256, None, 0, None) < 0
    assert lib.mbq_matmul_raw(R.Q2_K, None, None, 9, 8, 256, None, 0, None) < 0
    assert lib.mbq_matmul_raw(R.F16, None, None, 1, 8, 48, None, 0, None) < 0
    assert lib.mbq_matmul_raw(R.NVFP4, None, None, 1, 8, 96, None, 0, None) < 0
    assert lib.mbq_matmul_raw(16, None, None, 1, 8, 256, None, 0, None) < 0
    assert lib.mbq_matmul_raw(R.Q2_K, None, None, 1, 8, 256, None, 5, None) < 0
    assert lib.mbq_matmul_raw(R.Q2_K, None, None, 0, 8, 256, None, 0, None) == 0
