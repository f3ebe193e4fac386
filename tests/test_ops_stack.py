"""Weights that multiply one input, stacked by rows into one weight (mashbox_amd.ops.stack_rows): a layer's q, k and v,
or its gate and up, as the reference keeps its linear-attention layers' q, k and v (one weight w["qkv"], reference
src/mashbox/models/qwen3_8_27b/model.py:374, split after the product). One kernel launch then serves the group.

Oracle: oracle.ref's dequantization of each part's blocks and the float64 product of each part alone (tests/_check.py
bars); the stacked blocks are the parts' rows in order, byte for byte."""
import numpy as np
import pytest
import torch

from oracle import gen as G
from oracle import ref as R
from tests._check import assert_product, diff_bits

from mashbox_amd import ops

PARTS = [("q", 384), ("k", 64), ("v", 64)]


@pytest.fixture(autouse=True)
def _reset():
    yield
    ops.load_kernels(module="off")


def _parts(t, k, seed, rows=PARTS):
    rng = np.random.default_rng(seed)
    return rng, [(G.RAW[t](rng, n, k), t) for _, n in rows]


# ---------------------------------------------------------------------------------------------------- CPU: bytes
@pytest.mark.parametrize("t", [R.Q4_K, R.Q6_K, R.Q8_0, R.Q4_0, R.Q5_K])
def test_stack_rows_bytes(t):
    """the stacked blocks are the parts' rows in order (NumPy and torch parts alike), and their dequantization is the
    parts' dequantizations stacked: a row's blocks never depend on the rows beside it"""
    k = 512
    _, parts = _parts(t, k, [t, 140])
    raw, tt, sizes = ops.stack_rows(parts)
    assert tt == t and sizes == [n for _, n in PARTS]
    assert isinstance(raw, np.ndarray) and np.array_equal(raw, np.concatenate([r for r, _ in parts]))
    traw, _, _ = ops.stack_rows([(torch.from_numpy(r), t) for r, _ in parts])
    assert isinstance(traw, torch.Tensor) and np.array_equal(traw.numpy(), raw)
    mixed, _, _ = ops.stack_rows([(torch.from_numpy(parts[0][0]), t)] + parts[1:])
    assert np.array_equal(mixed, raw)
    want = np.concatenate([R.dequant(r, t, k) for r, _ in parts])
    assert diff_bits(R.dequant(raw, t, k), want) == 0


def test_stack_rows_refuses():
    rng = np.random.default_rng(141)
    a = G.RAW[R.Q4_K](rng, 16, 512)
    with pytest.raises(ValueError, match="types differ"):
        ops.stack_rows([(a, R.Q4_K), (G.RAW[R.Q6_K](rng, 16, 512), R.Q6_K)])
    with pytest.raises(ValueError, match="row length"):
        ops.stack_rows([(a, R.Q4_K), (G.RAW[R.Q4_K](rng, 16, 768), R.Q4_K)])
    with pytest.raises(ValueError, match="row length"):
        ops.stack_rows([(a[None], R.Q4_K)])
    with pytest.raises(ValueError, match="no parts"):
        ops.stack_rows([])


# ----------------------------------------------------------------------------------------------- GPU: products
@pytest.mark.gpu
@pytest.mark.parametrize("t", [R.Q4_K, R.Q6_K, R.Q8_0])
@pytest.mark.parametrize("m", [1, 4, 16, 64, 300])
def test_stacked_weight_products(t, m, monkeypatch, cuda):
    """prepare() of the stacked blocks (the default 16-row tiles) and one qmatmul per call: each part's output (a view
    of the result) against the float64 product of that part alone, and within the same bars of qmatmul on the part
    alone"""
    monkeypatch.delenv("MBQ_LAYOUT", raising=False)
    ops.load_kernels()
    k = 512
    rng, parts = _parts(t, k, [t, m, 142])
    raw, tt, sizes = ops.stack_rows(parts)
    h = ops.prepare(raw, tt, (sum(sizes), k))
    assert isinstance(h, ops.Packed)
    xb = G.acts(rng, m, k)
    x = torch.from_numpy(xb.astype(np.int16)).view(torch.bfloat16).to(cuda)
    xf = R.bf16_to_f32(xb).astype(np.float64)
    y = ops.qmatmul(x, h)
    assert y.dtype == torch.bfloat16 and tuple(y.shape) == (m, sum(sizes))
    outs = torch.split(y, sizes, -1)
    for (name, n), (r, _), o in zip(PARTS, parts, outs):
        assert tuple(o.shape) == (m, n) and o.data_ptr() >= y.data_ptr()
        ref = xf @ R.dequant(r, t, k).astype(np.float64).T
        assert_product(o.float().cpu().numpy(), ref, f"{name} of the stack m={m}")
        alone = ops.qmatmul(x, ops.prepare(r, t, (n, k)))
        assert_product(alone.float().cpu().numpy(), ref, f"{name} alone m={m}")


@pytest.mark.gpu
@pytest.mark.parametrize("m", [1, 4, 64])
def test_stacked_int8_linear(m, cuda):
    """the int8 linear's {q, s} stacked by rows (q and s concatenated) and repacked once: each part's output against
    the float64 product of that part alone"""
    from mashbox_amd import int8 as I8
    rng = np.random.default_rng([m, 143])
    k = 512
    ws = [G.int8_weights(rng, n, k) for _, n in PARTS]
    q = torch.from_numpy(np.concatenate([a for a, _ in ws])).to(cuda)
    s = torch.from_numpy(np.concatenate([b for _, b in ws])).to(cuda)
    xb = G.acts(rng, m, k)
    x = torch.from_numpy(xb.astype(np.int16)).view(torch.bfloat16).to(cuda)
    xf = R.bf16_to_f32(xb).astype(np.float64)
    for w in ({"q": q, "s": s}, I8.repack(q, s)):
        outs = torch.split(I8.linear(x, w), [n for _, n in PARTS], -1)
        for (name, n), (a, b), o in zip(PARTS, ws, outs):
            ref = (xf @ a.astype(np.float64).T) * b.astype(np.float64)
            assert_product(o.float().cpu().numpy(), ref, f"int8 {name} of the stack m={m}")
