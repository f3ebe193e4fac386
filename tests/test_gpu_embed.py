"""GPU: the int8 embedding rows (mbq_int8_embed through mashbox_amd.int8.embed) and int8 weights loaded from .bshj
files, against the oracle.

Bars: embed is bit for bit the reference's gather f32(q[toks]) * s[toks] rounded to bfloat16, with and without a pj
function (reference tests/cpu/qwen3_8_27b_embed_checks.py E1: every row residue mod 32, the last rows, shapes from one
row to a prefill-sized lookup); int8 weights loaded from a file equal its bytes, and the linear on them meets the product
bars (reference tests/cpu/qwen3_8_27b_checks.py T6 loads such a file)."""
import numpy as np
import pytest
import torch

from mashbox_amd import bshj
from mashbox_amd import int8 as I8
from oracle import gen as G
from oracle import ref as R
from tests import _bshj_write as BW
from tests._check import assert_product

pytestmark = pytest.mark.gpu


def _bits(y: torch.Tensor) -> np.ndarray:
    return y.view(torch.int16).cpu().numpy().view(np.uint16)


def _table(rng, n, d):
    return (rng.integers(-128, 128, (n, d), dtype=np.int8), rng.uniform(1e-4, 3e-2, n).astype(np.float32))


CASES = ([[[r]] for r in range(32)] + [[[4095]], [[4064]], [[31 + 32 * 7]]]
         + [(2, 1), (4, 1), (8, 1), (1, 4), (1, 8), (2, 4), (3, 5), (1, 40), (8, 64)])


@pytest.mark.parametrize("d", [192, 5120, 100], ids=["d192", "d5120", "d100_scalar"])
def test_embed_rows_bit_exact(d, cuda):
    rng = np.random.default_rng(d)
    n = 4096
    q, s = _table(rng, n, d)
    E = {"q": torch.from_numpy(q).to(cuda), "s": torch.from_numpy(s).to(cuda)}
    pj = lambda x: x * 1.5 + 0.25
    for c in CASES + [np.arange(n).reshape(1, n)]:
        toks = np.asarray(c) if not isinstance(c, tuple) else rng.integers(0, n, c)
        t = torch.from_numpy(toks.astype(np.int64)).to(cuda)
        want = R.int8_embed(q, s, toks)
        got = I8.embed(E, t)
        assert got.dtype == torch.bfloat16 and tuple(got.shape) == toks.shape + (d,)
        assert np.array_equal(_bits(got), R.bf16_round(want)), toks.shape
        gp = I8.embed(E, t, pj=pj)
        wp = (torch.from_numpy(want) * 1.5 + 0.25).to(torch.bfloat16)
        assert np.array_equal(_bits(gp), _bits(wp)), toks.shape


def test_embed_index_rule_and_empty_lookups(cuda):
    """negative ids count from the end, ids past either end are clamped (jax.numpy gather); an empty lookup gives an
    empty result; a plain bfloat16 table takes the same index rule"""
    rng = np.random.default_rng(3)
    n, d = 300, 64
    q, s = _table(rng, n, d)
    E = {"q": torch.from_numpy(q).to(cuda), "s": torch.from_numpy(s).to(cuda)}
    toks = np.array([-1, -n, -n - 1, n, n + 1000, 2 ** 31 - 1, -(2 ** 31), 5])
    got = I8.embed(E, torch.from_numpy(toks).to(cuda, torch.int32))
    assert np.array_equal(_bits(got), R.bf16_round(R.int8_embed(q, s, toks)))
    assert tuple(I8.embed(E, torch.zeros((2, 0), dtype=torch.int32, device=cuda)).shape) == (2, 0, d)
    plain = torch.from_numpy(R.bf16_round(rng.standard_normal((n, d)).astype(np.float32)).astype(np.int16)).view(torch.bfloat16).to(cuda)
    t = torch.from_numpy(toks).to(cuda)
    idx = np.clip(np.where(toks < 0, toks + n, toks), 0, n - 1)
    assert torch.equal(I8.embed(plain, t), plain[torch.from_numpy(idx).to(cuda)])


def test_int8_weights_from_a_bshj_file(tmp_path, cuda):
    """one int8 weight and a 3-layer stack loaded from a file: bytes equal, the linear meets the product bars, and the
    stacked layers run in place (weight l = {"q": q[l], "s": s[l]})"""
    rng = np.random.default_rng(4)
    k, n, L = 256, 96, 3
    T = {}
    for l in range(L):
        q, s = G.int8_weights(rng, n, k)
        T[f"model.layers.{l}.mlp.down_proj.weight"] = q
        T[f"model.layers.{l}.mlp.down_proj.weight_scale"] = s
    p = str(tmp_path / "tiny-int8.bshj")
    BW.write(p, T, {"bshj": {"quant": {"type": "TEST"}}})
    xb = G.acts(rng, 5, k)
    x = torch.from_numpy(xb.astype(np.int16)).view(torch.bfloat16).to(cuda)
    xf = R.bf16_to_f32(xb).astype(np.float64)
    with bshj.File(p) as f:
        P = bshj.prefix(f.tensors)
        assert P == "model."
        names = [f"{P}layers.{l}.mlp.down_proj.weight" for l in range(L)]
        one = bshj.int8_weight(f, names[1], device=cuda)
        st = bshj.int8_stack(f, names, device=cuda)
    assert torch.equal(one["q"].cpu(), torch.from_numpy(T[names[1]]))
    assert torch.equal(st["q"].cpu(), torch.from_numpy(np.stack([T[nm] for nm in names])))
    for l in range(L):
        q, s = T[names[l]], T[names[l] + "_scale"]
        ref = (xf @ q.astype(np.float64).T) * s
        y = I8.linear(x, {"q": st["q"][l], "s": st["s"][l]}, pj=lambda v: v).float().cpu().numpy()
        assert_product(y, ref, f"layer {l}")
    assert torch.equal(I8.linear(x, one), I8.linear(x, {"q": st["q"][1], "s": st["s"][1]}))
