"""Comparison bars shared by the tests.

- bit equality with NaN == NaN: reference tests/cpu/test_gguf_dequant.py:30-36 (and tests/contracts/test_ops.py:129-134)
- NMSE = sum (y - ref)^2 / sum ref^2 <= 2e-5 for bfloat16 activations: reference tests/contracts/test_ops.py:28-31,51
- max |y - ref| / max |ref| <= 1e-2 (bf16 out, fp32 accumulate): the bar BASELINE.json's north star sets
- a reference that is exactly zero gives exactly zero; every output is finite: tests/contracts/test_ops.py:32,143-147
"""
import numpy as np

NMSE_BF16 = 2e-5
MAX_REL = 1e-2


def diff_bits(got, want) -> int:
    """number of float32 values whose bits differ; NaN must be NaN on both sides"""
    a = np.ascontiguousarray(np.asarray(got, np.float32))
    b = np.ascontiguousarray(np.asarray(want, np.float32))
    assert a.shape == b.shape, (a.shape, b.shape)
    nan = np.isnan(a) | np.isnan(b)
    same = np.where(nan, np.isnan(a) & np.isnan(b), a.view(np.uint32) == b.view(np.uint32))
    return int(np.sum(~same))


def product_errors(y, ref):
    """-> (nmse, max_rel) of y against a float64 reference product"""
    y = np.asarray(y, np.float64)
    ref = np.asarray(ref, np.float64)
    assert y.shape == ref.shape, (y.shape, ref.shape)
    assert np.all(np.isfinite(y)), "non-finite output"
    den = float(np.sum(ref ** 2))
    if den == 0.0:
        assert np.all(y == 0.0), "reference is exactly zero, output is not"
        return 0.0, 0.0
    nmse = float(np.sum((y - ref) ** 2)) / den
    max_rel = float(np.max(np.abs(y - ref)) / np.max(np.abs(ref)))
    return nmse, max_rel


def assert_product(y, ref, what=""):
    nmse, mr = product_errors(y, ref)
    assert nmse <= NMSE_BF16 and mr <= MAX_REL, f"{what}: NMSE {nmse:.3e} (bar {NMSE_BF16}), max rel {mr:.3e} (bar {MAX_REL})"
    return nmse, mr


def assert_product_dev(y, ref, what=""):
    """assert_product on GPU tensors (torch, any float dtype; ref float64): every output finite, NMSE and max-rel
    computed in float64 on the device, so full-size outputs are compared whole without a host copy"""
    import torch
    y = y.to(torch.float64)
    ref = ref.to(torch.float64)
    assert tuple(y.shape) == tuple(ref.shape), (tuple(y.shape), tuple(ref.shape))
    assert bool(torch.isfinite(y).all()), f"{what}: non-finite output"
    den = float((ref * ref).sum())
    if den == 0.0:
        assert bool((y == 0).all()), f"{what}: reference is exactly zero, output is not"
        return 0.0, 0.0
    nmse = float(((y - ref) ** 2).sum()) / den
    mr = float((y - ref).abs().max() / ref.abs().max())
    assert nmse <= NMSE_BF16 and mr <= MAX_REL, (f"{what}: NMSE {nmse:.3e} (bar {NMSE_BF16}), max rel {mr:.3e} "
                                                 f"(bar {MAX_REL}); {_where_off(y, ref)}")
    return nmse, mr


def _where_off(y, ref):
    """where a 2-D product misses its bar: the outputs off by more than 1e-2 of max |ref|, their row and column ranges,
    and the 256 x 192 tiles (the specialized GEMM's) and 16-row blocks they fall in"""
    import torch
    if y.dim() != 2:
        y, ref = y.reshape(-1, y.shape[-1]), ref.reshape(-1, ref.shape[-1])
    bad = (y - ref).abs() > MAX_REL * ref.abs().max()
    idx = torch.nonzero(bad).cpu()
    if len(idx) == 0:
        return "no single output past 1e-2 of max |ref| (the NMSE bar failed on many small errors)"
    r, c = idx[:, 0], idx[:, 1]
    tiles = sorted({(int(a) // 256, int(b) // 192) for a, b in idx[:: max(1, len(idx) // 4096)].tolist()})
    return (f"{len(idx)} outputs past 1e-2 of max |ref| in rows {int(r.min())}-{int(r.max())} ({len(torch.unique(r))} "
            f"distinct), columns {int(c.min())}-{int(c.max())} ({len(torch.unique(c))} distinct), 256x192 tiles "
            f"{tiles[:24]}")
