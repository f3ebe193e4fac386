"""The ops boundary (mashbox_amd.ops) around the kernel package: routing, the preflight, the fallback to the exact path,
layer stacks read in place, the contract check. Counterparts of the reference's boundary tests
(reference tests/cpu/test_gguf_qwen35.py:183-374 stubs and forced failures, :639-806 layer=;
tests/contracts/test_ops.py:19-35 bars), with stub packages that wrap mashbox_amd.kernels and fail on purpose (host-side
exceptions only: no kernel faults)."""
import sys
import types

import numpy as np
import pytest

from oracle import gen as G
from oracle import ref as R
from tests._check import assert_product, diff_bits

import mashbox_amd.kernels as KQ
from mashbox_amd import ops


@pytest.fixture(autouse=True)
def _reset():
    yield
    ops.load_kernels(module="off")


# ------------------------------------------------------------------------------------------------ CPU: routing
def test_weight_path_and_device_bytes(monkeypatch):
    monkeypatch.delenv("MBQ_LAYOUT", raising=False)
    assert ops.load_kernels() == frozenset({2, 8, 12, 13, 14})
    assert ops.weight_path(12, (5120, 17408)) == "kq" and ops.weight_path(8, (17408, 5120)) == "kq"
    assert ops.weight_path(14, (256, 256)) == "kq"
    assert ops.weight_path(14, (256, 256), kernel_types=frozenset({8, 12})) == "exact"   # Q6_K left to the exact path
    assert ops.weight_path(12, (5, 100)) == "exact"                      # kq_covers: not whole super-blocks
    assert ops.weight_path(12, (256, 256), kernel_types=frozenset()) == "exact"
    nb = 5120 * R.row_bytes(12, 17408)
    # the default layout is the kernel package's 16-row tiles; MBQ_LAYOUT picks row-major planes or both
    tiles, rm = KQ.plane_bytes(KQ.TILED[12], (5120, 17408)), KQ.plane_bytes(12, (5120, 17408))
    assert ops.device_nbytes(12, (5120, 17408), nb) == tiles
    assert ops.device_nbytes(12, (3, 5120, 17408), 3 * nb) == 3 * tiles
    assert ops.device_nbytes(14, (256, 256), 12345, kernel_types=frozenset({8, 12})) == 12345
    assert ops.device_nbytes(14, (256, 256), 12345) == KQ.plane_bytes(KQ.TILED[14], (256, 256))
    monkeypatch.setenv("MBQ_LAYOUT", "rowmajor")
    assert ops.device_nbytes(12, (3, 5120, 17408), 3 * nb) == 3 * rm
    monkeypatch.setenv("MBQ_LAYOUT", "both")
    assert ops.device_nbytes(12, (3, 5120, 17408), 3 * nb) == 3 * (rm + tiles)
    monkeypatch.setenv("MBQ_LAYOUT", "diagonal")
    with pytest.raises(ValueError):
        ops.device_nbytes(12, (5120, 17408), nb)
    monkeypatch.delenv("MBQ_LAYOUT")
    ops.load_kernels(module="off")
    assert ops.weight_path(12, (256, 256)) == "exact"


def test_kernel_package_that_fails_to_load_leaves_every_type_exact(monkeypatch):
    msgs = []
    monkeypatch.setenv("MASHBOX_FAULT", "force:kernels-package")
    assert ops.load_kernels(log=msgs.append) == frozenset()
    assert msgs and "did not load" in msgs[0]
    monkeypatch.delenv("MASHBOX_FAULT")
    assert ops.load_kernels(module="no_such_kernel_module") == frozenset()
    assert "No module" in ops._KERNELS["error"]


def test_exact_chunk_rows_matches_the_oracle():
    for rows, cols in [(17408, 5120), (5120, 17408), (4096, 4096), (97, 3), (360, 64)]:
        for limit in (None, 64, 4096):
            assert ops.exact_chunk_rows(rows, cols, limit) == R.exact_chunk_rows(rows, cols, limit)


# ---------------------------------------------------------------------------------------------- GPU: the paths
def _x(rng, m, k, cuda):
    import torch
    xb = G.acts(rng, m, k)
    return xb, torch.from_numpy(xb.astype(np.int16)).view(torch.bfloat16).to(cuda)


@pytest.mark.gpu
@pytest.mark.parametrize("t", [R.Q4_0, R.Q8_0, R.Q4_K, R.Q5_K, R.Q6_K])
def test_kernel_and_exact_paths_match_the_oracle(t, cuda):
    import torch
    ops.load_kernels()
    rng = np.random.default_rng(500 + t)
    n, k = 96, R.TYPES[t][1] * 4
    raw = G.RAW[t](rng, n, k)
    hk, he = ops.prepare(raw, t, (n, k)), ops.prepare(raw, t, (n, k), use_kernel=False)
    assert isinstance(hk, ops.Packed) and isinstance(he, ops.Raw) and ops.route(hk) == "kernel"
    w = R.dequant(raw, t, k)
    assert diff_bits(ops.dequant(hk).cpu().numpy(), w) == 0 and diff_bits(ops.dequant(he).cpu().numpy(), w) == 0
    xb, x = _x(rng, 5, k, cuda)
    ref = R.bf16_to_f32(xb).astype(np.float64) @ w.astype(np.float64).T
    yk, ye = ops.qmatmul(x, hk), ops.qmatmul(x, he)
    assert yk.dtype == torch.bfloat16 and ye.dtype == torch.bfloat16
    assert_product(yk.float().cpu().numpy(), ref, "kq")
    assert_product(ye.float().cpu().numpy(), ref, "exact")
    # float32 activations on the exact path: the reference's float32 bars (tests/contracts/test_ops.py:19-35)
    xf = torch.from_numpy(rng.standard_normal((3, k)).astype(np.float32)).to(cuda)
    y = ops.qmatmul(xf, he).cpu().numpy().astype(np.float64)
    x64 = xf.cpu().numpy().astype(np.float64)
    ref32 = x64 @ w.astype(np.float64).T
    u = 2.0 ** -24
    gamma = k * u / (1 - k * u)
    assert np.all(np.abs(y - ref32) <= gamma * (np.abs(x64) @ np.abs(w.astype(np.float64)).T))
    assert float(np.sum((y - ref32) ** 2) / np.sum(ref32 ** 2)) <= 1e-8
    # the oracle's own exact path agrees
    assert np.allclose(R.qmatmul_exact(x64.astype(np.float32), raw, t, (n, k)), y, rtol=1e-5, atol=1e-5)


@pytest.mark.gpu
@pytest.mark.parametrize("t", [R.Q4_0, R.Q8_0, R.Q4_K, R.Q5_K, R.Q6_K])
def test_qmatmul_writes_bf16_directly(t, cuda):
    """qmatmul of bfloat16 activations returns the kernel's own bfloat16 output (no float32 result and cast): bit for
    bit kernels.matmul(..., out_dtype=bfloat16), which is the float32 result rounded to nearest even; for a handle, a
    layer of a held stack (At), and float32 activations (float32 result, then a cast to float32: the same values)"""
    import torch
    ops.load_kernels()
    rng = np.random.default_rng(900 + t)
    n, k = 200, R.TYPES[t][1] * 8
    st = np.stack([G.RAW[t](rng, n, k) for _ in range(2)])
    h = ops.prepare(st[0], t, (n, k))
    hs = ops.prepare(st, t, (n, k))
    for m in (1, 4, 16, 80):
        _, x = _x(rng, m, k, cuda)
        y = ops.qmatmul(x, h)
        assert y.dtype == torch.bfloat16
        direct = KQ.matmul(x, h.packed, out_dtype=torch.bfloat16)
        f32 = KQ.matmul(x, h.packed)
        assert torch.equal(y.view(torch.int16), direct.view(torch.int16)), f"m={m}: not the kernel's bf16 output"
        assert torch.equal(y.view(torch.int16), f32.to(torch.bfloat16).view(torch.int16)), f"m={m}: not RNE of f32"
        held, xs = ops.scan_split({"w": hs})
        w = ops.scan_join(held, xs, torch.tensor(1, dtype=torch.int32, device=cuda))["w"]
        ya = ops.qmatmul(x, w)
        assert torch.equal(ya.view(torch.int16),
                           KQ.matmul(x, hs.packed, layer=1, out_dtype=torch.bfloat16).view(torch.int16))
    xf = x.float()
    assert torch.equal(ops.qmatmul(xf, h), KQ.matmul(xf, h.packed))


@pytest.mark.gpu
def test_exact_path_chunks_large_weights(cuda, monkeypatch):
    """a weight over EXACT_CHUNK values is rebuilt a chunk of rows at a time: same values as one rebuild"""
    ops.load_kernels(module="off")
    rng = np.random.default_rng(9)
    n, k = 48, 512
    raw = G.q8_0_raw(rng, n, k)
    h = ops.prepare(raw, 8, (n, k))
    xb, x = _x(rng, 2, k, cuda)
    whole = ops.qmatmul(x.float(), h).cpu().numpy()
    monkeypatch.setattr(ops, "EXACT_CHUNK", 8 * k)
    assert ops.exact_chunk_rows(n, k) == 8
    chunked = ops.qmatmul(x.float(), h).cpu().numpy()
    ref = R.bf16_to_f32(xb).astype(np.float64) @ R.dequant(raw, 8, k).astype(np.float64).T
    assert_product(chunked, ref)
    assert np.max(np.abs(chunked - whole)) <= 1e-5 * np.max(np.abs(ref))


def _stub(name, fail, calls):
    """a kernel package that is mashbox_amd.kernels except that `fail` raises: "repack", "repack_host" or "matmul" """
    stub = types.ModuleType(name)
    stub.TYPES = KQ.TYPES
    stub.plane_bytes, stub.dequant, stub.picks_layer = KQ.plane_bytes, KQ.dequant, True

    def boom(what):
        raise RuntimeError(f"forced failure of the kernel's {what}")

    def repack(t, raw, shape, stacked=False):
        calls["repack"] += 1
        if fail == "repack":
            boom("repack")
        return KQ.repack(t, raw, shape, stacked)

    def repack_host(t, raw, shape):
        calls["repack"] += 1
        if fail in ("repack_host", "repack"):
            boom("repack_host")
        return KQ.repack_host(t, raw, shape)

    def matmul(x, planes, layer=None, out_dtype=None):
        calls["matmul"] += 1
        if fail == "matmul":
            boom("matmul")
        return KQ.matmul(x, planes, layer=layer)
    stub.repack, stub.repack_host, stub.matmul = repack, repack_host, matmul
    return stub


@pytest.mark.gpu
@pytest.mark.parametrize("fail", ["repack", "repack_host", "matmul", "force:quant-kernel"])
def test_kq_failure_falls_back_to_the_exact_path(fail, cuda, monkeypatch, capsys):
    """a failing repack or preflight: the weight loads on the exact path, every later weight of that (type, shape) too,
    one warning per (type, shape) names the type and the error, and the product equals the exact path's bit for bit"""
    import torch
    calls = {"repack": 0, "matmul": 0}
    name = "_stub_mbq_fail_" + fail.replace(":", "_").replace("-", "_")
    monkeypatch.setitem(sys.modules, name, _stub(name, fail, calls))
    if fail.startswith("force:"):
        monkeypatch.setenv("MASHBOX_FAULT", fail)
    assert ops.load_kernels(module=name) == frozenset({2, 8, 12, 13, 14})
    rng = np.random.default_rng(31)
    shapes = [(8, (40, 256)), (8, (40, 256)), (12, (24, 512)), (12, (24, 512)), (8, (16, 64))]
    raws = [G.RAW[t](rng, *s) for t, s in shapes]
    capsys.readouterr()
    hs = [ops.prepare(r, t, s) for r, (t, s) in zip(raws, shapes)]
    err = capsys.readouterr().err
    assert all(isinstance(h, ops.Raw) for h in hs), hs
    assert err.count("kq planes for") == 3, err                          # one per (type, shape)
    assert all(v is not True for v in ops._KERNELS.preflight.values()) and len(ops._KERNELS.preflight) == 3
    want = "forced" if fail.startswith("force:") else "forced failure"
    assert want in err and "exact path" in err, err
    ops.load_kernels(module="off")
    for h, r, (t, s) in zip(hs, raws, shapes):
        xb, x = _x(rng, 3, s[1], cuda)
        want = ops.qmatmul(x, ops.prepare(r, t, s))                       # the exact path, no package loaded
        assert np.array_equal(ops.qmatmul(x, h).view(torch.int16).cpu().numpy(), want.view(torch.int16).cpu().numpy())


@pytest.mark.gpu
def test_kq_preflight_runs_once_per_type_and_shape(cuda, monkeypatch):
    calls = {"repack": 0, "matmul": 0}
    monkeypatch.setitem(sys.modules, "_stub_mbq_ok", _stub("_stub_mbq_ok", None, calls))
    assert ops.load_kernels(module="_stub_mbq_ok") == frozenset({2, 8, 12, 13, 14})
    rng = np.random.default_rng(32)
    shapes = [(8, (40, 256))] * 3 + [(12, (24, 512))] * 2
    hs = [ops.prepare(G.RAW[t](rng, *s), t, s) for t, s in shapes]
    assert all(isinstance(h, ops.Packed) for h in hs)
    assert calls["matmul"] == 2 and calls["repack"] == 5, calls
    assert all(v is True for v in ops._KERNELS.preflight.values()) and len(ops._KERNELS.preflight) == 2
    ops.load_kernels(module="_stub_mbq_ok")
    assert ops._KERNELS.preflight == {}, "load_kernels starts the preflight over"


@pytest.mark.gpu
@pytest.mark.parametrize("t", [R.Q4_0, R.Q8_0, R.Q4_K, R.Q5_K, R.Q6_K])
def test_layer_stack_is_read_in_place(t, cuda):
    """a stack of layers loads as one Packed handle; scan_split holds it whole and scan_join hands the loop body
    At(stack, layer); the product equals the sliced layer's and the exact path's"""
    import torch
    ops.load_kernels()
    rng = np.random.default_rng(40 + t)
    L, n, k = 3, 40, R.TYPES[t][1] * 2
    st = np.stack([G.RAW[t](rng, n, k) for _ in range(L)])
    h = ops.prepare(st, t, (n, k))
    assert isinstance(h, ops.Packed) and ops._KERNELS.layer_preflight.get((t, (n, k))) is True
    held, xs = ops.scan_split({"mlp": {"wg": h, "bias": "b"}})
    assert held["mlp"]["wg"] is h and xs["mlp"]["wg"] is None and xs["mlp"]["bias"] == "b"
    xb, x = _x(rng, 4, k, cuda)
    for layer in range(L):
        w = ops.scan_join(held, xs, torch.tensor(layer, dtype=torch.int32, device=cuda))["mlp"]["wg"]
        assert isinstance(w, ops.At)
        got = ops.qmatmul(x, w).float().cpu().numpy()
        assert np.array_equal(got, ops.qmatmul(x, ops.slice_layer(h, layer)).float().cpu().numpy())
        ref = R.bf16_to_f32(xb).astype(np.float64) @ R.dequant(st[layer], t, k).astype(np.float64).T
        assert_product(got, ref, f"layer {layer}")
        assert diff_bits(ops.dequant(w).cpu().numpy(), R.dequant(st[layer], t, k)) == 0


@pytest.mark.gpu
@pytest.mark.parametrize("t", [R.Q4_0, R.Q8_0, R.Q4_K, R.Q5_K, R.Q6_K])
def test_contract_check_and_take_rows(t, cuda):
    ops.load_kernels()
    rng = np.random.default_rng(50 + t)
    k = R.TYPES[t][1] * 2
    raw = rng.integers(0, 256, (9, R.row_bytes(t, k)), dtype=np.uint8)
    raw[0], raw[1] = 0, 0xFF                                              # zero and NaN blocks
    assert ops.contract_check(t, raw, (9, k)) == (True, 0)
    assert ops.contract_check(11, raw, (9, k)) is None                   # Q3_K: no kernel planes
    w = R.dequant(raw, t, k)
    for h in (ops.prepare(raw, t, (9, k)), ops.prepare(raw, t, (9, k), use_kernel=False)):
        got = ops.take_rows(h, [3, 0, -1, 1]).cpu().numpy()
        assert diff_bits(got, w[[3, 0, -1, 1]]) == 0


# ------------------------------------------------------------------------------------------- mixed block types
def _mixed_case(rng, types, n, k):
    return [(G.RAW[t](rng, n, k), t) for t in types]


@pytest.mark.gpu
@pytest.mark.parametrize("index", ["host", "device"])
def test_mixed_role_picks_each_layer(index, cuda):
    """one role whose block types differ by layer (a Q4_K_M file keeps some layers' ffn_down in Q6_K): stack_mixed
    holds one stack per type with which / sub; scan_split keeps it whole and scan_join hands the loop body a Pick; the
    Pick's product, dequant and rows equal the layer's own handle bit for bit and the oracle (reference
    src/mashbox/ops/__init__.py:216-270,515,606; gguf/archs/dense.py:206-218)"""
    import torch
    ops.load_kernels()
    rng = np.random.default_rng(60)
    types = [R.Q4_K, R.Q6_K, R.Q4_K, R.Q6_K, R.Q4_K]
    n, k = 48, 512
    layers = _mixed_case(rng, types, n, k)
    h = ops.stack_mixed(layers, (n, k))
    assert isinstance(h, ops.Mixed) and h.types == (R.Q4_K, R.Q6_K) and len(h.stacks) == 2
    assert all(isinstance(s, ops.Packed) for s in h.stacks)
    assert h.which.tolist() == [0, 1, 0, 1, 0] and h.sub.tolist() == [0, 0, 1, 1, 2]
    held, xs = ops.scan_split({"mlp": {"wd": h, "norm": "n"}})
    assert held["mlp"]["wd"] is h and xs["mlp"]["norm"] == "n"
    xb, x = _x(rng, 3, k, cuda)
    for layer, (raw, t) in enumerate(layers):
        li = torch.tensor(layer, dtype=torch.int32, device=cuda) if index == "device" else layer
        w = ops.scan_join(held, xs, li)["mlp"]["wd"]
        assert isinstance(w, ops.Pick)
        one = ops.prepare(raw, t, (n, k))
        got = ops.qmatmul(x, w)
        assert np.array_equal(got.view(torch.int16).cpu().numpy(), ops.qmatmul(x, one).view(torch.int16).cpu().numpy())
        wf = R.dequant(raw, t, k)
        assert_product(got.float().cpu().numpy(), R.bf16_to_f32(xb).astype(np.float64) @ wf.astype(np.float64).T)
        assert diff_bits(ops.dequant(w).cpu().numpy(), wf) == 0
        assert diff_bits(ops.take_rows(w, [5, -1, 0]).cpu().numpy(), wf[[5, -1, 0]]) == 0
        assert diff_bits(ops.dequant(ops.slice_layer(h, layer)).cpu().numpy(), wf) == 0


@pytest.mark.gpu
def test_mixed_role_with_an_exact_path_stack(cuda):
    """a Mixed whose Q6_K stack runs on the exact path (kernel types without Q6_K): the Pick reads its index on the host
    and each layer equals its own exact or kernel handle"""
    import torch
    ops.load_kernels()
    rng = np.random.default_rng(61)
    types = [R.Q8_0, R.Q6_K, R.Q8_0]
    n, k = 40, 256
    layers = _mixed_case(rng, types, n, k)
    saved = ops._KERNELS.types
    ops._KERNELS.types = frozenset({R.Q8_0})
    try:
        h = ops.stack_mixed(layers, (n, k))
    finally:
        ops._KERNELS.types = saved
    assert isinstance(h.stacks[0], ops.Packed) and isinstance(h.stacks[1], ops.Raw)
    held, xs = ops.scan_split([h])
    xb, x = _x(rng, 2, k, cuda)
    for layer, (raw, t) in enumerate(layers):
        w = ops.scan_join(held, xs, torch.tensor(layer, dtype=torch.int32, device=cuda))[0]
        wf = R.dequant(raw, t, k)
        assert_product(ops.qmatmul(x, w).float().cpu().numpy(), R.bf16_to_f32(xb).astype(np.float64) @ wf.astype(np.float64).T)
        assert diff_bits(ops.dequant(w).cpu().numpy(), wf) == 0


@pytest.mark.gpu
@pytest.mark.parametrize("t", [R.Q4_0, R.Q8_0, R.Q4_K, R.Q5_K, R.Q6_K])
def test_take_rows_reads_only_the_rows_asked(t, cuda):
    """kernel planes: take_rows dequantizes the asked rows only (mbq_dequant_rows), bit for bit dequant(h)[ids], ids of
    any shape, negative ids from the end and past-the-end ids clamped as jax.numpy indexes; a stack's layer too"""
    import torch
    ops.load_kernels()
    rng = np.random.default_rng(70 + t)
    n, k = 300, R.TYPES[t][1] * 3
    st = np.stack([G.RAW[t](rng, n, k) for _ in range(2)])
    planes = KQ.repack_host(t, st, (n, k)).to(cuda)
    ids = np.array([[0, 7, n - 1], [-1, -n, 150]])
    for layer in range(2):
        w = R.dequant(st[layer], t, k)
        got = KQ.take_rows(planes, torch.from_numpy(ids).to(cuda), layer=layer).cpu().numpy()
        assert got.shape == (2, 3, k) and diff_bits(got, w[ids]) == 0
        dl = torch.tensor(layer, dtype=torch.int32, device=cuda)
        assert diff_bits(KQ.take_rows(planes, torch.from_numpy(ids).to(cuda), layer=dl).cpu().numpy(), w[ids]) == 0
    one = planes[1]
    clamp = KQ.take_rows(one, torch.tensor([n + 5, -n - 3], device=cuda)).cpu().numpy()
    w = R.dequant(st[1], t, k)
    assert diff_bits(clamp, w[[n - 1, 0]]) == 0
