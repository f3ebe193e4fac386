"""The GGUF reader (mashbox_amd/gguf.py) on files written from the container layout, and (GPU) a file taken through
the load path: gguf.File -> ops.prepare -> ops.qmatmul, against the oracle.

Mirrors the reference's reader contract (reference src/mashbox/gguf/reader.py:14,30-87): metadata values, tensor
dims reversed to (rows = out, cols = in), rows() as (..., rows, row_bytes), raw bytes never copied, split models read
as one with a missing shard named, little-endian v2/v3 only; and the load test of reference
tests/cpu/test_gguf_dense.py:98-118 (a file's weights through the kernel path against the exact product)."""
import os

import numpy as np
import pytest

from oracle import gen as G
from oracle import ref as R
from tests import _gguf_write as W
from tests._check import assert_product, diff_bits

from mashbox_amd import gguf

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def _model(rng):
    """a small two-layer model: a Q4_K ffn_down in layer 0 and Q6_K in layer 1 (a Q4_K_M mix), Q8_0 attention, a
    float32 norm"""
    return {
        "blk.0.attn_q.weight": (8, (64, 256), G.q8_0_raw(rng, 64, 256)),
        "blk.0.ffn_down.weight": (12, (48, 512), G.q4_k_raw(rng, 48, 512)),
        "blk.1.attn_q.weight": (8, (64, 256), G.q8_0_raw(rng, 64, 256)),
        "blk.1.ffn_down.weight": (14, (48, 512), G.q6_k_raw(rng, 48, 512)),
        "output_norm.weight": (0, (256,), rng.standard_normal(256).astype(np.float32).view(np.uint8)),
    }


META = {"general.architecture": "qwen3", "general.name": "tiny", "qwen3.block_count": ("u32", 2),
        "qwen3.rope.freq_base": ("f32", 1e6), "tokenizer.ggml.tokens": ["a", "b", "<s>"],
        "tokenizer.ggml.token_type": np.array([1, 1, 3], np.int32), "general.alignment": ("u32", 64)}


def test_reads_header_metadata_and_tensors(tmp_path):
    rng = np.random.default_rng(0)
    T = _model(rng)
    p = str(tmp_path / "m.gguf")
    W.write(p, META, T, align=64)
    with gguf.File(p) as f:
        assert f.version == 3 and f.arch == "qwen3" and f.get("general.name") == "tiny"
        assert f.get("qwen3.block_count") == 2 and abs(f.get("qwen3.rope.freq_base") - 1e6) < 1
        assert f.get("tokenizer.ggml.tokens") == ["a", "b", "<s>"]
        assert f.get("tokenizer.ggml.token_type").tolist() == [1, 1, 3] and f.get("missing", 7) == 7
        assert set(f.tensors) == set(T) and f.paths == [p] and f.size == os.path.getsize(p)
        for name, (t, shape, raw) in T.items():
            x = f.tensors[name]
            assert x.type == t and x.shape == shape, name
            rows = x.rows()
            want = raw.reshape(shape[:-1] + (-1,)) if len(shape) > 1 else raw
            assert rows.shape == want.shape and np.array_equal(rows, want), name
            assert not rows.flags.writeable, "tensor bytes are a read-only view of the map, never a copy"
        census, total = f.census()
        assert census["Q8_0"]["tensors"] == 2 and total == sum(np.asarray(r).nbytes for _, _, r in T.values())


def test_split_model_reads_as_one_and_names_a_missing_shard(tmp_path):
    rng = np.random.default_rng(1)
    T = _model(rng)
    paths = W.write_split(str(tmp_path / "m"), META, T, shards=3)
    for p in paths:                                            # opening any shard opens the whole model
        with gguf.File(p) as f:
            assert f.paths == paths and set(f.tensors) == set(T) and f.arch == "qwen3"
            assert f.get("split.no") == 0, "each key comes from the first shard that holds it"
            for name, (t, shape, raw) in T.items():
                assert np.array_equal(f.tensors[name].raw, np.asarray(raw).reshape(-1))
    os.remove(paths[1])
    with pytest.raises(gguf.GGUFError, match="missing: m-00002-of-00003.gguf"):
        gguf.File(paths[0])


def test_rejects_what_it_cannot_read(tmp_path):
    p = str(tmp_path / "bad.gguf")
    open(p, "wb").write(b"GGML" + bytes(60))
    with pytest.raises(gguf.GGUFError, match="not a GGUF"):
        gguf.File(p)
    open(p, "wb").write(b"GGUF" + (3 << 24).to_bytes(4, "little") + bytes(56))     # a big-endian version field
    with pytest.raises(gguf.GGUFError, match="little-endian"):
        gguf.File(p)
    W.write(p, {}, {"w": (8, (4, 64), np.zeros((4, 68), np.uint8))})
    b = open(p, "rb").read()
    open(p, "wb").write(b[:-40])
    with pytest.raises(gguf.GGUFError, match="past the end"):
        gguf.File(p)


FIXTURE = "/root/reference/tests/fixtures/gguf/qwen3-kquant.gguf"


@pytest.mark.skipif(not os.path.exists(FIXTURE), reason="the reference's fixture models are read where they exist")
def test_reads_the_reference_fixture_model():
    """the reference's llama-quantize fixture model: the tensors the committed golden slices came from have the same
    bytes (their sha256 is recorded in each fixture), and every K-quant / Q8_0 weight dequantizes through the oracle"""
    with gguf.File(FIXTURE) as f:
        assert f.arch == "qwen3"
        checked = 0
        for name in sorted(os.listdir(GOLDEN)):
            if not name.startswith("kquant_qwen3_"):
                continue
            z = np.load(os.path.join(GOLDEN, name), allow_pickle=False)
            src = str(z["source"]).split()                   # "<file> sha256 <hex> tensor <name> <type> (r, c) rows 0-15"
            x = f.tensors[src[src.index("tensor") + 1]]
            assert int(z["t"]) == x.type and int(z["cols"]) == x.shape[-1] and x.type_name == src[src.index("tensor") + 2]
            assert np.array_equal(x.rows()[:z["raw"].shape[0]], z["raw"]), name
            checked += 1
        assert checked >= 5
        for x in f.tensors.values():
            if x.type in R.TYPES and x.type in (8, 12, 13, 14) and len(x.shape) == 2:
                assert np.all(np.isfinite(R.dequant(x.rows(), x.type, x.shape[-1])))


@pytest.mark.gpu
def test_a_gguf_file_through_the_load_path(tmp_path, cuda):
    """write a model, read it back, prepare every weight (kernel planes; the Q4_K / Q6_K ffn_down as one Mixed role) and
    multiply: equal to the oracle's exact product, and dequant bit for bit"""
    import torch
    from mashbox_amd import ops
    ops.load_kernels()
    rng = np.random.default_rng(2)
    T = _model(rng)
    p = str(tmp_path / "m.gguf")
    W.write(p, META, T)
    with gguf.File(p) as f:
        for name, x in f.tensors.items():
            if x.type not in ops.TYPES or len(x.shape) != 2:
                continue                                          # the norm vectors: not matmul weights
            h = ops.prepare(x.rows(), x.type, x.shape)
            assert isinstance(h, ops.Packed if x.type in R.KERNEL_TYPES else ops.Raw), name
            assert diff_bits(ops.dequant(h).cpu().numpy(), R.dequant(x.rows(), x.type, x.shape[-1])) == 0
            xb = G.acts(rng, 3, x.shape[-1])
            y = ops.qmatmul(torch.from_numpy(xb.astype(np.int16)).view(torch.bfloat16).to(cuda), h)
            ref = R.bf16_to_f32(xb).astype(np.float64) @ R.dequant(x.rows(), x.type, x.shape[-1]).astype(np.float64).T
            assert_product(y.float().cpu().numpy(), ref, name)
        role = [f.tensors[f"blk.{l}.ffn_down.weight"] for l in range(2)]
        h = ops.stack_mixed([(x.rows(), x.type) for x in role], role[0].shape)
        assert isinstance(h, ops.Mixed) and h.types == (12, 14)
        held, xs = ops.scan_split({"wd": h})
        xb = G.acts(rng, 2, 512)
        x16 = torch.from_numpy(xb.astype(np.int16)).view(torch.bfloat16).to(cuda)
        for l, x in enumerate(role):
            w = ops.scan_join(held, xs, torch.tensor(l, dtype=torch.int32, device=cuda))["wd"]
            ref = R.bf16_to_f32(xb).astype(np.float64) @ R.dequant(x.rows(), x.type, 512).astype(np.float64).T
            assert_product(ops.qmatmul(x16, w).float().cpu().numpy(), ref, f"layer {l}")
    ops.load_kernels(module="off")
