"""The .bshj reader (mashbox_amd/bshj.py) on files written from the documented container layout, and the oracle's
int8 embedding rows. CPU only.

Mirrors the reference's loader checks: tensors read back bit for bit (bf16, f32, int8), a bad magic / major / newer
minor / nonzero reserved bytes / misaligned data / a record whose bytes disagree with its shape raise one ValueError
naming each problem
(reference src/mashbox/bshj.py:33-53); the int8 per-row weights are found by their `_scale` companion and the layer
prefix by its first name (reference src/mashbox/models/qwen3_8_27b/weights.py:27-28, 49-50)."""
import json
import os
import struct

import numpy as np
import pytest
import torch

from mashbox_amd import bshj
from oracle import ref as R
from tests import _bshj_write as W


def _tensors(rng):
    return {
        "model.language_model.layers.0.mlp.up_proj.weight": rng.integers(-127, 128, (24, 40), dtype=np.int8),
        "model.language_model.layers.0.mlp.up_proj.weight_scale": rng.uniform(1e-3, 1e-2, 24).astype(np.float32),
        "model.language_model.norm.weight": R.bf16_round(rng.standard_normal(40).astype(np.float32)),
        "model.language_model.embed_tokens.weight": rng.integers(-128, 128, (64, 40), dtype=np.int8),
        "model.language_model.embed_tokens.weight_scale": rng.uniform(1e-4, 3e-2, 64).astype(np.float32),
        "lm_head.weight": rng.standard_normal((7, 3)).astype(np.float32),
    }


def test_reads_every_tensor_back_bit_for_bit(tmp_path):
    rng = np.random.default_rng(0)
    T = _tensors(rng)
    p = str(tmp_path / "w.bshj")
    W.write(p, T, {"bshj": {"quant": {"type": "TEST"}}})
    with bshj.File(p) as f:
        assert f.meta()["bshj"] == {"quant": {"type": "TEST"}}
        assert set(f.tensors) == set(T)
        for name, a in T.items():
            got = f.array(name)
            assert got.shape == a.shape and np.array_equal(got.view(np.uint8), a.view(np.uint8)), name
        nw = f.torch_tensor("model.language_model.norm.weight")
        assert nw.dtype == torch.bfloat16
        assert np.array_equal(nw.view(torch.int16).numpy().view(np.uint16), T["model.language_model.norm.weight"])
        assert bshj.prefix(f.tensors) == "model.language_model."
        assert bshj.quantised(f, "model.language_model.layers.0.mlp.up_proj")
        assert not bshj.quantised(f, "lm_head")
        f.advise("lm_head.weight")
    assert bshj.prefix(["model.layers.0.x", "lm_head.weight"]) == "model."


def _raw_file(tmp_path, **kw):
    p = str(tmp_path / "bad.bshj")
    W.write(p, {"a": np.arange(8, dtype=np.int8)}, **kw)
    return p


@pytest.mark.parametrize("kw,msg", [(dict(magic=b"GGUF"), "is not BSHJ 1.x"), (dict(major=2), "is not BSHJ 1.x"),
                                    (dict(minor=2), "newer"), (dict(reserved=b"\x01" + bytes(15)), "reserved")])
def test_rejects_bad_fixed_headers(tmp_path, kw, msg):
    with pytest.raises(ValueError, match=msg):
        bshj.File(_raw_file(tmp_path, **kw))


def test_rejects_bad_layouts_and_records(tmp_path):
    p = _raw_file(tmp_path)
    b = bytearray(open(p, "rb").read())
    # data offset not a multiple of align
    bad = bytearray(b)
    bad[16:24] = struct.pack("<Q", struct.unpack("<Q", b[16:24])[0] + 8)
    open(p, "wb").write(bad)
    with pytest.raises(ValueError, match="not a multiple of the alignment"):
        bshj.File(p)
    # data running past the end of the file
    bad = bytearray(b)
    bad[32:40] = struct.pack("<Q", 1 << 40)
    open(p, "wb").write(bad)
    with pytest.raises(ValueError, match="runs past"):
        bshj.File(p)
    # a record whose nbytes disagrees with its shape
    jl = struct.unpack("<Q", b[8:16])[0]
    hdr = json.loads(bytes(b[64:64 + jl]).rstrip(b" "))
    hdr["tensors"]["a"]["nbytes"] = 9
    raw = json.dumps(hdr, separators=(",", ":")).encode()
    bad = bytearray(b)
    bad[64:64 + jl] = raw + b" " * (jl - len(raw))
    open(p, "wb").write(bad)
    with pytest.raises(ValueError, match="tensor a: 9 bytes"):
        bshj.File(p)
    open(p, "wb").close()
    with pytest.raises(ValueError, match="shorter than"):
        bshj.File(p)


def test_int8_weight_shape_rules(tmp_path):
    p = str(tmp_path / "w.bshj")
    W.write(p, {"x.weight": np.zeros((4, 8), np.int8), "x.weight_scale": np.ones(3, np.float32),
                "y.weight": np.zeros((4, 8), np.int8)})
    with bshj.File(p) as f:
        for name in ("x.weight", "y.weight"):
            with pytest.raises(ValueError, match="not an int8"):
                bshj.int8_weight(f, name, device="cpu")


def test_int8_embed_oracle_matches_torch():
    """the oracle's rows f32(q) * s equal torch's own CPU float32 product, and their bfloat16 rounding torch's cast; ids
    index as jax.numpy does (negative ids wrap once, then every id is clamped)"""
    rng = np.random.default_rng(1)
    n, d = 96, 40
    q = rng.integers(-128, 128, (n, d), dtype=np.int8)
    s = rng.uniform(1e-4, 3e-2, n).astype(np.float32)
    toks = np.array([[0, 1, 31, 32, n - 1], [-1, -n, -n - 5, n, n + 7]])
    want_idx = np.array([[0, 1, 31, 32, n - 1], [n - 1, 0, 0, n - 1, n - 1]])
    y = R.int8_embed(q, s, toks)
    t = torch.from_numpy(q).float()[torch.from_numpy(want_idx)] * torch.from_numpy(s)[torch.from_numpy(want_idx)][..., None]
    assert np.array_equal(y.view(np.uint32), t.numpy().view(np.uint32))
    assert np.array_equal(R.bf16_round(y), t.to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16))
