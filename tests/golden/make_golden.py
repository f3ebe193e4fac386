"""Writes the golden fixtures of tests/golden (run in the build container, where the reference tree is mounted).

    python tests/golden/make_golden.py [/root/reference]

Fixtures (NumPy .npz, no pickles):
  random_<TYPE>_k<KB>.npz    6 rows x KB blocks of random bytes with an all-zero row and an all-0xFF row (every fp16
                             scale value: normal, subnormal, inf, NaN), the shape of the reference's own dequant test
                             (reference tests/cpu/test_gguf_dequant.py:20-27); raw -> w (float32 dequant bits)
  kquant_<file>_<tensor>.npz real llama-quantize blocks: the first 16 rows of Q4_K, Q5_K, Q6_K and Q8_0 weights of the
                             reference's fixture models (reference tests/fixtures/gguf/*-kquant.gguf, Apache-2.0, made by
                             llama-quantize at llama.cpp a37cc46; the source file's sha256 is stored), with 3 bf16
                             activation rows x and their float64 product y64; also the exact path's other types those
                             files hold (Q5_1, Q2_K, Q3_K, IQ4_NL, IQ4_XS, F32)
  random_<TYPE>_k<KB>.npz    also for the exact path's other types (F32, F16, BF16, Q4_1, Q5_0, Q5_1, Q2_K, Q3_K,
                             IQ4_NL, IQ4_XS, TQ1_0, TQ2_0, MXFP4, NVFP4), KB blocks of 1, 2 and 16 (float types: 64,
                             128 and 1024 values)
Existing files are kept (their bytes do not change); --force writes every file again.
Expected values come from the oracle (oracle/ref.py), pinned independently by tests/test_oracle.py; the fixtures freeze
them so that a later change to the oracle or the kernels is checked against the same bytes.
"""
import hashlib
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)

from mashbox_amd import gguf  # noqa: E402
from oracle import gen as G  # noqa: E402
from oracle import ref as R  # noqa: E402

KQUANT = [("qwen3-kquant", ["blk.0.attn_k.weight", "blk.0.ffn_gate.weight", "blk.0.attn_q.weight", "token_embd.weight",
                            "blk.0.ffn_down.weight", "output.weight", "blk.0.ffn_up.weight"]),
          ("gemma4-kquant", ["blk.0.ffn_up.weight", "blk.0.ffn_down.weight", "blk.0.attn_v.weight",
                             "blk.2.attn_output.weight"]),
          ("qwen35-kquant", ["blk.0.attn_qkv.weight", "blk.0.ffn_down.weight"])]
# the exact path's other types in the same files
KQUANT_EXACT = [("gemma4-kquant", ["blk.0.attn_output.weight"]),
                ("qwen3-kquant", ["blk.0.attn_output.weight", "blk.0.attn_v.weight"]),
                ("qwen35-kquant", ["blk.0.ffn_up.weight", "blk.3.attn_output.weight", "blk.0.ssm_conv1d.weight"])]


def main(ref_root, force=False):
    def save(path, **arrays):
        if force or not os.path.exists(path):
            np.savez_compressed(path, **arrays)

    for t in R.KERNEL_TYPES + R.EXACT_ONLY:
        name = R.TYPES[t][0]
        for kb in (1, 2, 16):
            rng = np.random.default_rng(7000 + 10 * t + kb)
            cols = R.TYPES[t][1] * kb if R.TYPES[t][1] > 1 else 64 * kb
            raw = rng.integers(0, 256, size=(6, R.row_bytes(t, cols)), dtype=np.uint8)
            raw[0], raw[1] = 0, 0xFF
            save(os.path.join(HERE, f"random_{name}_k{kb}.npz"), t=t, cols=cols, raw=raw, w=R.dequant(raw, t, cols))
    for fname, tensors in KQUANT + KQUANT_EXACT:
        path = os.path.join(ref_root, "tests", "fixtures", "gguf", fname + ".gguf")
        sha = hashlib.sha256(open(path, "rb").read()).hexdigest()
        with gguf.File(path) as f:
            for tn in tensors:
                ten = f.tensors[tn]
                rows, cols = ten.shape
                raw = np.array(ten.rows()[:16])
                w = R.dequant(raw, ten.type, cols)
                rng = np.random.default_rng(len(tn) + cols)
                x = G.acts(rng, 3, cols)
                y64 = R.bf16_to_f32(x).astype(np.float64) @ w.astype(np.float64).T
                out = os.path.join(HERE, f"kquant_{fname.split('-')[0]}_{tn.replace('.weight', '').replace('.', '_')}.npz")
                save(out, t=ten.type, cols=cols, raw=raw, w=w, x=x, y64=y64,
                     source=np.array(f"{fname}.gguf sha256 {sha} tensor {tn} {ten.type_name} ({rows}, {cols}) rows 0-15"))
    for n in sorted(os.listdir(HERE)):
        if n.endswith(".npz"):
            print(n, os.path.getsize(os.path.join(HERE, n)))


if __name__ == "__main__":
    args = [a for a in sys.argv[1:] if a != "--force"]
    main(args[0] if args else "/root/reference", force="--force" in sys.argv[1:])
