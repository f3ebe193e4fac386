"""Seeded synthetic inputs for the five BASELINE configs. TEST INFRASTRUCTURE (see oracle/ref.py header).

Draws use numpy.random.default_rng(seed) in the order the config text lists them; fp16 and bf16 values are made by
round-to-nearest-even casts. The parity tests use these generators (seed 0 for the full-size config tests). The bench
does not import the oracle: its inputs come from mashbox_amd/synth.py, torch's RNG on the GPU with the same value
ranges and block layouts, so its timings are of the same kind of data but not of these exact draws.

Block generators follow the value ranges of BASELINE.json's configs; the Q8_0 one has the same form as the reference's
own generator tests/cpu/test_moe_bundle_dense.py:81-87 (fp16 d uniform, int8 q uniform in [-127, 127]).
"""
from __future__ import annotations

import numpy as np

from . import ref as R

# the 7 projections of one 27B-class layer (configs 4 and 5): name -> (rows N = out, cols K = in)
LAYER_27B = {
    "q": (6144, 5120), "k": (1024, 5120), "v": (1024, 5120), "o": (5120, 6144),
    "gate": (17408, 5120), "up": (17408, 5120), "down": (5120, 17408),
}


def acts(rng, m: int, k: int) -> np.ndarray:
    """x bf16 ~ N(0,1): (m, k) bfloat16 bits as uint16"""
    return R.bf16_round(rng.standard_normal((m, k), dtype=np.float32))


def q8_0_raw(rng, n: int, k: int, lo=1e-3, hi=1e-2) -> np.ndarray:
    """(n, row_bytes) uint8 Q8_0 blocks: d fp16 ~ U(lo, hi), qs int8 uniform in [-127, 127]"""
    nb = k // 32
    d = rng.uniform(lo, hi, (n, nb)).astype(np.float16).view(np.uint8).reshape(n, nb, 2)
    q = rng.integers(-127, 128, (n, nb, 32), dtype=np.int8).view(np.uint8)
    return np.concatenate([d, q], axis=-1).reshape(n, nb * 34)


def q4_0_raw(rng, n: int, k: int, lo=1e-3, hi=1e-2) -> np.ndarray:
    """(n, row_bytes) uint8 Q4_0 blocks: d fp16 ~ U(lo, hi); 4-bit quants uniform in [0, 15], two per byte (value i in
    the low nibble of byte i, value 16 + i in its high nibble; src/mashbox/ops/reference.py:66-70)"""
    nb = k // 32
    d = rng.uniform(lo, hi, (n, nb)).astype(np.float16).view(np.uint8).reshape(n, nb, 2)
    q = rng.integers(0, 16, (n, nb, 2, 16), dtype=np.uint8)
    return np.concatenate([d, q[:, :, 0] | (q[:, :, 1] << 4)], axis=-1).reshape(n, nb * 18)


def q4_k_raw(rng, n: int, k: int, lo=1e-3, hi=1e-2) -> np.ndarray:
    """(n, row_bytes) uint8 Q4_K super-blocks: d, dmin fp16 ~ U(lo, hi); 8 six-bit scales and mins uniform in
    [0, 63]; 4-bit quants uniform in [0, 15] (packed two per byte as the Q4_K layout holds them)"""
    nb = k // 256
    d = rng.uniform(lo, hi, (n, nb)).astype(np.float16).view(np.uint8).reshape(n, nb, 2)
    dmin = rng.uniform(lo, hi, (n, nb)).astype(np.float16).view(np.uint8).reshape(n, nb, 2)
    sc = rng.integers(0, 64, (n, nb, 8), dtype=np.uint8)
    mn = rng.integers(0, 64, (n, nb, 8), dtype=np.uint8)
    q = rng.integers(0, 16, (n, nb, 256), dtype=np.uint8)
    # sub-block 2g = low nibbles of bytes [32g, 32g+32), sub-block 2g+1 = their high nibbles (reference.py:58-60,148)
    q = q.reshape(n, nb, 4, 2, 32)
    qs = (q[:, :, :, 0, :] | (q[:, :, :, 1, :] << 4)).reshape(n, nb, 128)
    return np.concatenate([d, dmin, R.pack_scale_min_k4(sc, mn), qs], axis=-1).reshape(n, nb * 144)


def q5_k_raw(rng, n: int, k: int, lo=1e-3, hi=1e-2) -> np.ndarray:
    """(n, row_bytes) uint8 Q5_K super-blocks: d, dmin fp16 ~ U(lo, hi) / 2; 8 six-bit scales and mins uniform in
    [0, 63]; 5-bit quants uniform in [0, 31], packed as the Q5_K layout holds them (src/mashbox/ops/reference.py:150-159)"""
    nb = k // 256
    d = (rng.uniform(lo, hi, (n, nb)) / 2).astype(np.float16).view(np.uint8).reshape(n, nb, 2)
    dmin = (rng.uniform(lo, hi, (n, nb)) / 2).astype(np.float16).view(np.uint8).reshape(n, nb, 2)
    sc = rng.integers(0, 64, (n, nb, 8), dtype=np.uint8)
    mn = rng.integers(0, 64, (n, nb, 8), dtype=np.uint8)
    q = rng.integers(0, 32, (n, nb, 8, 32), dtype=np.uint8)           # value 32j + i
    # qs[32g + i]: low nibble = q(2g, i) & 15, high nibble = q(2g + 1, i) & 15; qh[i] bit j = q(j, i) >> 4
    qs = ((q[:, :, 0::2] & 15) | ((q[:, :, 1::2] & 15) << 4)).reshape(n, nb, 128)
    qh = sum(((q[:, :, j] >> 4) << j) for j in range(8)).astype(np.uint8)
    return np.concatenate([d, dmin, R.pack_scale_min_k4(sc, mn), qh, qs], axis=-1).reshape(n, nb * 176)


def q6_k_raw(rng, n: int, k: int, lo=1e-3, hi=1e-2) -> np.ndarray:
    """(n, row_bytes) uint8 Q6_K super-blocks: d fp16 ~ U(lo, hi) / 64; 16 int8 scales uniform in [-127, 127]; 6-bit
    quants uniform in [0, 63], packed as the Q6_K layout holds them (src/mashbox/ops/reference.py:164-173)"""
    nb = k // 256
    q = rng.integers(0, 64, (n, nb, 2, 4, 32), dtype=np.uint8)        # value 128g + 32r + i
    # ql[64g + 32j + i]: low nibble = q(g, j, i) & 15, high nibble = q(g, 2 + j, i) & 15
    ql = np.concatenate([(q[:, :, :, j] & 15) | ((q[:, :, :, 2 + j] & 15) << 4) for j in range(2)], -1)
    qh = sum(((q[:, :, :, r] >> 4) << (2 * r)) for r in range(4)).astype(np.uint8)
    sc = rng.integers(-127, 128, (n, nb, 16), dtype=np.int8).view(np.uint8)
    d = (rng.uniform(lo, hi, (n, nb)) / 64).astype(np.float16).view(np.uint8).reshape(n, nb, 2)
    return np.concatenate([ql.reshape(n, nb, 128), qh.reshape(n, nb, 64), sc, d], axis=-1).reshape(n, nb * 210)


def int8_weights(rng, n: int, k: int, lo=1e-3, hi=1e-2):
    """int8 per-output-channel: q (n, k) uniform in [-127, 127], s (n,) float32 ~ U(lo, hi)"""
    q = rng.integers(-127, 128, (n, k), dtype=np.int8)
    s = rng.uniform(lo, hi, n).astype(np.float32)
    return q, s


RAW = {R.Q4_0: q4_0_raw, R.Q8_0: q8_0_raw, R.Q4_K: q4_k_raw, R.Q5_K: q5_k_raw, R.Q6_K: q6_k_raw}


def config(idx: int, seed: int = 0, scale: float = 1.0):
    """inputs of BASELINE config idx (1..5). scale < 1 shrinks N (rows) for quick checks; K stays the config's.
    -> dict(kind, t (ggml type or 'int8'), m, projections=[(name, n, k, weights..., x)])"""
    rng = np.random.default_rng(seed)

    def rows(n):
        return max(16, int(round(n * scale / 16)) * 16) if scale != 1.0 else n

    if idx == 1:
        x = acts(rng, 1, 4096)
        q, s = int8_weights(rng, rows(4096), 4096)
        return dict(t="int8", m=1, projections=[("w", q.shape[0], 4096, (q, s), x)])
    if idx == 2:
        x = acts(rng, 1, 5120)
        raw = q8_0_raw(rng, rows(17408), 5120)
        return dict(t=R.Q8_0, m=1, projections=[("w", raw.shape[0], 5120, raw, x)])
    if idx == 3:
        x = acts(rng, 1, 17408)
        raw = q4_k_raw(rng, rows(5120), 17408)
        return dict(t=R.Q4_K, m=1, projections=[("w", raw.shape[0], 17408, raw, x)])
    if idx in (4, 5):
        m = 64 if idx == 4 else 2048
        projs = []
        for name, (n, k) in LAYER_27B.items():
            x = acts(rng, m, k)
            if idx == 4:
                q, s = int8_weights(rng, rows(n), k)
                projs.append((name, q.shape[0], k, (q, s), x))
            else:
                raw = q4_k_raw(rng, rows(n), k)
                projs.append((name, raw.shape[0], k, raw, x))
        return dict(t="int8" if idx == 4 else R.Q4_K, m=m, projections=projs)
    raise ValueError(f"no config {idx}")


def algorithmic_bytes(t, m: int, n: int, k: int) -> int:
    """packed weight bytes + scales + x + y (bf16) for one projection (the bench's GB/s numerator)"""
    if t == "int8":
        w = n * k + 4 * n
    else:
        w = n * R.row_bytes(t, k)
    return w + 2 * m * k + 2 * m * n
