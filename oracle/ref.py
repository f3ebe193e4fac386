"""CPU restatement of mashbox's quantized-linear exact path. TEST INFRASTRUCTURE ONLY.

This module is the parity checker for the MI355X kernels in `mashbox_amd`. Only `tests/`, `__graft_entry__.smoke()` and
the `cpu_baseline` leg of `bench.py` may import it, and only as the checker or the timed CPU baseline: the product path
(`mashbox_amd`) never imports, links or calls anything under `oracle/`.

It restates, from scratch in NumPy, what the reference computes (reference = /root/reference, mashbox-labs/mashbox):

  ggml type table, row bytes        src/mashbox/ops/reference.py:22-29, 390-395
  little-endian fp16 -> f32         src/mashbox/ops/reference.py:37-51   (_u16le, _f16)
  nibble split                      src/mashbox/ops/reference.py:58-60   (_nib)
  Q4_0 block                        src/mashbox/ops/reference.py:66-70   (_q4_0)
  Q8_0 block                        src/mashbox/ops/reference.py:101-103 (_q8_0)
  6-bit scale/min unpack            src/mashbox/ops/reference.py:132-139 (_scale_min_k4)
  Q4_K super-block                  src/mashbox/ops/reference.py:142-149 (_q4_k)
  Q5_K super-block                  src/mashbox/ops/reference.py:150-159 (_q5_k)
  Q6_K super-block                  src/mashbox/ops/reference.py:164-173 (_q6_k)
  dequant(raw, t, cols)             src/mashbox/ops/reference.py:398-409
  exact-path row chunking           src/mashbox/ops/__init__.py:555-571  (EXACT_CHUNK, exact_chunk_rows)
  exact-path product                src/mashbox/ops/__init__.py:574-576, 624-632 (_exact, qmatmul's Raw branch)
  int8 per-channel linear           src/mashbox/models/qwen3_8_27b/model.py:72-82 (linear)
  int8 per-row quantizer (fixture)  tests/cpu/qwen3_8_27b_checks.py:113-117 (int8_rows)
  int8 embedding rows               src/mashbox/models/qwen3_8_27b/model.py:132-139 (embed; its int8_rows at :117-129
                                    equals the plain gather q[toks])

The reference's own arithmetic follows gguf-py 0.19.0 (gguf/quants.py), a third-party package absent here; its published
algorithm is the one restated by the reference file above, and that is what this module follows.

How each function is pinned (tests/test_oracle.py):
  f16_to_f32      every one of the 65,536 fp16 bit patterns against an independent decoder built from the IEEE-754
                  binary16 definition (sign, exponent, fraction; subnormals; inf; NaN).
  dequant Q4_0    closed form: v = d * (q - 8) is exact in float32 (at most 11 + 4 significant bits), checked against
                  `fractions` on every code at several d; the nibble order against a per-index restatement of llama.cpp's
                  scalar loop (dequantize_row_q4_0) on random blocks; all-zero / all-0xFF blocks, zero signs included.
  dequant Q8_0    closed form: v = q * d is exact in float32 for every finite fp16 d and int8 q (<= 19 significant bits),
                  checked against Python `fractions` arithmetic on a brute-force grid; all-zero / all-0xFF blocks.
  dequant Q4_K    closed form: v = RN_f32(d*sc*q - dmin*m) with a single rounding, checked against exact `fractions`
                  arithmetic rounded once; the packer `pack_scale_min_k4` round-trips `scale_min_k4` over all 64^2
                  (sc, m) values per slot; the nibble order is pinned by real llama-quantize blocks from the reference's
                  fixture file tests/fixtures/gguf/qwen3-kquant.gguf, whose dequantized rows must be smooth
                  weight-like values (see tests/golden).
  dequant Q5_K    closed form: v = RN_f32(d*sc*q - dmin*m) with a single rounding (q < 32: at most 11 + 6 + 5 bits in
                  the product), checked against exact `fractions` arithmetic rounded once; the bit layout against a
                  per-index restatement of llama.cpp's scalar loop (dequantize_row_q5_K) on random blocks and on the real
                  llama-quantize blocks of the reference's fixture files; all-zero / all-0xFF blocks.
  dequant Q6_K    closed form: v = (d*sc)*(q - 32) is exact in float32 (at most 11 + 7 + 5 significant bits), checked
                  against `fractions` on a grid; the bit layout against a per-index restatement of llama.cpp's scalar
                  loop (ggml-quants.c dequantize_row_q6_K, the algorithm gguf-py restates) on random blocks and on the
                  real llama-quantize blocks of the reference's fixture files; all-zero / all-0xFF blocks.
  qmatmul_exact   against a float64 product (reference bars: tests/contracts/test_ops.py:22-31), and chunked == whole.
  int8_embed      against torch's own CPU float32 product and bfloat16 cast of the same gathered rows (an independent
                  implementation of the two IEEE-754 roundings), and the index rule against jax.numpy's documented one
                  (negative ids wrap once, the rest clamp) on every edge id.
  int8_linear     per element closed form: every bf16(x)*bf16(q) product is exact in float32; checked against a float64
                  product of the same values.
"""
from __future__ import annotations

import numpy as np

# ggml type id -> (name, values per block, bytes per block) for the types on this path
# (src/mashbox/ops/reference.py:22-29 lists every ggml type; the kernel path covers these five, the types the
# reference's own kernel package gives planes: src/mashbox/ops/bundle.py:39)
TYPES = {2: ("Q4_0", 32, 18), 8: ("Q8_0", 32, 34), 12: ("Q4_K", 256, 144), 13: ("Q5_K", 256, 176), 14: ("Q6_K", 256, 210)}
Q4_0, Q8_0, Q4_K, Q5_K, Q6_K = 2, 8, 12, 13, 14
QK_K = 256
EXACT_CHUNK = 1 << 24          # src/mashbox/ops/__init__.py:555


def row_bytes(t: int, cols: int) -> int:
    """bytes of one row of `cols` values in ggml type t (src/mashbox/ops/reference.py:390-395)"""
    _, bs, ts = TYPES[t]
    if cols % bs:
        raise ValueError(f"{TYPES[t][0]}: row of {cols} values is not a multiple of the block size {bs}")
    return cols // bs * ts


# ------------------------------------------------------------------------------------------------ bf16 / fp16 helpers
def f16_to_f32(b: np.ndarray) -> np.ndarray:
    """(..., 2k) little-endian uint8 -> (..., k) float32, exact (src/mashbox/ops/reference.py:37-51)"""
    b = np.ascontiguousarray(b, dtype=np.uint8)
    u = b[..., 0::2].astype(np.uint16) | (b[..., 1::2].astype(np.uint16) << np.uint16(8))
    return u.view(np.float16).astype(np.float32)


def bf16_round(x: np.ndarray) -> np.ndarray:
    """float32 -> bfloat16 bits (uint16), round to nearest even; NaN -> a quiet NaN (torch/XLA convention)"""
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32)
    nan = (u & np.uint32(0x7FFFFFFF)) > np.uint32(0x7F800000)
    r = (u + np.uint32(0x7FFF) + ((u >> np.uint32(16)) & np.uint32(1))) >> np.uint32(16)
    return np.where(nan, (u >> np.uint32(16)) | np.uint32(0x40), r).astype(np.uint16)


def bf16_to_f32(h: np.ndarray) -> np.ndarray:
    """bfloat16 bits (uint16) -> float32, exact"""
    return (np.asarray(h, dtype=np.uint16).astype(np.uint32) << np.uint32(16)).view(np.float32)


def as_bf16(x: np.ndarray) -> np.ndarray:
    """float32 values rounded to the nearest bfloat16, returned as float32"""
    return bf16_to_f32(bf16_round(x))


# --------------------------------------------------------------------------------------------------------- blocks
def nib(qs: np.ndarray) -> np.ndarray:
    """(..., n) bytes -> (..., 2, n): low nibbles, then high nibbles (src/mashbox/ops/reference.py:58-60)"""
    return np.stack([qs & np.uint8(0x0F), qs >> np.uint8(4)], axis=-2)


def q4_0_blocks(b: np.ndarray) -> np.ndarray:
    """(N, 18) blocks -> (N, 32) float32: d * f32(q - 8), q = low nibbles of bytes 2-17 (values 0-15) then their high
    nibbles (values 16-31) (src/mashbox/ops/reference.py:66-70)"""
    n = b.shape[0]
    d = f16_to_f32(b[:, :2])                                  # (N, 1)
    q = nib(b[:, 2:]).reshape(n, 32).astype(np.int8) - np.int8(8)
    with np.errstate(invalid="ignore", over="ignore"):
        return d * q.astype(np.float32)


def q8_0_blocks(b: np.ndarray) -> np.ndarray:
    """(N, 34) blocks -> (N, 32) float32: f32(q) * d (src/mashbox/ops/reference.py:101-103)"""
    d = f16_to_f32(b[:, :2])                                  # (N, 1)
    q = b[:, 2:].view(np.int8).astype(np.float32)
    return q * d


def scale_min_k4(s: np.ndarray):
    """(N, 12) packed bytes -> 8 six-bit scales, 8 six-bit mins, each (N, 8) uint8
    (src/mashbox/ops/reference.py:132-139)"""
    s = s.reshape(-1, 3, 4)
    d, m, md = s[:, 0], s[:, 1], s[:, 2]
    sc = np.concatenate([d & 0x3F, (md & 0x0F) | ((d >> 2) & 0x30)], axis=-1)
    mn = np.concatenate([m & 0x3F, (md >> 4) | ((m >> 2) & 0x30)], axis=-1)
    return sc.astype(np.uint8), mn.astype(np.uint8)


def pack_scale_min_k4(sc: np.ndarray, mn: np.ndarray) -> np.ndarray:
    """inverse of scale_min_k4: (N, 8) six-bit scales and mins -> (N, 12) bytes (the builder's generator needs it)"""
    sc = np.asarray(sc, np.uint8)
    mn = np.asarray(mn, np.uint8)
    out = np.empty(sc.shape[:-1] + (12,), np.uint8)
    out[..., 0:4] = (sc[..., 0:4] & 0x3F) | ((sc[..., 4:8] >> 4) << 6)
    out[..., 4:8] = (mn[..., 0:4] & 0x3F) | ((mn[..., 4:8] >> 4) << 6)
    out[..., 8:12] = (sc[..., 4:8] & 0x0F) | ((mn[..., 4:8] & 0x0F) << 4)
    return out


def q4_k_blocks(b: np.ndarray) -> np.ndarray:
    """(N, 144) super-blocks -> (N, 256) float32: (d*sc_j)*q - dmin*m_j (src/mashbox/ops/reference.py:142-149)"""
    n = b.shape[0]
    d, dmin = f16_to_f32(b[:, 0:2]), f16_to_f32(b[:, 2:4])    # (N, 1) each
    sc, mn = scale_min_k4(b[:, 4:16])
    ds = (d * sc.astype(np.float32)).reshape(n, 8, 1)
    dm = (dmin * mn.astype(np.float32)).reshape(n, 8, 1)
    q = nib(b[:, 16:].reshape(n, 4, 32)).reshape(n, 8, 32).astype(np.float32)
    with np.errstate(invalid="ignore", over="ignore"):
        return (ds * q - dm).reshape(n, QK_K)


def q5_k_blocks(b: np.ndarray) -> np.ndarray:
    """(N, 176) super-blocks -> (N, 256) float32: (d*sc_j)*q - dmin*m_j over 8 sub-blocks of 32, q = low | high << 4
    (src/mashbox/ops/reference.py:150-159). Bytes: d, dmin fp16 0-3, 12 scale bytes 4-15 (as Q4_K), qh 16-47, qs 48-175.
    Value 32j + i: low = nibble j % 2 of qs[32 (j // 2) + i], high = bit j of qh[i]."""
    n = b.shape[0]
    d, dmin = f16_to_f32(b[:, 0:2]), f16_to_f32(b[:, 2:4])    # (N, 1) each
    sc, mn = scale_min_k4(b[:, 4:16])
    ds = (d * sc.astype(np.float32)).reshape(n, 8, 1)
    dm = (dmin * mn.astype(np.float32)).reshape(n, 8, 1)
    lo = nib(b[:, 48:].reshape(n, 4, 32)).reshape(n, 8, 32)
    hi = ((b[:, 16:48].reshape(n, 1, 32) >> np.arange(8, dtype=np.uint8).reshape(1, 8, 1)) & np.uint8(1))
    q = (lo | (hi << np.uint8(4))).astype(np.float32)
    with np.errstate(invalid="ignore", over="ignore"):
        return (ds * q - dm).reshape(n, QK_K)


def q6_k_blocks(b: np.ndarray) -> np.ndarray:
    """(N, 210) super-blocks -> (N, 256) float32: (d*sc_j)*(q - 32) over 16 sub-blocks of 16 values
    (src/mashbox/ops/reference.py:164-173). Bytes: ql 0-127 (low nibbles), qh 128-191 (2-bit highs), sc 192-207 (int8),
    d 208-209 (fp16). Value 128g + 32r + i (g < 2, r < 4, i < 32): low = nibble r // 2 of ql[64g + 32 (r % 2) + i],
    high = bits 2r, 2r + 1 of qh[32g + i]."""
    n = b.shape[0]
    ql, qh = b[:, :128], b[:, 128:192]
    sc = b[:, 192:208].view(np.int8).astype(np.float32)
    d = f16_to_f32(b[:, 208:210])                              # (N, 1)
    ds = (d * sc).reshape(n, 16, 1)
    lo = nib(ql.reshape(n, 2, 64)).reshape(n, 8, 32)
    hi = ((qh.reshape(n, 2, 1, 32) >> np.array([0, 2, 4, 6], np.uint8).reshape(1, 1, 4, 1)) & np.uint8(3)).reshape(n, 8, 32)
    q = ((lo | (hi << np.uint8(4))).astype(np.int16) - 32).astype(np.float32).reshape(n, 16, 16)
    with np.errstate(invalid="ignore", over="ignore"):
        return (ds * q).reshape(n, QK_K)


BLOCKS = {Q4_0: q4_0_blocks, Q8_0: q8_0_blocks, Q4_K: q4_k_blocks, Q5_K: q5_k_blocks, Q6_K: q6_k_blocks}


def dequant(raw: np.ndarray, t: int, cols: int) -> np.ndarray:
    """raw (..., row_bytes(t, cols)) uint8 -> (..., cols) float32, exact (src/mashbox/ops/reference.py:398-409)"""
    _, bs, ts = TYPES[t]
    raw = np.ascontiguousarray(raw, dtype=np.uint8)
    lead = raw.shape[:-1]
    with np.errstate(invalid="ignore", over="ignore"):
        out = BLOCKS[t](raw.reshape(-1, ts))
    return out.reshape(lead + (cols,))


# ---------------------------------------------------------------------------------------------------- exact product
def exact_chunk_rows(rows: int, cols: int, limit: int | None = None) -> int:
    """rows per rebuild step: the largest divisor of rows with rows*cols <= limit (src/mashbox/ops/__init__.py:558-571)"""
    limit = EXACT_CHUNK if limit is None else limit
    if rows * cols <= limit:
        return rows
    best, d = 1, 1
    while d * d <= rows:
        if rows % d == 0:
            for c in (d, rows // d):
                if c * cols <= limit and c > best:
                    best = c
        d += 1
    return best


def qmatmul_exact(x: np.ndarray, raw: np.ndarray, t: int, shape, limit: int | None = None, threads: int = 1) -> np.ndarray:
    """x (..., cols) float32 values @ W.T -> (..., rows) float32 (NOT yet rounded to x's dtype).

    The exact path: the float32 weights are rebuilt from the blocks a chunk of rows at a time and multiplied with a
    float32 dot (src/mashbox/ops/__init__.py:574-576, 624-632). The caller rounds to the activation dtype (bf16).
    threads > 1 runs the row chunks concurrently (XLA:CPU runs the reference's program on all host cores)."""
    rows, cols = int(shape[-2]), int(shape[-1])
    rb = row_bytes(t, cols)
    raw = np.ascontiguousarray(raw, dtype=np.uint8).reshape(rows, rb)
    x = np.asarray(x, np.float32)
    rc = exact_chunk_rows(rows, cols, limit)
    out = np.empty(x.shape[:-1] + (rows,), np.float32)

    def chunk(a):
        w = dequant(raw[a:a + rc], t, cols)                   # (rc, cols) f32
        out[..., a:a + rc] = x @ w.T

    starts = range(0, rows, rc)
    if threads > 1 and len(starts) > 1:
        from concurrent.futures import ThreadPoolExecutor
        with ThreadPoolExecutor(min(threads, len(starts))) as ex:
            list(ex.map(chunk, starts))
    else:
        for a in starts:
            chunk(a)
    return out


def int8_linear(x_bf16: np.ndarray, q: np.ndarray, s: np.ndarray) -> np.ndarray:
    """(x_bf16 @ bf16(q).T with float32 accumulation) * s -> float32, before the rounding to bf16
    (src/mashbox/models/qwen3_8_27b/model.py:72-78). x_bf16: float32 values that are bfloat16-representable."""
    xq = np.asarray(x_bf16, np.float32)
    return (xq @ np.asarray(q, np.int8).astype(np.float32).T) * np.asarray(s, np.float32)


def int8_rows(w: np.ndarray):
    """symmetric int8, one float32 scale per output row (tests/cpu/qwen3_8_27b_checks.py:113-117)"""
    w32 = w.astype(np.float32)
    am = np.abs(w32).max(-1)
    s = np.where(am > 0, am / np.float32(127.0), np.float32(1.0)).astype(np.float32)
    return np.clip(np.round(w32 / s[:, None]), -127, 127).astype(np.int8), s


def int8_embed(q: np.ndarray, s: np.ndarray, toks) -> np.ndarray:
    """rows of toks of the int8 table (q (N, D), s (N,)) as float32 f32(q) * s, before the rounding to bfloat16
    (src/mashbox/models/qwen3_8_27b/model.py:132-139); ids index as jax.numpy: + N when negative, then clamped"""
    n = q.shape[0]
    t = np.asarray(toks, np.int64)
    t = np.clip(np.where(t < 0, t + n, t), 0, n - 1)
    return q[t].astype(np.float32) * np.asarray(s, np.float32)[t][..., None]
