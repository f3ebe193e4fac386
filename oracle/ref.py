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
  the exact path's other types      src/mashbox/ops/reference.py:73-98 (Q4_1, Q5_0, Q5_1), :106-129 (Q2_K, Q3_K),
                                    :176-192 (TQ1_0, TQ2_0), :195-236 (MXFP4, NVFP4), :348-369 (IQ4_NL, IQ4_XS),
                                    :372-381 (F32, F16, BF16)
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
  the exact path's other types (tests/test_oracle_types.py)
                  Q4_1, Q5_0, Q5_1, Q2_K, Q3_K, IQ4_NL, IQ4_XS, TQ1_0, TQ2_0: per-index restatements of llama.cpp's
                  scalar loops (ggml-quants.c dequantize_row_*) in exact `fractions` arithmetic rounded once, on random
                  blocks, rows of several blocks and the real llama-quantize blocks of the reference's fixture files;
                  Q3_K's scales also through llama.cpp's kmask word shuffle; edge blocks.
                  MXFP4, NVFP4: k * 2^(e - 128) and E4M3(s) / 2 * k in exact rationals, k from the OCP E2M1 definition
                  doubled, on every exponent / scale byte and code. F16, BF16, F32: every pattern against the IEEE-754
                  definitions. The IQ4 code book: the published ggml table (no definition derives it).
  qmatmul_exact   against a float64 product (reference bars: tests/contracts/test_ops.py:22-31), and chunked == whole.
  int8_embed      against torch's own CPU float32 product and bfloat16 cast of the same gathered rows (an independent
                  implementation of the two IEEE-754 roundings), and the index rule against jax.numpy's documented one
                  (negative ids wrap once, the rest clamp) on every edge id.
  int8_linear     per element closed form: every bf16(x)*bf16(q) product is exact in float32; checked against a float64
                  product of the same values.
"""
from __future__ import annotations

import numpy as np

# ggml type id -> (name, values per block, bytes per block) (src/mashbox/ops/reference.py:22-29). The kernel path
# covers the first five, the types the reference's own kernel package gives planes (src/mashbox/ops/bundle.py:39); the
# exact path (dequant, qmatmul_exact) every type below. The reference's seven other types (IQ2_XXS, IQ2_XS, IQ2_S,
# IQ3_XXS, IQ3_S, IQ1_S, IQ1_M) decode through codebooks that gguf-py ships (reference.py:243-252), absent here.
TYPES = {2: ("Q4_0", 32, 18), 8: ("Q8_0", 32, 34), 12: ("Q4_K", 256, 144), 13: ("Q5_K", 256, 176), 14: ("Q6_K", 256, 210),
         0: ("F32", 1, 4), 1: ("F16", 1, 2), 30: ("BF16", 1, 2), 3: ("Q4_1", 32, 20), 6: ("Q5_0", 32, 22),
         7: ("Q5_1", 32, 24), 10: ("Q2_K", 256, 84), 11: ("Q3_K", 256, 110), 20: ("IQ4_NL", 32, 18),
         23: ("IQ4_XS", 256, 136), 34: ("TQ1_0", 256, 54), 35: ("TQ2_0", 256, 66), 39: ("MXFP4", 32, 17),
         40: ("NVFP4", 64, 36)}
Q4_0, Q8_0, Q4_K, Q5_K, Q6_K = 2, 8, 12, 13, 14
F32, F16, BF16, Q4_1, Q5_0, Q5_1, Q2_K, Q3_K, IQ4_NL, IQ4_XS, TQ1_0, TQ2_0, MXFP4, NVFP4 = (
    0, 1, 30, 3, 6, 7, 10, 11, 20, 23, 34, 35, 39, 40)
KERNEL_TYPES = (Q4_0, Q8_0, Q4_K, Q5_K, Q6_K)
EXACT_ONLY = (F32, F16, BF16, Q4_1, Q5_0, Q5_1, Q2_K, Q3_K, IQ4_NL, IQ4_XS, TQ1_0, TQ2_0, MXFP4, NVFP4)
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


def _u32(b: np.ndarray) -> np.ndarray:
    """(N, 4) little-endian bytes -> (N, 1) uint32"""
    b = b.astype(np.uint32)
    return (b[:, 0] | (b[:, 1] << 8) | (b[:, 2] << 16) | (b[:, 3] << 24)).reshape(-1, 1)


def _q5_high(qh4: np.ndarray) -> np.ndarray:
    """(N, 4) bytes of a 32-bit mask -> (N, 32) uint8: bit j for value j (src/mashbox/ops/reference.py:80-82)"""
    return ((_u32(qh4) >> np.arange(32, dtype=np.uint32)) & np.uint32(1)).astype(np.uint8)


def q4_1_blocks(b: np.ndarray) -> np.ndarray:
    """(N, 20) blocks -> (N, 32): d * q + m, d and m fp16 at bytes 0-3, q the nibbles of bytes 4-19 (low halves first)
    (src/mashbox/ops/reference.py:73-77)"""
    n = b.shape[0]
    d, m = f16_to_f32(b[:, 0:2]), f16_to_f32(b[:, 2:4])
    q = nib(b[:, 4:]).reshape(n, 32).astype(np.float32)
    return d * q + m


def q5_0_blocks(b: np.ndarray) -> np.ndarray:
    """(N, 22) blocks -> (N, 32): d * (q - 16), q = nibble | bit j of the 32-bit mask at bytes 2-5 << 4
    (src/mashbox/ops/reference.py:85-90)"""
    n = b.shape[0]
    d = f16_to_f32(b[:, 0:2])
    q = nib(b[:, 6:]).reshape(n, 32) | (_q5_high(b[:, 2:6]) << np.uint8(4))
    return d * (q.astype(np.int16) - 16).astype(np.float32)


def q5_1_blocks(b: np.ndarray) -> np.ndarray:
    """(N, 24) blocks -> (N, 32): d * q + m, q = nibble | mask bit << 4, mask at bytes 4-7
    (src/mashbox/ops/reference.py:93-98)"""
    n = b.shape[0]
    d, m = f16_to_f32(b[:, 0:2]), f16_to_f32(b[:, 2:4])
    q = nib(b[:, 8:]).reshape(n, 32) | (_q5_high(b[:, 4:8]) << np.uint8(4))
    return d * q.astype(np.float32) + m


_SHIFT2 = np.array([0, 2, 4, 6], np.uint8).reshape(1, 1, 4, 1)


def _two_bit(qs: np.ndarray) -> np.ndarray:
    """(N, 64) bytes -> (N, 256) 2-bit codes: value 128 h + 32 s + i = bits 2s, 2s+1 of byte 32 h + i"""
    n = qs.shape[0]
    return ((qs.reshape(n, 2, 1, 32) >> _SHIFT2) & np.uint8(3)).reshape(n, 256)


def q2_k_blocks(b: np.ndarray) -> np.ndarray:
    """(N, 84) super-blocks -> (N, 256): (d * (sc & 15)) * q - dmin * (sc >> 4) over 16 sub-blocks of 16; scales at
    bytes 0-15, codes 16-79, d 80-81, dmin 82-83 (src/mashbox/ops/reference.py:106-114)"""
    n = b.shape[0]
    sc = b[:, :16]
    d, dmin = f16_to_f32(b[:, 80:82]), f16_to_f32(b[:, 82:84])
    dl = (d * (sc & np.uint8(15)).astype(np.float32)).reshape(n, 16, 1)
    ml = (dmin * (sc >> np.uint8(4)).astype(np.float32)).reshape(n, 16, 1)
    q = _two_bit(b[:, 16:80]).reshape(n, 16, 16).astype(np.float32)
    return (dl * q - ml).reshape(n, QK_K)


def q3_k_scales(sc: np.ndarray) -> np.ndarray:
    """(N, 12) bytes -> (N, 16) signed 6-bit scales: low 4 bits from the nibbles of bytes 0-7 (low halves, then high
    halves), high 2 bits from the 2-bit fields of bytes 8-11 (src/mashbox/ops/reference.py:120-123)"""
    n = sc.shape[0]
    lo = (sc[:, :8].reshape(n, 1, 8) >> np.array([0, 4], np.uint8).reshape(1, 2, 1)).reshape(n, 16) & np.uint8(15)
    hi = (sc[:, 8:].reshape(n, 1, 4) >> np.array([0, 2, 4, 6], np.uint8).reshape(1, 4, 1)).reshape(n, 16) & np.uint8(3)
    return (lo | (hi << np.uint8(4))).astype(np.int16) - 32


def q3_k_blocks(b: np.ndarray) -> np.ndarray:
    """(N, 110) super-blocks -> (N, 256): (d * s) * (q - 4 (1 - h)) over 16 sub-blocks of 16; high-bit mask at bytes
    0-31 (value 32 j + i: bit j of byte i), codes 32-95, scales 96-107, d 108-109 (src/mashbox/ops/reference.py:117-129)"""
    n = b.shape[0]
    d = f16_to_f32(b[:, 108:110])
    dl = (d * q3_k_scales(b[:, 96:108]).astype(np.float32)).reshape(n, 16, 1)
    ql = _two_bit(b[:, 32:96]).astype(np.int16)
    h = ((b[:, :32].reshape(n, 1, 32) >> np.arange(8, dtype=np.uint8).reshape(1, 8, 1)) & np.uint8(1)).reshape(n, 256)
    q = (ql - 4 * (h ^ np.uint8(1)).astype(np.int16)).astype(np.float32).reshape(n, 16, 16)
    return (dl * q).reshape(n, QK_K)


# the IQ4_NL / IQ4_XS code book (src/mashbox/ops/reference.py:348; ggml's kvalues_iq4nl)
KV_IQ4 = np.array([-127, -104, -83, -65, -49, -35, -22, -10, 1, 13, 25, 38, 53, 69, 89, 113], np.float32)


def iq4_nl_blocks(b: np.ndarray) -> np.ndarray:
    """(N, 18) blocks -> (N, 32): d * KV_IQ4[q], q the nibbles of bytes 2-17 (src/mashbox/ops/reference.py:351-356)"""
    n = b.shape[0]
    d = f16_to_f32(b[:, 0:2])
    return d * KV_IQ4[nib(b[:, 2:]).reshape(n, 32)]


def iq4_xs_blocks(b: np.ndarray) -> np.ndarray:
    """(N, 136) super-blocks -> (N, 256): (d * (s - 32)) * KV_IQ4[q] over 8 sub-blocks of 32; the 6-bit s of sub-block
    j = nibble j % 2 of byte 4 + j // 2 | bits 2j, 2j+1 of the 16-bit word at bytes 2-3 << 4; codes at bytes 8-135,
    16 per sub-block (src/mashbox/ops/reference.py:359-369)"""
    n = b.shape[0]
    d = f16_to_f32(b[:, 0:2])
    lo = (b[:, 4:8].reshape(n, 4, 1) >> np.array([0, 4], np.uint8).reshape(1, 1, 2)).reshape(n, 8) & np.uint8(15)
    hw = (b[:, 2].astype(np.uint16) | (b[:, 3].astype(np.uint16) << np.uint16(8))).reshape(n, 1)
    hi = ((hw >> (2 * np.arange(8, dtype=np.uint16))) & np.uint16(3)).astype(np.uint8)
    s = (lo | (hi << np.uint8(4))).astype(np.int16) - 32
    dl = (d * s.astype(np.float32)).reshape(n, 8, 1)
    q = nib(b[:, 8:].reshape(n, 8, 16)).reshape(n, 8, 32)
    return (dl * KV_IQ4[q]).reshape(n, QK_K)


_POW3 = np.array([1, 3, 9, 27, 81], np.uint8)


def tq1_0_blocks(b: np.ndarray) -> np.ndarray:
    """(N, 54) super-blocks -> (N, 256): d * (t - 1), t = ((byte * 3^k mod 256) * 3) >> 8 for k = 0..4 over bytes 0-31
    (values 0-159), bytes 32-47 (160-239), k = 0..3 over bytes 48-51 (240-255); d at 52-53
    (src/mashbox/ops/reference.py:176-185)"""
    n = b.shape[0]
    d = f16_to_f32(b[:, 52:54])
    q0 = (b[:, :32].reshape(n, 1, 32) * _POW3.reshape(1, 5, 1)).reshape(n, 160)
    q1 = (b[:, 32:48].reshape(n, 1, 16) * _POW3.reshape(1, 5, 1)).reshape(n, 80)
    q2 = (b[:, 48:52].reshape(n, 1, 4) * _POW3[:4].reshape(1, 4, 1)).reshape(n, 16)
    q = np.concatenate([q0, q1, q2], -1).astype(np.uint16)               # uint8 products: taken mod 256
    t = ((q * np.uint16(3)) >> np.uint16(8)).astype(np.int16) - 1
    return d * t.astype(np.float32)


def tq2_0_blocks(b: np.ndarray) -> np.ndarray:
    """(N, 66) super-blocks -> (N, 256): d * (q - 1), q the 2-bit codes of bytes 0-63 (as Q2_K's), d at 64-65
    (src/mashbox/ops/reference.py:188-192)"""
    d = f16_to_f32(b[:, 64:66])
    return d * (_two_bit(b[:, :64]).astype(np.int16) - 1).astype(np.float32)


# the FP4 (E2M1) values doubled, as ggml's kvalues_mxfp4 (src/mashbox/ops/reference.py:195)
KV_FP4 = np.array([0, 1, 2, 3, 4, 6, 8, 12, 0, -1, -2, -3, -4, -6, -8, -12], np.int32)


def mxfp4_blocks(b: np.ndarray) -> np.ndarray:
    """(N, 17) blocks -> (N, 32): KV_FP4[q] * 2^(e - 128), e the byte 0, q the nibbles of bytes 1-16, with the float32
    bits built from integers (subnormal results exact, overflow to inf, zero codes +0) (src/mashbox/ops/reference.py:198-219)"""
    n = b.shape[0]
    e = b[:, :1].astype(np.int64)
    q = nib(b[:, 1:]).reshape(n, 32).astype(np.int64)
    odd = np.array([0, 1, 1, 3, 1, 3, 1, 3] * 2, np.int64)[q]
    p = np.array([0, 0, 1, 0, 2, 1, 3, 2] * 2, np.int64)[q]
    x = p + e - 128                                                       # |value| = odd * 2^x
    E = np.where(odd == 3, x + 1, x)
    normal = ((E + 127) << 23) | np.where(odd == 3, 1 << 22, 0)
    sub = odd << np.clip(x + 149, 0, 30)
    bits = np.where(E < -126, sub, normal)
    bits = np.where(E > 127, 0x7F800000, bits)
    bits = np.where(odd == 0, 0, bits)
    bits = bits | np.where((q >= 8) & (odd != 0), 0x80000000, 0)
    return bits.astype(np.uint32).view(np.float32)


def ue4m3_half(x: np.ndarray) -> np.ndarray:
    """unsigned E4M3 scale bytes -> float32 half values; bytes 0x00 and 0x7F give 0 (src/mashbox/ops/reference.py:222-227)"""
    e = ((x >> np.uint8(3)) & np.uint8(15)).astype(np.int32)
    man = (x & np.uint8(7)).astype(np.float32)
    p2 = ((e + 120).astype(np.uint32) << np.uint32(23)).view(np.float32)    # 2^(e - 7)
    raw = np.where(e == 0, man * np.float32(2.0 ** -9), (np.float32(1) + man / np.float32(8)) * p2)
    return np.where((x == 0) | (x == 0x7F), np.float32(0), raw * np.float32(0.5)).astype(np.float32)


def nvfp4_blocks(b: np.ndarray) -> np.ndarray:
    """(N, 36) blocks -> (N, 64): ue4m3_half(byte s) * KV_FP4[q] over 4 sub-blocks of 16; sub-block s's codes: low
    nibbles of bytes 4 + 8s .. 11 + 8s, then their high nibbles (src/mashbox/ops/reference.py:230-236)"""
    n = b.shape[0]
    d = ue4m3_half(b[:, :4]).reshape(n, 4, 1)
    q = nib(b[:, 4:].reshape(n, 4, 8)).reshape(n, 4, 16)
    return (d * KV_FP4[q].astype(np.float32)).reshape(n, 64)


def f32_values(b: np.ndarray) -> np.ndarray:
    """(N, 4k) little-endian bytes -> (N, k) float32, the bits as stored (src/mashbox/ops/reference.py:372-373)"""
    return np.ascontiguousarray(b).view("<u4").astype(np.uint32).view(np.float32)


def f16_values(b: np.ndarray) -> np.ndarray:
    """(N, 2k) -> (N, k): fp16 -> float32 (src/mashbox/ops/reference.py:376-377)"""
    return f16_to_f32(b)


def bf16_values(b: np.ndarray) -> np.ndarray:
    """(N, 2k) -> (N, k): bfloat16 bits << 16 (src/mashbox/ops/reference.py:380-381)"""
    b = np.ascontiguousarray(b, dtype=np.uint8)
    return bf16_to_f32(b[..., 0::2].astype(np.uint16) | (b[..., 1::2].astype(np.uint16) << np.uint16(8)))


BLOCKS = {Q4_0: q4_0_blocks, Q8_0: q8_0_blocks, Q4_K: q4_k_blocks, Q5_K: q5_k_blocks, Q6_K: q6_k_blocks,
          Q4_1: q4_1_blocks, Q5_0: q5_0_blocks, Q5_1: q5_1_blocks, Q2_K: q2_k_blocks, Q3_K: q3_k_blocks,
          IQ4_NL: iq4_nl_blocks, IQ4_XS: iq4_xs_blocks, TQ1_0: tq1_0_blocks, TQ2_0: tq2_0_blocks, MXFP4: mxfp4_blocks,
          NVFP4: nvfp4_blocks}
FLOATS = {F32: f32_values, F16: f16_values, BF16: bf16_values}


def dequant(raw: np.ndarray, t: int, cols: int) -> np.ndarray:
    """raw (..., row_bytes(t, cols)) uint8 -> (..., cols) float32, exact (src/mashbox/ops/reference.py:398-409); the
    float types convert whole rows, the block types one block at a time"""
    _, bs, ts = TYPES[t]
    raw = np.ascontiguousarray(raw, dtype=np.uint8)
    lead = raw.shape[:-1]
    with np.errstate(invalid="ignore", over="ignore"):
        out = FLOATS[t](raw.reshape(-1, raw.shape[-1])) if t in FLOATS else BLOCKS[t](raw.reshape(-1, ts))
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
