"""Pins the CPU oracle (oracle/ref.py) before it is trusted as the parity checker. CPU only, no GPU.

Each check compares the oracle with something independent of its own formula, chosen so that a plausible slip fails:
  - fp16 decode: every one of the 65,536 bit patterns against a decoder written from the IEEE-754 binary16 definition
    (a wrong exponent bias, a lost subnormal or a NaN turned into inf fails);
  - Q8_0 / Q4_K block values: exact rational arithmetic (`fractions`) rounded once to float32 with integer
    arithmetic, on brute-force grids and random blocks (a dropped term, a wrong sign, a double rounding fails);
  - Q4_K layout: the scalar per-index form of the 6-bit scale/min unpack and the scalar dequant loop of llama.cpp's
    ggml-quants.c (get_scale_min_k4, dequantize_row_q4_K; the published algorithm gguf-py 0.19.0 restates in vector
    form and reference src/mashbox/ops/reference.py:132-149 follows) on random bytes (a nibble order, a sub-block
    grouping or a scale/min swap fails);
  - Q4_0: the scalar loop of llama.cpp's dequantize_row_q4_0 per index and the exact closed form over every code (a
    nibble-half swap or a dropped -8 fails), edge blocks;
  - Q5_K: the scalar loop of llama.cpp's dequantize_row_q5_K per index, in exact rationals rounded once (a high bit
    taken from the wrong qh bit or nibble half fails), random and edge blocks, real llama-quantize Q5_K blocks;
  - Q6_K: the scalar loop of llama.cpp's dequantize_row_q6_K per index, in exact rationals rounded once (a swapped
    nibble, a wrong 2-bit shift, a scale index off by a sub-block or a missing -32 fails), random blocks, edge blocks
    and every real llama-quantize Q6_K block of the golden fixtures;
  - the 6-bit packer: round trip over all 64 x 64 (scale, min) pairs in all 8 slots;
  - bf16 rounding: torch's own float32 -> bfloat16 cast on ties, NaN, inf, subnormals and random values;
  - exact product: the float64 product and the reference's float32 bars (reference tests/contracts/test_ops.py:19-35:
    NMSE <= 1e-8 and the gamma_K dot bound), chunked == whole;
  - exact_chunk_rows: a brute-force search of the definition (reference src/mashbox/ops/__init__.py:558-571) and the
    chunk counts of the BASELINE shapes;
  - the committed golden fixtures under tests/golden (random and real llama-quantize blocks).
"""
import os
from fractions import Fraction

import numpy as np
import pytest

from oracle import gen as G
from oracle import ref as R
from tests._check import diff_bits

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


# --------------------------------------------------------------------------------------------- exact float helpers
def f16_from_definition(h: int) -> float:
    """IEEE-754 binary16: 1 sign bit, 5 exponent bits (bias 15), 10 fraction bits; float('nan') for NaN"""
    s, e, f = (h >> 15) & 1, (h >> 10) & 31, h & 1023
    sign = -1.0 if s else 1.0
    if e == 31:
        return float("nan") if f else sign * float("inf")
    if e == 0:
        return sign * f * 2.0 ** -24
    return sign * (1024 + f) * 2.0 ** (e - 25)


def f32_round(v: Fraction, zero: float = 0.0) -> np.float32:
    """the float32 nearest to the rational v (ties to even), by integer arithmetic: rounded exactly once. An exact zero
    takes the sign IEEE-754 gives it, passed in as `zero` (+0.0 or -0.0): a rational has no signed zero"""
    if v == 0:
        return np.float32(zero)
    sign = -1 if v < 0 else 1
    a = abs(v)
    e = a.numerator.bit_length() - a.denominator.bit_length()       # 2^e <= a < 2^(e+2)
    while Fraction(2) ** e > a:
        e -= 1
    while Fraction(2) ** (e + 1) <= a:
        e += 1
    e = max(e, -126)                                                 # subnormal range keeps the quantum 2^-149
    q = Fraction(2) ** (e - 23)                                      # the spacing of float32 values at a
    n = a / q
    lo = n.numerator // n.denominator
    rem = n - lo
    if rem > Fraction(1, 2) or (rem == Fraction(1, 2) and lo % 2 == 1):
        lo += 1
    out = float(lo) * float(q)                                       # exact: lo <= 2^24 and q a power of two
    return np.float32(sign * out)


def f16_bytes(vals) -> np.ndarray:
    return np.asarray(vals, np.float16).view(np.uint8)


# ----------------------------------------------------------------------------------------------------- fp16 / bf16
def test_f16_decode_every_bit_pattern():
    h = np.arange(65536, dtype=np.uint32)
    b = np.stack([h & 0xFF, h >> 8], -1).astype(np.uint8).reshape(-1)
    got = R.f16_to_f32(b)
    want = np.array([f16_from_definition(int(v)) for v in h], np.float32)
    assert diff_bits(got, want) == 0
    assert np.sum(np.isnan(got)) == 2 * 1023                          # every NaN pattern stays NaN
    assert got[1] == np.float32(2.0 ** -24)                           # smallest subnormal survives


def test_bf16_round_matches_torch():
    torch = pytest.importorskip("torch")
    rng = np.random.default_rng(5)
    u = np.concatenate([
        rng.integers(0, 2 ** 32, 200_000, dtype=np.uint64).astype(np.uint32),
        np.array([0x3F808000, 0x3F818000, 0x3F80C000, 0x7F7FFFFF, 0x7F800000, 0xFF800000, 0x00000001, 0x80008000,
                  0x7FC00000, 0x7F800001, 0x33800000, 0x3F807FFF], np.uint32),                 # ties, extremes
    ])
    f = u.view(np.float32)
    want = torch.from_numpy(f.copy()).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    got = R.bf16_round(f)
    nan = np.isnan(f)
    assert np.array_equal(got[~nan], want[~nan])
    assert np.all(np.isnan(R.bf16_to_f32(got[nan])))


# ------------------------------------------------------------------------------------------------------------- Q8_0
def test_q8_0_is_the_exact_product():
    """v = q * d exactly, for every int8 code and a grid of fp16 scales spanning subnormal to max"""
    ds = np.concatenate([[2.0 ** -24, 2.0 ** -14 - 2.0 ** -24, 6.1e-5, 1e-3, 0.0078, 1.0, 3.14, 65504.0],
                         np.random.default_rng(0).uniform(1e-3, 1e-2, 24)]).astype(np.float16)
    ds = np.concatenate([ds, -ds])
    q = np.arange(-128, 128, dtype=np.int16).astype(np.int8).reshape(8, 32)
    blocks = []
    for d in ds:
        for row in q:
            blocks.append(np.concatenate([f16_bytes([d]), row.view(np.uint8)]))
    raw = np.stack(blocks)
    got = R.dequant(raw, R.Q8_0, 32)
    for i, (d, row) in enumerate(((d, row) for d in ds for row in q)):
        want = [f32_round(Fraction(int(c)) * Fraction(float(d)), np.float32(int(c)) * d) for c in row]
        assert diff_bits(got[i], np.array(want, np.float32)) == 0, (float(d), i)


def test_q8_0_edge_blocks():
    raw = np.zeros((3, 34), np.uint8)
    raw[1] = 0xFF                                   # d = NaN: every value NaN
    raw[2, :2] = f16_bytes([np.float16("inf")])     # d = inf: q * inf (q = 0 gives NaN)
    raw[2, 2:] = np.arange(32, dtype=np.int8).view(np.uint8)
    v = R.dequant(raw, R.Q8_0, 32)
    assert np.all(v[0] == 0) and not np.signbit(v[0]).any()
    assert np.all(np.isnan(v[1]))
    assert np.isnan(v[2, 0]) and np.all(np.isinf(v[2, 1:]))


# ------------------------------------------------------------------------------------------------------------- Q4_K
def ggml_scale_min_k4(j: int, q: bytes):
    """llama.cpp ggml-quants.c get_scale_min_k4, per index"""
    if j < 4:
        return q[j] & 63, q[j + 4] & 63
    return (q[j + 4] & 0xF) | ((q[j - 4] >> 6) << 4), (q[j + 4] >> 4) | ((q[j] >> 6) << 4)


def _zero(ds, q, dm):
    """sign of an exact-zero d*sc*q - dmin*m under IEEE-754 (both terms are exact float32 values)"""
    with np.errstate(all="ignore"):
        return np.float32(float(ds)) * np.float32(q) - np.float32(float(dm))


def ggml_q4_k_row(block: bytes):
    """llama.cpp dequantize_row_q4_K for one super-block, in exact rationals rounded once per value"""
    d = Fraction(f16_from_definition(block[0] | block[1] << 8))
    mn = Fraction(f16_from_definition(block[2] | block[3] << 8))
    scales, q = block[4:16], block[16:144]
    out, is_, qo = [], 0, 0
    for _ in range(0, 256, 64):
        sc, m = ggml_scale_min_k4(is_, scales)
        d1, m1 = d * sc, mn * m
        sc, m = ggml_scale_min_k4(is_ + 1, scales)
        d2, m2 = d * sc, mn * m
        out += [f32_round(d1 * (q[qo + l] & 0xF) - m1, _zero(d1, q[qo + l] & 0xF, m1)) for l in range(32)]
        out += [f32_round(d2 * (q[qo + l] >> 4) - m2, _zero(d2, q[qo + l] >> 4, m2)) for l in range(32)]
        qo += 32
        is_ += 2
    return np.array(out, np.float32)


def test_scale_min_k4_matches_the_scalar_form():
    rng = np.random.default_rng(11)
    s = rng.integers(0, 256, (500, 12), dtype=np.uint8)
    sc, mn = R.scale_min_k4(s)
    for i in range(s.shape[0]):
        for j in range(8):
            assert (int(sc[i, j]), int(mn[i, j])) == ggml_scale_min_k4(j, bytes(s[i])), (i, j)


def test_pack_scale_min_k4_round_trips_every_value():
    a = np.arange(64, dtype=np.uint8)
    sc_all, mn_all = np.meshgrid(a, a, indexing="ij")
    sc_all, mn_all = sc_all.reshape(-1), mn_all.reshape(-1)                  # 4096 pairs
    for slot in range(8):
        sc = np.zeros((4096, 8), np.uint8)
        mn = np.zeros((4096, 8), np.uint8)
        sc[:, slot], mn[:, slot] = sc_all, mn_all
        sc[:, (slot + 3) % 8], mn[:, (slot + 5) % 8] = sc_all[::-1], mn_all[::-1]   # neighbours must not bleed
        s2, m2 = R.scale_min_k4(R.pack_scale_min_k4(sc, mn))
        assert np.array_equal(s2, sc) and np.array_equal(m2, mn), slot


def test_q4_k_matches_the_scalar_loop_on_random_blocks():
    """random finite blocks: every scale, min, code and subnormal scale; one rounding per value"""
    rng = np.random.default_rng(12)
    raw = rng.integers(0, 256, (24, 144), dtype=np.uint8)
    d = rng.choice(np.array([2.0 ** -24, 3e-5, 1e-3, 0.5, 7.0, 65504.0, -2.5], np.float16), (24, 2))
    raw[:, 0:4] = d.view(np.uint8).reshape(24, 4)
    got = R.dequant(raw, R.Q4_K, 256)
    for i in range(raw.shape[0]):
        assert diff_bits(got[i], ggml_q4_k_row(bytes(raw[i]))) == 0, i


def test_q4_k_edge_blocks():
    raw = np.zeros((3, 144), np.uint8)
    raw[1] = 0xFF                                          # d = dmin = NaN
    raw[2, 2:4] = f16_bytes([np.float16(0.25)])            # d = 0: value = -dmin * m
    raw[2, 4:16] = R.pack_scale_min_k4(np.full((1, 8), 5, np.uint8), np.arange(8, dtype=np.uint8)[None] * 9)[0]
    v = R.dequant(raw, R.Q4_K, 256)
    assert np.all(v[0] == 0)
    assert np.all(np.isnan(v[1]))
    want = -0.25 * np.repeat(np.arange(8) * 9.0, 32)
    assert np.array_equal(v[2], want.astype(np.float32))


# ------------------------------------------------------------------------------------------------------------- Q4_0
def ggml_q4_0_row(block: bytes):
    """llama.cpp dequantize_row_q4_0 for one block (fp16 d, qs[16]), per index; an exact zero takes the sign float32
    x0 * d gives it"""
    d = f16_from_definition(block[0] | block[1] << 8)
    y = [None] * 32
    for j in range(16):
        x0, x1 = (block[2 + j] & 0x0F) - 8, (block[2 + j] >> 4) - 8
        for idx, xv in ((j, x0), (j + 16, x1)):
            with np.errstate(all="ignore"):
                zero = np.float32(xv) * np.float32(d)
            y[idx] = f32_round(Fraction(d) * xv, zero)
    return np.array(y, np.float32)


def test_q4_0_matches_the_scalar_loop_on_random_blocks():
    rng = np.random.default_rng(16)
    raw = rng.integers(0, 256, (40, 18), dtype=np.uint8)
    d = rng.choice(np.array([2.0 ** -24, 3e-5, 1e-3, 0.5, 7.0, 65504.0, -2.5, 0.0, -0.0], np.float16), 40)
    raw[:, 0:2] = d.view(np.uint8).reshape(40, 2)
    got = R.dequant(raw, R.Q4_0, 32)
    for i in range(raw.shape[0]):
        assert diff_bits(got[i], ggml_q4_0_row(bytes(raw[i]))) == 0, i


def test_q4_0_closed_form_and_edge_blocks():
    for dv in (np.float16(65504.0), np.float16(-1.0009765625), np.float16(2.0 ** -24), np.float16(-0.0999)):
        raw = np.zeros((16, 18), np.uint8)
        raw[:, 0:2] = np.array([dv], np.float16).view(np.uint8)
        raw[:, 2:] = (np.arange(16, dtype=np.uint8) * 17)[:, None]        # code c in both nibbles of every byte
        v = R.dequant(raw, R.Q4_0, 32)
        for c in range(16):
            assert np.all(v[c] == np.float32(Fraction(float(dv)) * (c - 8)))
        assert np.all(np.signbit(v[8]) == np.signbit(np.float32(dv)))    # d * (+0) keeps the sign of d
    raw = np.zeros((2, 18), np.uint8)
    raw[1] = 0xFF
    v = R.dequant(raw, R.Q4_0, 32)
    assert np.all(v[0] == 0) and np.all(np.isnan(v[1]))


# ------------------------------------------------------------------------------------------------------------- Q5_K
def ggml_q5_k_row(block: bytes):
    """llama.cpp dequantize_row_q5_K for one super-block (d, dmin, scales[12], qh[32], qs[128]), per index, in exact
    rationals rounded once per value"""
    d = Fraction(f16_from_definition(block[0] | block[1] << 8))
    mn = Fraction(f16_from_definition(block[2] | block[3] << 8))
    scales, qh, ql = block[4:16], block[16:48], block[48:176]
    out, is_, qo, u1, u2 = [], 0, 0, 1, 2
    for _ in range(0, 256, 64):
        sc, m = ggml_scale_min_k4(is_, scales)
        d1, m1 = d * sc, mn * m
        sc, m = ggml_scale_min_k4(is_ + 1, scales)
        d2, m2 = d * sc, mn * m
        for l in range(32):
            q = (ql[qo + l] & 0xF) + (16 if qh[l] & u1 else 0)
            out.append(f32_round(d1 * q - m1, _zero(d1, q, m1)))
        for l in range(32):
            q = (ql[qo + l] >> 4) + (16 if qh[l] & u2 else 0)
            out.append(f32_round(d2 * q - m2, _zero(d2, q, m2)))
        qo += 32
        is_ += 2
        u1 <<= 2
        u2 <<= 2
    return np.array(out, np.float32)


def test_q5_k_matches_the_scalar_loop_on_random_blocks():
    """random finite blocks: every scale, min, code, high bit and subnormal scale; one rounding per value"""
    rng = np.random.default_rng(15)
    raw = rng.integers(0, 256, (24, 176), dtype=np.uint8)
    d = rng.choice(np.array([2.0 ** -24, 3e-5, 1e-3, 0.5, 7.0, 65504.0, -2.5, 0.0], np.float16), (24, 2))
    raw[:, 0:4] = d.view(np.uint8).reshape(24, 4)
    got = R.dequant(raw, R.Q5_K, 256)
    for i in range(raw.shape[0]):
        assert diff_bits(got[i], ggml_q5_k_row(bytes(raw[i]))) == 0, i


def test_q5_k_edge_blocks():
    raw = np.zeros((3, 176), np.uint8)
    raw[1] = 0xFF                                          # d = dmin = NaN
    raw[2, 0:2] = f16_bytes([np.float16(0.5)])             # d = 0.5, dmin = 0
    raw[2, 4:16] = R.pack_scale_min_k4(np.arange(1, 9, dtype=np.uint8)[None], np.zeros((1, 8), np.uint8))[0]
    raw[2, 16:48] = 0b10100101                             # high bits of sub-blocks 0, 2, 5, 7
    raw[2, 48:176] = 0x73                                  # low nibbles 3 (even sub-blocks) and 7 (odd)
    v = R.dequant(raw, R.Q5_K, 256)
    assert np.all(v[0] == 0)
    assert np.all(np.isnan(v[1]))
    j = np.arange(256) // 32
    q = np.where(j % 2 == 0, 3, 7) + 16 * ((0b10100101 >> j) & 1)
    assert np.array_equal(v[2], (0.5 * (j + 1) * q).astype(np.float32))


# ------------------------------------------------------------------------------------------------------------- Q6_K
def ggml_q6_k_row(block: bytes):
    """llama.cpp dequantize_row_q6_K for one super-block (ql[128], qh[64], int8 scales[16], fp16 d), per index, in exact
    rationals rounded once per value; an exact zero takes the sign float32 (d * sc) * q gives it"""
    d = f16_from_definition(block[208] | block[209] << 8)
    ql, qh = block[0:128], block[128:192]
    sc = np.frombuffer(block[192:208], np.int8)
    y = [None] * 256
    for h in range(2):                                   # n = 0, 128
        for l in range(32):
            is_ = l // 16
            q = [(ql[64 * h + l] & 0xF) | (((qh[32 * h + l] >> 0) & 3) << 4),
                 (ql[64 * h + l + 32] & 0xF) | (((qh[32 * h + l] >> 2) & 3) << 4),
                 (ql[64 * h + l] >> 4) | (((qh[32 * h + l] >> 4) & 3) << 4),
                 (ql[64 * h + l + 32] >> 4) | (((qh[32 * h + l] >> 6) & 3) << 4)]
            for r in range(4):
                s = int(sc[8 * h + is_ + 2 * r])
                qv = q[r] - 32
                with np.errstate(all="ignore"):
                    zero = (np.float32(d) * np.float32(s)) * np.float32(qv)
                y[128 * h + 32 * r + l] = f32_round(Fraction(d) * s * qv, zero)
    return np.array(y, np.float32)


def test_q6_k_matches_the_scalar_loop_on_random_blocks():
    """random blocks with finite d (subnormal to the fp16 maximum, both signs): every code, scale and zero sign"""
    rng = np.random.default_rng(13)
    raw = rng.integers(0, 256, (24, 210), dtype=np.uint8)
    d = rng.choice(np.array([2.0 ** -24, 3e-5, 1e-3, 0.5, 7.0, 65504.0, -2.5, 0.0], np.float16), 24)
    raw[:, 208:210] = d.view(np.uint8).reshape(24, 2)
    raw[3, 192:208] = 0                                   # sc = 0: signed zeros
    got = R.dequant(raw, R.Q6_K, 256)
    for i in range(raw.shape[0]):
        assert diff_bits(got[i], ggml_q6_k_row(bytes(raw[i]))) == 0, i


def test_q6_k_closed_form_is_exact():
    """(d * sc) * (q - 32) has at most 11 + 7 + 5 significant bits: the float32 value is the exact product for every
    finite fp16 d, int8 sc and 6-bit q (brute force over sc and q at several d)"""
    for dv in (np.float16(65504.0), np.float16(-1.0009765625), np.float16(2.0 ** -24), np.float16(0.0999)):
        for s in range(-128, 128, 5):
            for q in range(64):
                exact = Fraction(float(dv)) * s * (q - 32)
                got = (np.float32(dv) * np.float32(s)) * np.float32(q - 32)
                assert Fraction(float(got)) == exact, (dv, s, q)


def test_q6_k_edge_blocks():
    raw = np.zeros((3, 210), np.uint8)
    raw[1] = 0xFF                                          # d = NaN
    raw[2, 208:210] = f16_bytes([np.float16(0.5)])
    raw[2, 192:208] = np.arange(-8, 8, dtype=np.int8).view(np.uint8)
    raw[2, 0:128] = 0x21                                   # every low nibble 1 or 2
    raw[2, 128:192] = 0b11100100                           # 2-bit highs 0, 1, 2, 3 for r = 0..3
    v = R.dequant(raw, R.Q6_K, 256)
    assert np.all(v[0] == 0) and np.all(np.signbit(v[0]))  # (0 * 0) * -32 = -0
    assert np.all(np.isnan(v[1]))
    idx = np.arange(256)
    r = (idx % 128) // 32
    low = np.where(r < 2, 1, 2)
    want = 0.5 * np.arange(-8, 8)[idx // 16] * (low + 16 * r - 32)
    assert np.array_equal(v[2], want.astype(np.float32))


def test_generators_make_blocks_of_the_stated_ranges():
    rng = np.random.default_rng(3)
    raw = G.q4_k_raw(rng, 16, 512)
    b = raw.reshape(-1, 144)
    d, dm = R.f16_to_f32(b[:, 0:2]), R.f16_to_f32(b[:, 2:4])
    assert np.all((d >= 9.9e-4) & (d <= 1.001e-2)) and np.all((dm >= 9.9e-4) & (dm <= 1.001e-2))
    sc, mn = R.scale_min_k4(b[:, 4:16])
    assert sc.max() <= 63 and mn.max() <= 63 and sc.max() > 50 and mn.min() < 10
    q8 = G.q8_0_raw(rng, 16, 512).reshape(-1, 34)
    qs = q8[:, 2:].view(np.int8)
    assert qs.min() >= -127 and qs.max() <= 127
    q6 = G.q6_k_raw(rng, 16, 512).reshape(-1, 210)
    d6, sc6 = R.f16_to_f32(q6[:, 208:210]), q6[:, 192:208].view(np.int8)
    assert np.all((d6 >= 9.9e-4 / 64) & (d6 <= 1.001e-2 / 64)) and sc6.min() >= -127 and sc6.max() <= 127
    ds6 = d6.repeat(16, 0) * sc6.reshape(-1, 1)
    w6 = R.dequant(q6, R.Q6_K, 256).reshape(-1, 16)[ds6[:, 0] != 0] / ds6[ds6[:, 0] != 0]
    assert w6.min() == -32 and w6.max() == 31 and np.array_equal(w6, np.round(w6))
    q5 = G.q5_k_raw(rng, 16, 512).reshape(-1, 176)
    d5 = R.f16_to_f32(q5[:, 0:2])
    assert np.all((d5 >= 9.9e-4 / 2) & (d5 <= 1.001e-2 / 2))
    sc5, mn5 = R.scale_min_k4(q5[:, 4:16])
    ok = (sc5 > 0).reshape(-1)
    w5 = (R.dequant(q5, R.Q5_K, 256).reshape(-1, 32) + (R.f16_to_f32(q5[:, 2:4]) * mn5).reshape(-1, 1))[ok] / \
        (d5 * sc5).reshape(-1, 1)[ok]
    w5 = np.round(w5)
    assert w5.min() == 0 and w5.max() == 31


# ------------------------------------------------------------------------------------------------- exact product
def test_exact_chunk_rows_is_the_largest_fitting_divisor():
    for rows in (1, 2, 7, 12, 36, 97, 128, 360):
        for cols in (1, 3, 10, 64):
            for limit in (1, 5, 64, 500, 4096):
                want = rows if rows * cols <= limit else max(
                    [c for c in range(1, rows + 1) if rows % c == 0 and c * cols <= limit] or [1])
                assert R.exact_chunk_rows(rows, cols, limit) == want, (rows, cols, limit)
    # chunk counts at the BASELINE shapes (rows per chunk, number of chunks)
    table = {(4096, 4096): 4096, (17408, 5120): 2176, (5120, 17408): 640, (6144, 5120): 3072, (1024, 5120): 1024,
             (5120, 6144): 2560}
    for (r, c), want in table.items():
        assert R.exact_chunk_rows(r, c) == want


@pytest.mark.parametrize("t", [R.Q4_0, R.Q8_0, R.Q4_K, R.Q5_K, R.Q6_K])
def test_exact_product_meets_the_float32_bars(t):
    """reference tests/contracts/test_ops.py:19-35: NMSE <= 1e-8 and |y - ref| <= gamma_K (|x| @ |W|.T)"""
    rng = np.random.default_rng(20 + t)
    n, k = 37, R.TYPES[t][1] * 4
    raw = G.RAW[t](rng, n, k)
    x = rng.standard_normal((5, k)).astype(np.float32)
    y = R.qmatmul_exact(x, raw, t, (n, k))
    w = R.dequant(raw, t, k).astype(np.float64)
    ref = x.astype(np.float64) @ w.T
    u = 2.0 ** -24
    gamma = k * u / (1 - k * u)
    assert np.all(np.abs(y - ref) <= gamma * (np.abs(x.astype(np.float64)) @ np.abs(w).T))
    assert float(np.sum((y - ref) ** 2) / np.sum(ref ** 2)) <= 1e-8
    # chunked rebuild (rows at a time) gives the same values as the whole-weight product, within the same bound
    yc = R.qmatmul_exact(x, raw, t, (n, k), limit=k)          # one row per chunk
    assert np.all(np.abs(yc - ref) <= gamma * (np.abs(x.astype(np.float64)) @ np.abs(w).T))
    yt = R.qmatmul_exact(x, raw, t, (n, k), limit=k, threads=4)
    assert np.array_equal(yt, yc)


def test_int8_linear_is_the_scaled_product():
    rng = np.random.default_rng(30)
    x = R.as_bf16(rng.standard_normal((3, 96)).astype(np.float32))
    q, s = G.int8_weights(rng, 11, 96)
    y = R.int8_linear(x, q, s)
    ref = (x.astype(np.float64) @ q.astype(np.float64).T) * s.astype(np.float64)
    u = 2.0 ** -24
    gamma = 97 * u / (1 - 97 * u)
    bound = gamma * (np.abs(x.astype(np.float64)) @ np.abs(q.astype(np.float64)).T) * s
    assert np.all(np.abs(y - ref) <= bound + np.abs(ref) * u)


def test_int8_rows_quantizer():
    """symmetric per-row int8 (reference tests/cpu/qwen3_8_27b_checks.py:113-117): q * s reproduces w within s / 2"""
    rng = np.random.default_rng(31)
    w = rng.standard_normal((6, 40)).astype(np.float32)
    w[2] = 0.0
    q, s = R.int8_rows(w)
    assert s[2] == 1.0 and np.all(q[2] == 0)
    assert np.all(np.abs(q.astype(np.float32) * s[:, None] - w) <= s[:, None] / 2 + 1e-7)
    assert np.all(np.abs(q).max(-1)[[0, 1, 3, 4, 5]] == 127)


# ------------------------------------------------------------------------------------------------- golden fixtures
def _golden():
    if not os.path.isdir(GOLDEN):
        return []
    return sorted(f for f in os.listdir(GOLDEN) if f.endswith(".npz"))


@pytest.mark.parametrize("name", _golden())
def test_oracle_reproduces_golden_fixture(name):
    z = np.load(os.path.join(GOLDEN, name), allow_pickle=False)
    t, cols = int(z["t"]), int(z["cols"])
    assert diff_bits(R.dequant(z["raw"], t, cols), z["w"]) == 0
    if "x" in z.files:
        y = R.qmatmul_exact(R.bf16_to_f32(z["x"]), z["raw"], t, (z["raw"].shape[0], cols))
        ref = z["y64"]
        assert float(np.sum((y - ref) ** 2) / np.sum(ref ** 2)) <= 1e-8


def test_golden_fixtures_are_present():
    names = _golden()
    assert any(n.startswith("random_") for n in names)
    assert any("kquant" in n for n in names)


def test_real_llama_quantize_blocks_match_the_scalar_forms():
    """real Q4_K / Q5_K / Q6_K / Q8_0 blocks from the reference's fixture models (via tests/golden): the oracle equals
    llama.cpp's scalar dequant loops (Q4_K, Q5_K, Q6_K) and the exact product (Q8_0) on every third block"""
    seen = set()
    for name in _golden():
        if not name.startswith("kquant_"):
            continue
        z = np.load(os.path.join(GOLDEN, name), allow_pickle=False)
        t, cols, raw = int(z["t"]), int(z["cols"]), z["raw"]
        if t not in (R.Q8_0, R.Q4_K, R.Q5_K, R.Q6_K):
            continue                                  # the exact path's other types: tests/test_oracle_types.py
        got = R.dequant(raw, t, cols)
        _, bs, ts = R.TYPES[t]
        blocks = raw.reshape(-1, ts)
        vals = got.reshape(-1, bs)
        for i in range(0, blocks.shape[0], 3):
            b = bytes(blocks[i])
            if t == R.Q4_K:
                want = ggml_q4_k_row(b)
            elif t == R.Q6_K:
                want = ggml_q6_k_row(b)
            elif t == R.Q5_K:
                want = ggml_q5_k_row(b)
            else:
                d = Fraction(f16_from_definition(b[0] | b[1] << 8))
                want = np.array([f32_round(Fraction(int(c)) * d, np.float32(int(c)) * np.float32(float(d)))
                             for c in np.frombuffer(b[2:], np.int8)], np.float32)
            assert diff_bits(vals[i], want) == 0, (name, i)
        seen.add(t)
    assert seen == {R.Q8_0, R.Q4_K, R.Q5_K, R.Q6_K}
