"""Pins the oracle's exact-path types beyond the five kernel types (oracle/ref.py: F32, F16, BF16, Q4_1, Q5_0, Q5_1,
Q2_K, Q3_K, IQ4_NL, IQ4_XS, TQ1_0, TQ2_0, MXFP4, NVFP4). CPU only, no GPU.

The reference dequantizes every ggml type (src/mashbox/ops/reference.py:22-29, 396-409) with gguf-py 0.19.0's
arithmetic (its own test: reference tests/cpu/test_gguf_dequant.py, bit for bit against gguf-py, absent here). Each
oracle function is checked against something written independently of its vector form, chosen so that a plausible
slip fails:
  - Q4_1, Q5_0, Q5_1, Q2_K, Q3_K, IQ4_NL, IQ4_XS, TQ1_0, TQ2_0: the scalar loops of llama.cpp's ggml-quants.c
    (dequantize_row_q4_1 ... dequantize_row_tq2_0; the published algorithm gguf-py restates), per index, in exact
    rationals rounded once to float32 with integer arithmetic. Q3_K's scales come through llama.cpp's kmask word
    shuffle, a different derivation from the oracle's per-sub-block fields; TQ1_0 through its base-3 loops over the
    byte runs, with the uint8 products wrapping as C's do;
  - MXFP4: k * 2^(e - 128) in exact rationals, k from the OCP MX E2M1 definition (sign, 2 exponent bits of bias 1,
    1 mantissa bit) doubled, rounded once (subnormal results and overflow included): the oracle builds the bits with
    integer shifts instead;
  - NVFP4: the E4M3 scale from its definition (bias 7, subnormals below exponent 1) halved, times the doubled E2M1
    value, in exact rationals;
  - F16 / BF16 / F32: every bit pattern decoded from the IEEE-754 definitions (binary16, bfloat16 = the top half of
    binary32, binary32 itself);
  - edge blocks (all zero bits, all one bits) and closed forms on every code;
  - real blocks from the reference's fixture models (tests/golden kquant_* fixtures of Q5_1, Q2_K, Q3_K, IQ4_NL,
    IQ4_XS made by llama-quantize).
The IQ4 code book (ggml's kvalues_iq4nl) has no definition to derive it from; the oracle's copy is checked against the
published table's known properties (16 increasing odd-spaced values, the same table the real IQ4 blocks dequantize
through to smooth weights).
"""
import os
import struct
from fractions import Fraction

import numpy as np
import pytest

from oracle import ref as R
from tests._check import diff_bits
from tests.test_oracle import GOLDEN, f16_from_definition, f32_round


def _f16(b, o):
    return f16_from_definition(b[o] | b[o + 1] << 8)


def _np_zero(*ops):
    """the IEEE-754 float32 result of a chain of operations, used only for the sign of an exact zero"""
    with np.errstate(all="ignore"):
        v = np.float32(ops[0])
        for op, a in zip(ops[1::2], ops[2::2]):
            v = v * np.float32(a) if op == "*" else v + np.float32(a) if op == "+" else v - np.float32(a)
        return v


def _rnd(v: Fraction, zero) -> np.float32:
    return f32_round(v, zero)


# ---------------------------------------------------------------------------------------------- scalar loops
def ggml_q4_1_row(b: bytes):
    """dequantize_row_q4_1: y[j] = x0 * d + m, y[j + 16] = x1 * d + m"""
    d, m = _f16(b, 0), _f16(b, 2)
    y = [None] * 32
    for j in range(16):
        for idx, x in ((j, b[4 + j] & 0x0F), (j + 16, b[4 + j] >> 4)):
            y[idx] = _rnd(Fraction(x) * Fraction(d) + Fraction(m), _np_zero(x, "*", d, "+", m))
    return np.array(y, np.float32)


def ggml_q5_0_row(b: bytes):
    """dequantize_row_q5_0: xh_0 = ((qh >> j) << 4) & 0x10, xh_1 = (qh >> (j + 12)) & 0x10, x = (nibble | xh) - 16"""
    d = _f16(b, 0)
    qh = struct.unpack("<I", bytes(b[2:6]))[0]
    y = [None] * 32
    for j in range(16):
        x0 = ((b[6 + j] & 0x0F) | (((qh >> j) << 4) & 0x10)) - 16
        x1 = ((b[6 + j] >> 4) | ((qh >> (j + 12)) & 0x10)) - 16
        for idx, x in ((j, x0), (j + 16, x1)):
            y[idx] = _rnd(Fraction(x) * Fraction(d), _np_zero(x, "*", d))
    return np.array(y, np.float32)


def ggml_q5_1_row(b: bytes):
    """dequantize_row_q5_1: as Q5_0 without the -16, plus m"""
    d, m = _f16(b, 0), _f16(b, 2)
    qh = struct.unpack("<I", bytes(b[4:8]))[0]
    y = [None] * 32
    for j in range(16):
        x0 = (b[8 + j] & 0x0F) | (((qh >> j) << 4) & 0x10)
        x1 = (b[8 + j] >> 4) | ((qh >> (j + 12)) & 0x10)
        for idx, x in ((j, x0), (j + 16, x1)):
            y[idx] = _rnd(Fraction(x) * Fraction(d) + Fraction(m), _np_zero(x, "*", d, "+", m))
    return np.array(y, np.float32)


def ggml_q2_k_row(b: bytes):
    """dequantize_row_q2_K: two halves of 128 values, four shifts each, two scale bytes per shift"""
    sc, q = b[0:16], b[16:80]
    d, mn = _f16(b, 80), _f16(b, 82)
    y, is_, qo = [], 0, 0
    for _ in range(2):
        shift = 0
        for _ in range(4):
            for half in (0, 16):
                s = sc[is_]
                is_ += 1
                dl, ml = Fraction(d) * (s & 0xF), Fraction(mn) * (s >> 4)
                fdl, fml = _np_zero(d, "*", s & 0xF), _np_zero(mn, "*", s >> 4)
                for l in range(16):
                    x = (q[qo + half + l] >> shift) & 3
                    y.append(_rnd(dl * x - ml, _np_zero(fdl, "*", x, "-", fml)))
            shift += 2
        qo += 32
    return np.array(y, np.float32)


def ggml_q3_k_scales(scb: bytes):
    """llama.cpp's scale unpack of dequantize_row_q3_K: three little-endian words shuffled with kmask1 / kmask2"""
    kmask1, kmask2 = 0x03030303, 0x0F0F0F0F
    aux = list(struct.unpack("<3I", bytes(scb))) + [0]
    tmp = aux[2]
    aux[2] = ((aux[0] >> 4) & kmask2) | (((tmp >> 4) & kmask1) << 4)
    aux[3] = ((aux[1] >> 4) & kmask2) | (((tmp >> 6) & kmask1) << 4)
    aux[0] = (aux[0] & kmask2) | (((tmp >> 0) & kmask1) << 4)
    aux[1] = (aux[1] & kmask2) | (((tmp >> 2) & kmask1) << 4)
    return [int(v) for v in np.frombuffer(struct.pack("<4I", *[a & 0xFFFFFFFF for a in aux]), np.int8)]


def ggml_q3_k_row(b: bytes):
    """dequantize_row_q3_K: the high-bit mask m moves one bit per shift; a clear bit subtracts 4"""
    hm, q = b[0:32], b[32:96]
    d = _f16(b, 108)
    scales = ggml_q3_k_scales(b[96:108])
    y, is_, m, qo = [], 0, 1, 0
    for _ in range(2):
        shift = 0
        for _ in range(4):
            for half in (0, 16):
                s = scales[is_] - 32
                is_ += 1
                dl, fdl = Fraction(d) * s, _np_zero(d, "*", s)
                for l in range(16):
                    x = ((q[qo + half + l] >> shift) & 3) - (0 if hm[half + l] & m else 4)
                    y.append(_rnd(dl * x, _np_zero(fdl, "*", x)))
            shift += 2
            m <<= 1
        qo += 32
    return np.array(y, np.float32)


KV_IQ4_PUBLISHED = (-127, -104, -83, -65, -49, -35, -22, -10, 1, 13, 25, 38, 53, 69, 89, 113)


def ggml_iq4_nl_row(b: bytes):
    """dequantize_row_iq4_nl: y[j] = d * kv[qs[j] & 0xf], y[j + 16] = d * kv[qs[j] >> 4]"""
    d = _f16(b, 0)
    y = [None] * 32
    for j in range(16):
        for idx, c in ((j, b[2 + j] & 0xF), (j + 16, b[2 + j] >> 4)):
            k = KV_IQ4_PUBLISHED[c]
            y[idx] = _rnd(Fraction(d) * k, _np_zero(d, "*", k))
    return np.array(y, np.float32)


def ggml_iq4_xs_row(b: bytes):
    """dequantize_row_iq4_xs: ls = ((scales_l[ib / 2] >> 4 (ib % 2)) & 0xf) | (((scales_h >> 2 ib) & 3) << 4)"""
    d = _f16(b, 0)
    sh = b[2] | b[3] << 8
    y = []
    for ib in range(8):
        ls = ((b[4 + ib // 2] >> 4 * (ib % 2)) & 0xF) | (((sh >> 2 * ib) & 3) << 4)
        dl, fdl = Fraction(d) * (ls - 32), _np_zero(d, "*", ls - 32)
        qs = b[8 + 16 * ib: 24 + 16 * ib]
        lo = [KV_IQ4_PUBLISHED[c & 0xF] for c in qs]
        hi = [KV_IQ4_PUBLISHED[c >> 4] for c in qs]
        y += [_rnd(dl * k, _np_zero(fdl, "*", k)) for k in lo + hi]
    return np.array(y, np.float32)


def ggml_tq1_0_row(b: bytes):
    """dequantize_row_tq1_0: base-3 digits by uint8 products with 1, 3, 9, 27, 81 (wrapping), ((q * 3) >> 8) - 1"""
    pow3 = (1, 3, 9, 27, 81, 243)
    d = _f16(b, 52)
    qs, qh = b[0:48], b[48:52]
    codes = []
    for n in range(5):
        codes += [(qs[m] * pow3[n]) & 0xFF for m in range(32)]
    for n in range(5):
        codes += [(qs[32 + m] * pow3[n]) & 0xFF for m in range(16)]
    for n in range(4):
        codes += [(qh[j] * pow3[n]) & 0xFF for j in range(4)]
    return np.array([_rnd(Fraction((((c * 3) >> 8) - 1)) * Fraction(d), _np_zero((((c * 3) >> 8) - 1), "*", d))
                     for c in codes], np.float32)


def ggml_tq2_0_row(b: bytes):
    """dequantize_row_tq2_0: for each run of 32 bytes, four 2-bit fields, (q - 1) * d"""
    d = _f16(b, 64)
    y = []
    for j in (0, 32):
        for l in range(4):
            for m in range(32):
                x = ((b[j + m] >> (2 * l)) & 3) - 1
                y.append(_rnd(Fraction(x) * Fraction(d), _np_zero(x, "*", d)))
    return np.array(y, np.float32)


def e2m1(code: int) -> Fraction:
    """OCP MX E2M1: sign bit 3, exponent bits 1-2 (bias 1), mantissa bit 0; exponent 0 is subnormal (m * 0.5)"""
    s, e, m = (code >> 3) & 1, (code >> 1) & 3, code & 1
    v = Fraction(m, 2) if e == 0 else (1 + Fraction(m, 2)) * Fraction(2) ** (e - 1)
    return -v if s else v


def mxfp4_row(b: bytes):
    """k * 2^(e - 128) with k = 2 * E2M1(code), exact, rounded once (a zero code gives +0)"""
    e = b[0]
    codes = [c & 0xF for c in b[1:17]] + [c >> 4 for c in b[1:17]]
    return np.array([f32_round(2 * e2m1(c) * Fraction(2) ** (e - 128), 0.0) for c in codes], np.float32)


def e4m3_unsigned(x: int) -> Fraction:
    """the NVFP4 block scale: E4M3 of the byte's low 7 bits (bias 7; exponent 0: m * 2^-9), the codes 0x00 and 0x7F
    read as 0"""
    if x in (0x00, 0x7F):
        return Fraction(0)
    e, m = (x >> 3) & 15, x & 7
    return Fraction(m, 512) if e == 0 else Fraction(8 + m) * Fraction(2) ** (e - 10)


def nvfp4_row(b: bytes):
    """4 sub-blocks of 16: E4M3(scale s) / 2 * 2 * E2M1(code)"""
    y = []
    for s in range(4):
        d = e4m3_unsigned(b[s]) / 2
        qs = b[4 + 8 * s: 12 + 8 * s]
        y += [f32_round(d * 2 * e2m1(c), _np_zero(float(d), "*", float(2 * e2m1(c))))      # 0 * -k is -0
              for c in [c & 0xF for c in qs] + [c >> 4 for c in qs]]
    return np.array(y, np.float32)


SCALAR = {R.Q4_1: ggml_q4_1_row, R.Q5_0: ggml_q5_0_row, R.Q5_1: ggml_q5_1_row, R.Q2_K: ggml_q2_k_row,
          R.Q3_K: ggml_q3_k_row, R.IQ4_NL: ggml_iq4_nl_row, R.IQ4_XS: ggml_iq4_xs_row, R.TQ1_0: ggml_tq1_0_row,
          R.TQ2_0: ggml_tq2_0_row, R.MXFP4: mxfp4_row, R.NVFP4: nvfp4_row}
# byte offsets of each block type's fp16 scales (kept finite in the random-block checks)
F16_AT = {R.Q4_1: (0, 2), R.Q5_0: (0,), R.Q5_1: (0, 2), R.Q2_K: (80, 82), R.Q3_K: (108,), R.IQ4_NL: (0,),
          R.IQ4_XS: (0,), R.TQ1_0: (52,), R.TQ2_0: (64,), R.MXFP4: (), R.NVFP4: ()}
NAME = {t: R.TYPES[t][0] for t in R.TYPES}


def random_blocks(t: int, n: int, seed: int) -> np.ndarray:
    """n random blocks of type t whose fp16 scales are finite (subnormal, negative and signed zeros included)"""
    rng = np.random.default_rng(seed)
    ts = R.TYPES[t][2]
    raw = rng.integers(0, 256, (n, ts), dtype=np.uint8)
    pool = np.array([2.0 ** -24, 3e-5, 1e-3, 0.5, 7.0, 65504.0, -2.5, 0.0, -0.0, -1.0009765625], np.float16)
    for o in F16_AT[t]:
        raw[:, o:o + 2] = rng.choice(pool, n).view(np.uint8).reshape(n, 2)
    return raw


@pytest.mark.parametrize("t", sorted(SCALAR), ids=NAME.get)
def test_block_types_match_the_scalar_loops_on_random_blocks(t):
    raw = random_blocks(t, 48, 300 + t)
    bs = R.TYPES[t][1]
    got = R.dequant(raw, t, bs)
    for i in range(raw.shape[0]):
        assert diff_bits(got[i], SCALAR[t](bytes(raw[i]))) == 0, (NAME[t], i)


@pytest.mark.parametrize("t", sorted(SCALAR), ids=NAME.get)
def test_rows_of_several_blocks_keep_block_order(t):
    """a row of 5 blocks dequantizes block by block, in order (a block stride or a row reshape slip fails)"""
    raw = random_blocks(t, 15, 400 + t).reshape(3, -1)
    bs = R.TYPES[t][1]
    got = R.dequant(raw, t, 5 * bs)
    for r in range(3):
        for k in range(5):
            blk = bytes(raw[r, k * R.TYPES[t][2]:(k + 1) * R.TYPES[t][2]])
            assert diff_bits(got[r, k * bs:(k + 1) * bs], SCALAR[t](blk)) == 0, (NAME[t], r, k)


def test_mxfp4_every_exponent_and_code():
    """all 256 exponents x 16 codes: subnormal results, the largest finite values and the overflow to inf"""
    raw = np.zeros((256, 17), np.uint8)
    raw[:, 0] = np.arange(256)
    raw[:, 1:9] = np.array([0x10, 0x32, 0x54, 0x76, 0x98, 0xBA, 0xDC, 0xFE], np.uint8)    # codes 0..15 in order
    got = R.dequant(raw, R.MXFP4, 32)
    for e in range(256):
        with np.errstate(over="ignore"):
            want = mxfp4_row(bytes(raw[e]))
        assert diff_bits(got[e], want) == 0, e
    assert np.isinf(got[255, 2]) and got[0, 1] == np.float32(2.0 ** -127)       # code 4: 4 * 2^127; code 2: 2 * 2^-128


def test_nvfp4_every_scale_byte():
    raw = np.zeros((64, 36), np.uint8)
    raw[:, :4] = np.arange(256, dtype=np.uint8).reshape(64, 4)
    raw[:, 4:] = np.tile(np.array([0x10, 0x32, 0x54, 0x76, 0x98, 0xBA, 0xDC, 0xFE], np.uint8), 4)
    got = R.dequant(raw, R.NVFP4, 64)
    for i in range(64):
        assert diff_bits(got[i], nvfp4_row(bytes(raw[i]))) == 0, i


def test_e2m1_doubled_is_the_fp4_table():
    """the oracle's FP4 table (ggml's kvalues_mxfp4) is twice the OCP E2M1 value of each code"""
    assert [int(2 * e2m1(c)) for c in range(16)] == [int(v) for v in R.KV_FP4]


def test_iq4_table_is_the_published_one():
    kv = [int(v) for v in R.KV_IQ4]
    assert kv == list(KV_IQ4_PUBLISHED)
    assert all(a < b for a, b in zip(kv, kv[1:])) and kv[0] == -127 and kv[8] == 1


def test_q3_k_scales_two_derivations():
    """the oracle's per-field scale unpack against llama.cpp's kmask shuffle, on random and every-value bytes"""
    rng = np.random.default_rng(31)
    scb = rng.integers(0, 256, (200, 12), dtype=np.uint8)
    scb[0], scb[1] = 0, 0xFF
    got = R.q3_k_scales(scb)
    for i in range(scb.shape[0]):
        assert [int(v) for v in got[i]] == [v - 32 for v in ggml_q3_k_scales(bytes(scb[i]))], i


def test_tq1_0_codes_cover_minus_one_zero_one():
    """every byte value's five base-3 digits come out in {-1, 0, 1}, and the packer's digits round-trip"""
    raw = np.zeros((256, 54), np.uint8)
    raw[:, :32] = np.arange(256, dtype=np.uint8).reshape(256, 1)
    raw[:, 52:54] = np.array([1.0], np.float16).view(np.uint8)
    v = R.dequant(raw, R.TQ1_0, 256)
    assert set(np.unique(v[:, :160])) <= {-1.0, 0.0, 1.0}
    # byte b holds digits t_k with b = ceil(sum t_k 3^(4 - k) * 256 / 243) (ggml's packing): the first digit read is
    # the most significant
    for digits in [(0, 0, 0, 0, 0), (2, 1, 0, 2, 1), (2, 2, 2, 2, 2), (1, 0, 1, 0, 1)]:
        n = sum(d * 3 ** (4 - k) for k, d in enumerate(digits))
        b = (n * 256 + 242) // 243
        row = R.dequant(np.concatenate([np.full((1, 32), b, np.uint8), np.zeros((1, 20), np.uint8),
                                        np.array([1.0], np.float16).view(np.uint8).reshape(1, 2)], 1), R.TQ1_0, 256)
        assert [int(row[0, 32 * k]) for k in range(5)] == [d - 1 for d in digits], digits


@pytest.mark.parametrize("t", sorted(SCALAR), ids=NAME.get)
def test_edge_blocks(t):
    """all-zero blocks give zeros; all-one blocks give NaN where the fp16 scale is NaN (0xFFFF), and the fp8 / E4M3
    types their largest codes"""
    ts, bs = R.TYPES[t][2], R.TYPES[t][1]
    raw = np.zeros((2, ts), np.uint8)
    raw[1] = 0xFF
    v = R.dequant(raw, t, bs)
    assert np.all(v[0] == 0) and not np.any(np.signbit(v[0]) & (t in (R.MXFP4, R.NVFP4)))
    if t == R.MXFP4:
        assert np.all(np.isneginf(v[1]))                               # -12 * 2^127
    elif t == R.NVFP4:
        assert np.all(v[1] == np.float32(-12 * 240))                   # 0xFF: E4M3 1.875 * 2^8 = 480, halved
    else:
        assert np.all(np.isnan(v[1]))


def test_float_types_every_bit_pattern():
    """F16 and BF16 on all 65,536 patterns, F32 on a spread of patterns, against the IEEE-754 definitions"""
    h = np.arange(65536, dtype=np.uint32)
    raw = np.stack([(h & 0xFF), (h >> 8)], -1).astype(np.uint8).reshape(1, -1)
    f16 = R.dequant(raw, R.F16, 65536)[0]
    want = np.array([f16_from_definition(int(v)) for v in h], np.float64)
    with np.errstate(invalid="ignore"):
        same = (np.isnan(f16) & np.isnan(want)) | (f16.astype(np.float64) == want) & (np.signbit(f16) == np.signbit(want))
    assert np.all(same)
    bf = R.dequant(raw, R.BF16, 65536)[0]
    assert np.array_equal(bf.view(np.uint32), h << 16)                 # bfloat16: the top half of a binary32
    rng = np.random.default_rng(5)
    u = rng.integers(0, 2 ** 32, 4096, dtype=np.uint64).astype(np.uint32)
    f32 = R.dequant(u.view(np.uint8).reshape(1, -1), R.F32, 4096)[0]
    assert np.array_equal(f32.view(np.uint32), u)


def test_float_types_keep_odd_row_lengths():
    """block size 1: any row length, leading axes kept"""
    rng = np.random.default_rng(6)
    raw = rng.integers(0, 256, (2, 3, 2 * 37), dtype=np.uint8)
    v = R.dequant(raw, R.BF16, 37)
    assert v.shape == (2, 3, 37)
    assert np.array_equal(v[1, 2].view(np.uint32) >> 16, raw[1, 2].view("<u2").astype(np.uint32))


def _golden_new():
    if not os.path.isdir(GOLDEN):
        return []
    out = []
    for f in sorted(os.listdir(GOLDEN)):
        if f.endswith(".npz"):
            z = np.load(os.path.join(GOLDEN, f), allow_pickle=False)
            if int(z["t"]) in R.EXACT_ONLY:
                out.append(f)
    return out


def test_real_blocks_of_the_new_types_match_the_scalar_forms():
    """llama-quantize blocks of Q5_1, Q2_K, Q3_K, IQ4_NL and IQ4_XS from the reference's fixture models (via
    tests/golden): the oracle equals llama.cpp's scalar loops on every second block"""
    seen = set()
    for name in _golden_new():
        if not name.startswith("kquant_"):
            continue
        z = np.load(os.path.join(GOLDEN, name), allow_pickle=False)
        t, cols, raw = int(z["t"]), int(z["cols"]), z["raw"]
        if t not in SCALAR:
            continue
        got = R.dequant(raw, t, cols)
        _, bs, ts = R.TYPES[t]
        blocks, vals = raw.reshape(-1, ts), got.reshape(-1, bs)
        for i in range(0, blocks.shape[0], 2):
            assert diff_bits(vals[i], SCALAR[t](bytes(blocks[i]))) == 0, (name, i)
        # smooth weight-like values: finite, centred, no code book slip that would blow up a row's scale
        assert np.all(np.isfinite(got)) and abs(float(got.mean())) < 0.1 * float(np.abs(got).mean())
        seen.add(t)
    assert seen == {R.Q5_1, R.Q2_K, R.Q3_K, R.IQ4_NL, R.IQ4_XS}
