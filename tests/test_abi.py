"""The C ABI of libmbq.so without a GPU: it loads, exports every entry point include/mbq.h declares, and its host-side
entry points (type table, shapes, plane sizes, the host repack and its inverse, argument checks) behave as declared.
No entry point that launches a kernel is called with valid arguments here."""
import ctypes
import os
import re

import numpy as np
import pytest

from oracle import gen as G
from oracle import ref as R

import mashbox_amd._lib as L
import mashbox_amd.kernels as KQ

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _declared():
    names = []
    for h in sorted(os.listdir(os.path.join(ROOT, "include"))):
        if h.endswith(".h"):
            src = open(os.path.join(ROOT, "include", h)).read()
            src = re.sub(r"/\*.*?\*/", "", src, flags=re.S)
            names += re.findall(r"\b(mbq_\w+)\s*\(", src)
    return sorted(set(names))


def test_library_exports_every_declared_symbol():
    lib = L.lib()
    names = _declared()
    assert len(names) >= 12, names
    for n in names:
        assert hasattr(lib, n), f"{n} declared in include/ but not exported by libmbq.so"
    assert set(names) == set(L._SIGS), "ctypes signatures and include/mbq.h disagree"


def test_type_table_and_shapes():
    lib = L.lib()
    assert lib.mbq_version() >= 100
    assert lib.mbq_has_type(8) == 1 and lib.mbq_has_type(12) == 1 and lib.mbq_has_type(14) == 1
    assert lib.mbq_has_type(13) == 1 and lib.mbq_has_type(2) == 1 and lib.mbq_has_type(11) == 0
    assert lib.mbq_has_type(3) == 0 and lib.mbq_has_type(6) == 0
    assert lib.mbq_row_bytes(2, 4096) == R.row_bytes(2, 4096) == 2304
    assert lib.mbq_row_bytes(13, 5120) == R.row_bytes(13, 5120) == 3520
    assert lib.mbq_row_bytes(14, 2560) == R.row_bytes(14, 2560) == 2100
    assert lib.mbq_row_bytes(8, 5120) == R.row_bytes(8, 5120) == 5440
    assert lib.mbq_row_bytes(12, 17408) == R.row_bytes(12, 17408) == 9792
    assert lib.mbq_row_bytes(12, 100) < 0
    assert KQ.kq_covers(8, (17408, 5120)) and KQ.kq_covers(12, (5120, 17408))
    assert not KQ.kq_covers(12, (5, 100)) and not KQ.kq_covers(11, (256, 256)) and KQ.kq_covers(13, (256, 256))
    assert KQ.kq_covers(14, (151936, 2560)) and not KQ.kq_covers(14, (8, 128))
    assert KQ.kq_covers(2, (5, 96)) and not KQ.kq_covers(2, (5, 100))
    for t, (n, k) in [(8, (17408, 5120)), (12, (5120, 17408)), (12, (1, 256)), (8, (3, 32)), (14, (151936, 2560)),
                      (14, (1, 256)), (14, (3, 512)), (13, (1, 256)), (13, (17408, 5120)), (2, (1, 32)),
                      (2, (4096, 4096)), (2, (7, 96))]:
        pb = KQ.plane_bytes(t, (n, k))
        file_bytes = n * R.row_bytes(t, k)
        planes = {14: 4, 13: 3}.get(t, 2)                             # each plane pads to 256 bytes
        assert pb % 256 == 0 and file_bytes <= pb < file_bytes + 256 * planes


@pytest.mark.parametrize("t", [R.Q4_0, R.Q8_0, R.Q4_K, R.Q5_K, R.Q6_K])
def test_host_repack_is_lossless(t):
    rng = np.random.default_rng(40 + t)
    for n, kb in [(1, 1), (7, 3), (130, 2)]:
        k = R.TYPES[t][1] * kb
        raw = rng.integers(0, 256, (n, R.row_bytes(t, k)), dtype=np.uint8)
        p = KQ.repack_host(t, raw, (n, k), threads=3)
        back = np.zeros_like(raw)
        rc = L.lib().mbq_unpack_host(t, ctypes.c_void_p(p.buf.data_ptr()), n, k, back.ctypes.data_as(ctypes.c_void_p),
                                     back.size)
        assert rc == 0 and np.array_equal(back, raw)


def test_q4_k_unit_layout_yields_bf16_pairs():
    """a Q4_K plane dword t of a unit holds quants 8t..8t+7 so that ((w >> 4p) & 0x000F000F) | 0x43004300 is the
    bfloat16 pair (128 + q[8t+2p], 128 + q[8t+2p+1]): checked on the host against the oracle's nibble split"""
    rng = np.random.default_rng(41)
    raw = G.q4_k_raw(rng, 2, 256)
    p = KQ.repack_host(R.Q4_K, raw, (2, 256)).buf.numpy()
    units = p[:2 * 128].view(np.uint32).reshape(2, 8, 4)            # (row, sub-block, dword)
    b = raw.reshape(2, 144)
    q = R.nib(b[:, 16:].reshape(2, 4, 32)).reshape(2, 8, 32)        # oracle's quant order
    for p_ in range(4):
        pair = ((units >> np.uint32(4 * p_)) & np.uint32(0x000F000F)) | np.uint32(0x43004300)
        lo = R.bf16_to_f32((pair & 0xFFFF).astype(np.uint16)) - 128
        hi = R.bf16_to_f32((pair >> 16).astype(np.uint16)) - 128
        for t_ in range(4):
            assert np.array_equal(lo[:, :, t_], q[:, :, 8 * t_ + 2 * p_])
            assert np.array_equal(hi[:, :, t_], q[:, :, 8 * t_ + 2 * p_ + 1])


def test_q4_0_unit_layout_yields_bf16_pairs():
    """a Q4_0 unit holds its block's 32 quants in the Q4_K order, so the Q4_K pair rule gives (128 + q, 128 + q') of
    values 8t + 2p, 8t + 2p + 1; and the d plane holds the blocks' scales in file order: checked on the host against the
    oracle's dequant of blocks with d = 1 (its values are then q - 8)"""
    rng = np.random.default_rng(44)
    raw = G.q4_0_raw(rng, 3, 160).reshape(15, 18)
    d = raw[:, 0:2].copy()
    raw[:, 0:2] = np.array([1.0], np.float16).view(np.uint8)
    raw = raw.reshape(3, 90)
    q = (R.dequant(raw, R.Q4_0, 160) + 8).astype(np.int64).reshape(3, 5, 32)   # (row, unit, value)
    p = KQ.repack_host(R.Q4_0, raw, (3, 160)).buf.numpy()
    units = p[:3 * 80].view(np.uint32).reshape(3, 5, 4)
    for p_ in range(4):
        pair = ((units >> np.uint32(4 * p_)) & np.uint32(0x000F000F)) | np.uint32(0x43004300)
        lo = R.bf16_to_f32((pair & 0xFFFF).astype(np.uint16)) - 128
        hi = R.bf16_to_f32((pair >> 16).astype(np.uint16)) - 128
        for t_ in range(4):
            assert np.array_equal(lo[:, :, t_], q[:, :, 8 * t_ + 2 * p_])
            assert np.array_equal(hi[:, :, t_], q[:, :, 8 * t_ + 2 * p_ + 1])
    raw = raw.reshape(15, 18)
    raw[:, 0:2] = d
    p = KQ.repack_host(R.Q4_0, raw.reshape(3, 90), (3, 160)).buf.numpy()
    assert np.array_equal(p[256:256 + 30], d.reshape(-1))           # the d plane starts at the next 256-byte boundary


def test_q6_k_unit_layout_yields_quant_bytes():
    """a Q6_K unit: low nibbles of dword t and the high bits of dword t / 2, masked and shifted as the kernels do
    (q6k_bytes: (ql & 0x0F0F0F0F) | (qh << 4 or qh) & 0x30303030, ((ql >> 4) & 0x0F0F0F0F) | (qh << 2 or qh >> 2) &
    0x30303030), are the 6-bit quants of values 8t..8t+3 and 8t+4..8t+7 as bytes: checked on the host against the
    oracle's dequant of blocks with d = 1 and every scale 1 (its values are then q - 32)"""
    rng = np.random.default_rng(42)
    raw = G.q6_k_raw(rng, 3, 512).reshape(6, 210)
    raw[:, 192:208] = 1
    raw[:, 208:210] = np.array([1.0], np.float16).view(np.uint8)
    raw = raw.reshape(3, 420)
    q = (R.dequant(raw, R.Q6_K, 512) + 32).astype(np.uint32).reshape(3, 16, 32)   # (row, unit, value)
    p = KQ.repack_host(R.Q6_K, raw, (3, 512)).buf.numpy()
    L_ = 3 * 256
    ql = p[:L_].view(np.uint32).reshape(3, 16, 4)
    hi_off = (L_ + 255) // 256 * 256
    qh = p[hi_off:hi_off + 3 * 128].view(np.uint32).reshape(3, 16, 2)
    m3, m0f = np.uint32(0x30303030), np.uint32(0x0F0F0F0F)
    for t_ in range(4):
        h = qh[:, :, t_ >> 1]
        h0 = (h & m3) if t_ & 1 else ((h << np.uint32(4)) & m3)
        h1 = ((h >> np.uint32(2)) & m3) if t_ & 1 else ((h << np.uint32(2)) & m3)
        lo = (ql[:, :, t_] & m0f) | h0
        hi = ((ql[:, :, t_] >> np.uint32(4)) & m0f) | h1
        for j in range(4):
            assert np.array_equal((lo >> np.uint32(8 * j)) & np.uint32(0xFF), q[:, :, 8 * t_ + j])
            assert np.array_equal((hi >> np.uint32(8 * j)) & np.uint32(0xFF), q[:, :, 8 * t_ + 4 + j])


def test_q5_k_unit_layout_yields_quant_bytes():
    """a Q5_K unit: low nibbles as Q6_K's, and the high-bit word rotated right by 2t + 28 (2t + 29) so that bit 4 of
    every byte is the high bit of value 8t + j (8t + 4 + j), as q5k_bytes does: checked on the host against the oracle's
    dequant of blocks with d = 1, dmin = 0 and every scale 1 (its values are then q)"""
    rng = np.random.default_rng(43)
    raw = G.q5_k_raw(rng, 3, 512).reshape(6, 176)
    raw[:, 0:4] = np.array([1.0, 0.0], np.float16).view(np.uint8)
    raw[:, 4:16] = R.pack_scale_min_k4(np.ones((6, 8), np.uint8), np.zeros((6, 8), np.uint8))
    raw = raw.reshape(3, 352)
    q = R.dequant(raw, R.Q5_K, 512).astype(np.uint32).reshape(3, 16, 32)   # (row, unit, value)
    p = KQ.repack_host(R.Q5_K, raw, (3, 512)).buf.numpy()
    ql = p[:3 * 256].view(np.uint32).reshape(3, 16, 4)
    qh = p[768:768 + 3 * 64].view(np.uint32).reshape(3, 16)
    rot = lambda v, s: ((v >> np.uint32(s)) | (v << np.uint32(32 - s))) if s else v
    m1, m0f = np.uint32(0x10101010), np.uint32(0x0F0F0F0F)
    for t_ in range(4):
        lo = (rot(qh, (2 * t_ + 28) % 32) & m1) | (ql[:, :, t_] & m0f)
        hi = (rot(qh, (2 * t_ + 29) % 32) & m1) | ((ql[:, :, t_] >> np.uint32(4)) & m0f)
        for j in range(4):
            assert np.array_equal((lo >> np.uint32(8 * j)) & np.uint32(0xFF), q[:, :, 8 * t_ + j])
            assert np.array_equal((hi >> np.uint32(8 * j)) & np.uint32(0xFF), q[:, :, 8 * t_ + 4 + j])


def test_argument_errors_are_reported_without_a_launch():
    lib = L.lib()
    null = ctypes.c_void_p(0)
    assert lib.mbq_matmul(11, null, 0, None, 1, null, 1, 8, 256, null, 0, null) == -1
    assert b"type" in lib.mbq_last_error()
    assert lib.mbq_matmul(12, null, 0, None, 1, null, 1, 8, 200, null, 0, null) == -1
    assert b"multiple" in lib.mbq_last_error()
    assert lib.mbq_matmul(12, null, 0, None, 1, null, 1, 8, 256, null, 0, null) == -1   # NULL planes
    assert lib.mbq_matmul(12, ctypes.c_void_p(16), 5, None, 2, null, 1, 8, 256, null, 0, null) == -1
    assert b"layer" in lib.mbq_last_error()
    assert lib.mbq_matmul(12, ctypes.c_void_p(16), 0, None, 1, null, 1, 8, 256, null, 7, null) == -1
    assert lib.mbq_int8_linear(null, null, null, 1, 8, 100, null, 1, null) == -1         # K % 16
    small = np.zeros(16, np.uint8)
    raw = np.zeros((1, 144), np.uint8)
    assert lib.mbq_repack_host(12, raw.ctypes.data_as(ctypes.c_void_p), 1, 256,
                               small.ctypes.data_as(ctypes.c_void_p), small.size, 1) == -3
    with pytest.raises(L.MbqError):
        L.check(-1, "x")


@pytest.mark.parametrize("n,k", [(1, 16), (17, 48), (33, 1040), (130, 4096)])
def test_int8_tiled_repack_is_lossless(n, k):
    """the load-time int8 repack (16-row tiles of 16 rows x 64 bytes, then the scales) inverts exactly; its padding
    rows and columns are zero; plane bytes = 16-row-rounded rows x 64-rounded K + the scale plane, each 256-aligned"""
    from mashbox_amd import int8 as I8
    rng = np.random.default_rng([n, k])
    q, s = G.int8_weights(rng, n, k)
    p = I8.repack_host(q, s, threads=3)
    np16, kp = (n + 15) // 16 * 16, (k + 63) // 64 * 64
    a256 = lambda v: (v + 255) // 256 * 256
    assert p.stride == a256(a256(np16 * kp) + np16 * 4)
    buf = p.buf.numpy()
    q2, s2 = np.zeros_like(q), np.zeros_like(s)
    assert L.lib().mbq_int8_unpack_host(buf.ctypes.data_as(ctypes.c_void_p), n, k, q2.ctypes.data_as(ctypes.c_void_p),
                                        s2.ctypes.data_as(ctypes.c_void_p)) == 0
    assert np.array_equal(q2, q) and np.array_equal(s2.view(np.uint32), s.view(np.uint32))
    # tile (rt, kc) row r holds q[16 rt + r, 64 kc : 64 kc + 64], zero past n or k
    tiles = buf[:np16 * kp].reshape(np16 // 16, kp // 64, 16, 64).view(np.int8)
    full = np.zeros((np16, kp), np.int8)
    full[:n, :k] = q
    assert np.array_equal(tiles.transpose(0, 2, 1, 3).reshape(np16, kp), full)
    sc = buf[a256(np16 * kp):a256(np16 * kp) + np16 * 4].view(np.float32)
    assert np.array_equal(sc[:n].view(np.uint32), s.view(np.uint32)) and not sc[n:].any()
    assert L.lib().mbq_covers(L.I8T, n, k) == 1 and L.lib().mbq_covers(L.I8T, n, k + 8) == 0
    assert L.lib().mbq_dequant(L.I8T, None, 0, None, 1, n, k, None, None) < 0


@pytest.mark.parametrize("n,kb", [(1, 1), (17, 2), (130, 3)])
def test_q4_k_tiled_repack_is_lossless(n, kb):
    """Q4_K blocks into 16-row tiles (MBQ_Q4KT) and back, exactly. The tiles hold the row-major planes' bytes: quant
    block (rt, kc) row r = the 64 bytes at 64 kc of row 16 rt + r's qs plane, header block (rt, sb) row r = that row's
    header sb; the rows of the last tile past n are zero; plane bytes = the two planes over 16-row-rounded rows, each
    256-aligned"""
    k = 256 * kb
    rng = np.random.default_rng([n, kb, 12])
    raw = rng.integers(0, 256, (n, R.row_bytes(R.Q4_K, k)), dtype=np.uint8)
    p = KQ.repack_host(R.Q4_K, raw, (n, k), threads=3, tiled=True)
    rm = KQ.repack_host(R.Q4_K, raw, (n, k))
    assert p.t == L.Q4KT and rm.t == R.Q4_K
    np16 = (n + 15) // 16 * 16
    a256 = lambda v: (v + 255) // 256 * 256
    assert p.stride == a256(a256(np16 * k // 2) + np16 * (k // 256) * 16)
    buf, rmb = p.buf.numpy(), rm.buf.numpy()
    full = np.zeros((np16, k // 2), np.uint8)
    full[:n] = rmb[:n * k // 2].reshape(n, k // 2)
    tiles = buf[:np16 * k // 2].reshape(np16 // 16, k // 128, 16, 64)
    assert np.array_equal(tiles.transpose(0, 2, 1, 3).reshape(np16, k // 2), full)
    mfull = np.zeros((np16, k // 256, 16), np.uint8)
    mfull[:n] = rmb[a256(n * k // 2):a256(n * k // 2) + n * (k // 256) * 16].reshape(n, k // 256, 16)
    mo = a256(np16 * k // 2)
    heads = buf[mo:mo + np16 * (k // 256) * 16].reshape(np16 // 16, k // 256, 16, 16)
    assert np.array_equal(heads.transpose(0, 2, 1, 3).reshape(np16, k // 256, 16), mfull)
    back = np.zeros_like(raw)
    assert L.lib().mbq_unpack_host(L.Q4KT, ctypes.c_void_p(p.buf.data_ptr()), n, k, back.ctypes.data_as(ctypes.c_void_p),
                                   back.size) == 0
    assert np.array_equal(back, raw)
    assert L.lib().mbq_covers(L.Q4KT, n, k) == 1 and L.lib().mbq_covers(L.Q4KT, n, k + 32) == 0
    assert L.lib().mbq_has_type(L.Q4KT) == 0 and L.lib().mbq_row_bytes(L.Q4KT, k) < 0     # not a ggml type
    assert L.lib().mbq_dequant_raw(L.Q4KT, None, n, k, None, None) < 0                    # its blocks are Q4_K's
    with pytest.raises(NotImplementedError):
        KQ.repack_host(99, np.zeros((1, 18), np.uint8), (1, 32), tiled=True)


def test_raw_type_table():
    """mbq_row_bytes knows every ggml type (the file's row bytes, reference ops/reference.py:22-29, 390-395) and
    mbq_has_raw_type names the exact path's types: all but the seven code-book types, which mbq_dequant_raw refuses
    before touching the GPU"""
    from mashbox_amd import gguf
    lib = L.lib()
    for t, (name, bs, ts) in gguf.GGML_TYPES.items():
        cols = bs * 6
        assert lib.mbq_row_bytes(t, cols) == 6 * ts, name
        if bs > 1:
            assert lib.mbq_row_bytes(t, cols + 1) < 0, name
        assert lib.mbq_has_raw_type(t) == (1 if t in R.TYPES else 0), name
        if t in R.TYPES:
            assert R.row_bytes(t, cols) == 6 * ts
    assert set(R.TYPES) == set(R.KERNEL_TYPES) | set(R.EXACT_ONLY)
    assert len(set(gguf.GGML_TYPES) - set(R.TYPES)) == 7
    for t in set(gguf.GGML_TYPES) - set(R.TYPES):
        assert lib.mbq_dequant_raw(t, None, 1, 256, None, None) < 0
        assert "code book" in L.lib().mbq_last_error().decode()
    for t in (-12, 4, 5, 41, 99):
        assert lib.mbq_has_raw_type(t) == 0 and lib.mbq_row_bytes(t, 256) < 0
    for t in R.KERNEL_TYPES:
        assert lib.mbq_has_type(t) == 1 and lib.mbq_has_raw_type(t) == 1
    for t in R.EXACT_ONLY:
        assert lib.mbq_has_type(t) == 0                                   # no kernel planes: the exact path only
    # argument checks before any launch: empty shapes, partial blocks, the float types' any row length
    assert lib.mbq_dequant_raw(R.Q3_K, None, 0, 256, None, None) < 0
    assert lib.mbq_dequant_raw(R.Q3_K, None, 4, 200, None, None) < 0
    assert lib.mbq_dequant_raw(R.NVFP4, None, 4, 96, None, None) < 0
    assert lib.mbq_row_bytes(R.BF16, 37) == 74 and lib.mbq_row_bytes(R.F32, 3) == 12


@pytest.mark.parametrize("n,kb", [(1, 1), (17, 2), (130, 3)])
def test_q6_k_tiled_repack_is_lossless(n, kb):
    """Q6_K blocks into 16-row tiles (MBQ_Q6KT) and back, exactly; the low-nibble tiles hold the row-major planes' bytes
    (16 rows x 64 bytes per 128-value chunk, as MBQ_Q4KT's); rows of the last tile past n are zero"""
    k = 256 * kb
    rng = np.random.default_rng([n, kb, 14])
    raw = rng.integers(0, 256, (n, R.row_bytes(R.Q6_K, k)), dtype=np.uint8)
    p = KQ.repack_host(R.Q6_K, raw, (n, k), threads=3, tiled=True)
    rm = KQ.repack_host(R.Q6_K, raw, (n, k))
    assert p.t == L.Q6KT
    np16 = (n + 15) // 16 * 16
    full = np.zeros((np16, k // 2), np.uint8)
    full[:n] = rm.buf.numpy()[:n * k // 2].reshape(n, k // 2)
    tiles = p.buf.numpy()[:np16 * k // 2].reshape(np16 // 16, k // 128, 16, 64)
    assert np.array_equal(tiles.transpose(0, 2, 1, 3).reshape(np16, k // 2), full)
    back = np.zeros_like(raw)
    assert L.lib().mbq_unpack_host(L.Q6KT, ctypes.c_void_p(p.buf.data_ptr()), n, k, back.ctypes.data_as(ctypes.c_void_p),
                                   back.size) == 0
    assert np.array_equal(back, raw)


@pytest.mark.parametrize("n,k", [(1, 32), (17, 64), (33, 96), (130, 1056)])
def test_q8_0_tiled_repack_is_lossless(n, k):
    """Q8_0 blocks into 16-row tiles (MBQ_Q8T) and back, exactly. Quant block (rt, kc) row r = values 64 kc .. of row
    16 rt + r, value v of the chunk at byte 16 ((v % 32) // 8) + 8 (v // 32) + v % 8 (lane group g's 16 bytes: its 8
    values of each 32-value block); scale block (rt, kc) row r = that row's two fp16 block scales of the chunk; rows
    past n and the half chunk past k are zero"""
    rng = np.random.default_rng([n, k, 8])
    raw = rng.integers(0, 256, (n, R.row_bytes(R.Q8_0, k)), dtype=np.uint8)
    p = KQ.repack_host(R.Q8_0, raw, (n, k), threads=3, tiled=True)
    assert p.t == L.Q8T
    np16, kp = (n + 15) // 16 * 16, (k + 63) // 64 * 64
    a256 = lambda v: (v + 255) // 256 * 256
    assert p.stride == a256(a256(np16 * kp) + np16 * kp // 16)
    buf = p.buf.numpy()
    blocks = raw.reshape(n, k // 32, 34)
    q = np.zeros((np16, kp), np.uint8)
    q[:n, :k] = blocks[:, :, 2:].reshape(n, k)
    d = np.zeros((np16, kp // 32, 2), np.uint8)
    d[:n, :k // 32] = blocks[:, :, :2]
    v = np.arange(64)
    pos = 16 * ((v % 32) // 8) + 8 * (v // 32) + v % 8
    assert sorted(pos) == list(range(64))
    tiles = buf[:np16 * kp].reshape(np16 // 16, kp // 64, 16, 64)[..., pos]
    assert np.array_equal(tiles.transpose(0, 2, 1, 3).reshape(np16, kp), q)
    so = a256(np16 * kp)
    ds = buf[so:so + np16 * kp // 16].reshape(np16 // 16, kp // 64, 16, 4)
    assert np.array_equal(ds.transpose(0, 2, 1, 3).reshape(np16, kp // 32, 2), d)
    back = np.zeros_like(raw)
    assert L.lib().mbq_unpack_host(L.Q8T, ctypes.c_void_p(p.buf.data_ptr()), n, k, back.ctypes.data_as(ctypes.c_void_p),
                                   back.size) == 0
    assert np.array_equal(back, raw)
    assert L.lib().mbq_covers(L.Q8T, n, k) == 1 and L.lib().mbq_covers(L.Q8T, n, k + 16) == 0
