// Kernel-plane layout of one (N, K) weight, shared by the host repack and the device kernels.
//
// The GGUF blocks of a row are split into two planes so that every lane of a wave reads whole 16-byte vectors:
//
//   Q4_0 (ggml 2, 32 values / 18 B per block; reference src/mashbox/ops/reference.py:66-70)
//     qs   (N, K/32, 16 B)         one 16-byte unit per block, its 32 quants in the Q4_K unit order below
//     d    fp16  (N, K/32)         the blocks' scales (in the sc plane, as Q8_0's)
//   value = d * (q - 8), exact in float32
//   Q8_0 (ggml 8, 32 values / 34 B per block; reference src/mashbox/ops/reference.py:101-103)
//     qs   int8  (N, K)            the blocks' 32 quants, in file order
//     d    fp16  (N, K/32)         the blocks' scales
//   Q4_K (ggml 12, 256 values / 144 B per super-block; reference src/mashbox/ops/reference.py:132-149)
//     qs   (N, K/32, 16 B)         one 16-byte unit per sub-block of 32 quants; dword t of a unit holds quants
//                                  8t..8t+7 with quant 8t+2p in bits 4p..4p+3 and quant 8t+2p+1 in bits 16+4p..19+4p,
//                                  so ((dword >> 4p) & 0x000F000F) | 0x43004300 is the bfloat16 pair
//                                  (128 + q[8t+2p], 128 + q[8t+2p+1]) in one AND-OR
//     meta (N, K/256, 16 B)        the super-block's first 16 bytes as stored: d fp16, dmin fp16, 12 scale bytes
//   Q5_K (ggml 13, 256 values / 176 B per super-block; reference src/mashbox/ops/reference.py:150-159)
//     qs   (N, K/32, 16 B)         low 4 bits of the 5-bit quants q of 32 values, as the Q6_K low nibbles below
//     qh   (N, K/32, 4 B)          their high bits; byte j, bit 2t + h = the high bit of q[8t+4h+j] (t = 0..3, h = 0, 1),
//                                  so one rotate moves the high bits of four values to bit 4 of their bytes and one
//                                  bit-field insert joins them to the low nibbles (q5k_bytes in mbq_device.h)
//     meta (N, K/256, 16 B)        the super-block's first 16 bytes as stored: d fp16, dmin fp16, 12 scale bytes
//   value = (d * sc) * q - dmin * m, one rounding (as Q4_K)
//   Q6_K (ggml 14, 256 values / 210 B per super-block; reference src/mashbox/ops/reference.py:164-173)
//     qs   (N, K/32, 16 B)         low 4 bits of the 6-bit quants q of 32 values; dword t, byte j: bits 0-3 = q[8t+j],
//                                  bits 4-7 = q[8t+4+j] (values counted inside the unit of 32)
//     qh   (N, K/32, 8 B)          high 2 bits of the same 32 quants; dword h, byte j: bits 2r, 2r+1 = q[16h+4r+j]
//                                  (r = 0..3), so one AND and at most one shift move the high bits of four values to
//                                  bits 4-5 of their bytes, and an AND-OR with the low nibbles leaves q[8t..8t+3] and
//                                  q[8t+4..8t+7] as bytes (q6k_bytes in mbq_device.h)
//     sc   (N, K/16)   int8        the sub-block scales, in file order
//     d    (N, K/256)  fp16        the super-block scales
//   value = (d * sc) * (q - 32), exact in float32
//
//   int8 per output channel (MBQ_INT8 planes, repacked once at load from the (N, K) int8 quants and (N,) float32
//   scales of reference src/mashbox/models/qwen3_8_27b/model.py:72-82; internal type T_I8T)
//     qs   (NP / 16, KP / 64) blocks of 1 KiB (NP = N rounded up to 16, KP = K rounded up to 64): block (rt, kc) holds
//                                  rows 16 rt .. 16 rt + 15, 64 bytes each (values 64 kc .. 64 kc + 63), so the 16
//                                  rows x 64 bytes a wave loads as one MFMA B tile are one contiguous KiB
//     s    f32 (NP)                the per-row scales
//   padding rows and columns are zero (scale 0)
//
//   Q4_K in 16-row tiles (MBQ_Q4KT planes, repacked once at load from the same Q4_K blocks; internal type T_Q4KT)
//     qs   (NP / 16, K / 128) blocks of 1 KiB: block (rt, kc) holds rows 16 rt .. 16 rt + 15, 64 bytes each (the
//                                  four Q4_K units of values 128 kc .. 128 kc + 127, as in the row-major qs plane), so
//                                  a wave's 16-row MFMA B tile of 128 values is one contiguous KiB
//     meta (NP / 16, K / 256) blocks of 256 bytes: block (rt, sb) holds the 16-byte super-block headers (d, dmin,
//                                  12 scale bytes, as stored) of super-block sb of rows 16 rt .. 16 rt + 15
//   padding rows are zero (d = dmin = 0: value 0)
//
//   Q4_0 in 16-row tiles (MBQ_Q40T planes, repacked once at load from the same Q4_0 blocks; internal type T_Q40T)
//     qs   (NP / 16, KP / 128) blocks of 1 KiB (KP = K rounded up to 128): row r at 64 r, the four units of the chunk
//                                  (the row-major qs plane's bytes), as MBQ_Q4KT's
//     d    (NP / 16, KP / 128) blocks of 128 B: row r at 8 r, the fp16 scales of the chunk's four blocks
//   rows past N and blocks past K are zero (scale 0)
//
//   Q5_K in 16-row tiles (MBQ_Q5KT planes, repacked once at load from the same Q5_K blocks; internal type T_Q5KT): the
//   low nibbles and the super-block headers as MBQ_Q4KT's, and the high bits in (NP / 16, K / 128) blocks of 256 B
//   (row r at 16 r: the chunk's four units' 4-byte words); rows past N zero
//
//   Q6_K in 16-row tiles (MBQ_Q6KT planes, repacked once at load from the same Q6_K blocks; internal type T_Q6KT): the
//   four planes of row-major Q6_K, each in 16-row tiles of 128-value chunks (rows past N zero):
//     qs   (NP / 16, K / 128) blocks of 1 KiB: row r at 64 r (its four units' low nibbles), as MBQ_Q4KT's
//     qh   (NP / 16, K / 128) blocks of 512 B: row r at 32 r (the four units' 8 bytes of high bits)
//     sc   (NP / 16, K / 128) blocks of 128 B: row r at 8 r (the chunk's 8 sub-block scales)
//     d    (NP / 16, K / 256) blocks of 32 B: row r at 2 r (the super-block scale)
//
//   Q8_0 in 16-row tiles (MBQ_Q8T planes, repacked once at load from the same Q8_0 blocks; internal type T_Q8T)
//     qs   (NP / 16, KP / 64) blocks of 1 KiB (KP = K rounded up to 64): row r of block (rt, kc) holds the int8
//                                  quants of values 64 kc .. 64 kc + 63 of row 16 rt + r, 16-byte group g = values
//                                  8g .. 8g + 7 of the chunk's first 32-value block, then the same of its second, so
//                                  that lane group g's one 128-bit load holds its 8 values of each block
//     d    (NP / 16, KP / 64) blocks of 64 bytes: row r holds the fp16 scales of its two 32-value blocks of the chunk
//   padding rows and the padding half-chunk past K are zero (scale 0)
//
// Every plane starts 256-byte aligned and the whole is rounded up to 256 bytes, so a stack of weights is a plain array
// of these records (mbq_plane_bytes apart). The byte count is the file's plus at most 256 bytes of zero padding per
// plane.
#pragma once
#include <stdint.h>

namespace mbq {

// T_INT8: the caller's row-major int8 weights (mbq_int8_linear); T_I8T: int8 weights repacked into 16-row tiles
// (mbq_matmul with MBQ_I8T planes); T_Q40T, T_Q4KT, T_Q5KT, T_Q6KT and T_Q8T: the GGUF types' blocks repacked into
// 16-row tiles (MBQ_Q40T, MBQ_Q4KT, MBQ_Q5KT, MBQ_Q6KT and MBQ_Q8T planes)
enum : int { T_Q4_0 = 2, T_Q8_0 = 8, T_Q4_K = 12, T_Q5_K = 13, T_Q6_K = 14, T_INT8 = -8, T_I8T = -9, T_Q8T = -10,
             T_Q40T = -11, T_Q4KT = -12, T_Q5KT = -13, T_Q6KT = -14 };
// the other ggml types whose file blocks the exact path dequantizes (mbq_dequant_raw, no planes)
enum : int { T_F32 = 0, T_F16 = 1, T_Q4_1 = 3, T_Q5_0 = 6, T_Q5_1 = 7, T_Q2_K = 10, T_Q3_K = 11, T_IQ4_NL = 20,
             T_IQ4_XS = 23, T_BF16 = 30, T_TQ1_0 = 34, T_TQ2_0 = 35, T_MXFP4 = 39, T_NVFP4 = 40 };

// values and bytes of one block of ggml type t ({0, 0} for an id that is not a ggml type): the table of reference
// src/mashbox/ops/reference.py:22-29 (gguf-py's GGML_QUANT_SIZES), which fixes every GGUF file's row bytes
struct GgmlBlock { int values, bytes; };
constexpr GgmlBlock ggml_block(int t) {
    switch (t) {
        case 0: return {1, 4};     case 1: return {1, 2};     case 2: return {32, 18};   case 3: return {32, 20};
        case 6: return {32, 22};   case 7: return {32, 24};   case 8: return {32, 34};   case 10: return {256, 84};
        case 11: return {256, 110}; case 12: return {256, 144}; case 13: return {256, 176}; case 14: return {256, 210};
        case 16: return {256, 66}; case 17: return {256, 74}; case 18: return {256, 98}; case 19: return {256, 50};
        case 20: return {32, 18};  case 21: return {256, 110}; case 22: return {256, 82}; case 23: return {256, 136};
        case 29: return {256, 56}; case 30: return {1, 2};    case 34: return {256, 54}; case 35: return {256, 66};
        case 39: return {32, 17};  case 40: return {64, 36};
    }
    return {0, 0};
}
// the alignment (bytes) every block start of ggml type t keeps when its blocks start there: the largest power of two, at
// most 4, that divides the block bytes (the raw kernels read the blocks with loads that assume it)
constexpr int raw_block_align(int t) {
    const int b = ggml_block(t).bytes;
    return b % 4 == 0 ? 4 : b % 2 == 0 ? 2 : 1;
}
// the ggml types mbq_dequant_raw reads: every one but the seven whose values come from gguf-py's code books (IQ2_XXS,
// IQ2_XS, IQ2_S, IQ3_XXS, IQ3_S, IQ1_S, IQ1_M: reference src/mashbox/ops/reference.py:243-252)
inline bool raw_type(int t) {
    switch (t) {
        case T_F32: case T_F16: case T_BF16: case T_Q4_0: case T_Q4_1: case T_Q5_0: case T_Q5_1: case T_Q8_0:
        case T_Q2_K: case T_Q3_K: case T_Q4_K: case T_Q5_K: case T_Q6_K: case T_IQ4_NL: case T_IQ4_XS: case T_TQ1_0:
        case T_TQ2_0: case T_MXFP4: case T_NVFP4: return true;
    }
    return false;
}
// int8 types: 16-byte units of 16 values, a per-row float32 scale applied to the sum
constexpr bool int8_type(int t) { return t == T_INT8 || t == T_I8T; }
// T_I8T: bytes between consecutive 16-row tiles of the quant plane, and the byte offset of (row, K offset k0) (k0 a
// multiple of 64)
constexpr int64_t i8t_tile_bytes(int64_t k) { return (k + 63) / 64 * 1024; }
constexpr int64_t i8t_off(int64_t row, int64_t k, int64_t k0) { return (row >> 4) * i8t_tile_bytes(k) + (k0 >> 6) * 1024 + (row & 15) * 64; }

// T_Q4KT: bytes between consecutive 16-row tiles of the quant plane, the byte offset of (row, value 0) in it (a value
// k of the row-major qs plane's byte b = k / 2 sits at + (b / 64) * 1024 + b % 64), and the offset of (row, super-block
// 0) in the meta plane (super-block sb at + 256 sb)
constexpr int64_t q4kt_tile_bytes(int64_t k) { return k / 128 * 1024; }
constexpr int64_t q4kt_off(int64_t row, int64_t k) { return (row >> 4) * q4kt_tile_bytes(k) + (row & 15) * 64; }
constexpr int64_t q4kt_meta_off(int64_t row, int64_t k) { return (row >> 4) * (k / 256) * 256 + (row & 15) * 16; }
// T_Q8T: offset of (row, chunk 0)'s two fp16 scales in the d plane (chunk kc of 64 values at + 64 kc); its quants sit
// at i8t_off, value v (0..63) of a chunk row at byte q8t_byte(v)
constexpr int64_t q8t_d_off(int64_t row, int64_t k) { return (row >> 4) * ((k + 63) / 64) * 64 + (row & 15) * 4; }
constexpr int q8t_byte(int v) { return ((v & 31) >> 3) * 16 + (v >> 5) * 8 + (v & 7); }
// T_Q6KT: offsets of (row, chunk 0) in the qh and sc planes (chunk kc at + 512 kc, + 128 kc) and of (row, super-block 0)
// in the d plane (super-block sb at + 32 sb); its low nibbles sit at q4kt_off
constexpr int64_t q6kt_h_off(int64_t row, int64_t k) { return (row >> 4) * (k / 128) * 512 + (row & 15) * 32; }
constexpr int64_t q6kt_s_off(int64_t row, int64_t k) { return (row >> 4) * (k / 128) * 128 + (row & 15) * 8; }
constexpr int64_t q6kt_d_off(int64_t row, int64_t k) { return (row >> 4) * (k / 256) * 32 + (row & 15) * 2; }
// tiled plane types (16-row tiles, any number of rows)
constexpr bool tiled_type(int t) { return t == T_I8T || t == T_Q4KT || t == T_Q8T || t == T_Q6KT || t == T_Q5KT || t == T_Q40T; }
// T_Q40T: offsets of (row, chunk 0) in the qs plane (chunk kc of 128 values at + 1024 kc) and the d plane (+ 128 kc)
constexpr int64_t q40t_off(int64_t row, int64_t k) { return (row >> 4) * ((k + 127) / 128) * 1024 + (row & 15) * 64; }
constexpr int64_t q40t_d_off(int64_t row, int64_t k) { return (row >> 4) * ((k + 127) / 128) * 128 + (row & 15) * 8; }
// the Q4_0 value format, in row-major or tiled planes
constexpr bool q40_like(int t) { return t == T_Q4_0 || t == T_Q40T; }
// T_Q5KT: offset of (row, chunk 0) in the high-bit plane (chunk kc at + 256 kc); low nibbles and headers as T_Q4KT's
constexpr int64_t q5kt_h_off(int64_t row, int64_t k) { return (row >> 4) * (k / 128) * 256 + (row & 15) * 16; }
// the Q5_K value format, in row-major or tiled planes
constexpr bool q5k_like(int t) { return t == T_Q5_K || t == T_Q5KT; }
// the Q6_K value format, in row-major or tiled planes
constexpr bool q6k_like(int t) { return t == T_Q6_K || t == T_Q6KT; }
// the Q4_K value format, in row-major or tiled planes
constexpr bool q4k_like(int t) { return t == T_Q4_K || t == T_Q4KT; }
// the Q8_0 value format, in row-major or tiled planes
constexpr bool q8_like(int t) { return t == T_Q8_0 || t == T_Q8T; }

// the K-quants: 256-value super-blocks, kernel units of 32 values (16 bytes of low nibbles)
constexpr bool kquant(int t) {
    return t == T_Q4_K || t == T_Q5_K || t == T_Q6_K || t == T_Q4KT || t == T_Q5KT || t == T_Q6KT;
}
// types whose kernel unit is 16 bytes of nibbles for 32 values (the K-quants and Q4_0); Q8_0 and int8 units are 16
// bytes for 16 values
constexpr bool unit32(int t) { return kquant(t) || q40_like(t); }
// Q4_0 and Q4_K: a unit's 16 bytes are the whole 4-bit quants, in the Q4_K order
constexpr bool nib4(int t) { return q4k_like(t) || q40_like(t); }

constexpr int64_t align256(int64_t v) { return (v + 255) & ~int64_t(255); }

// plane offsets and sizes in bytes; hi (the Q6_K high bits) and d (the Q6_K super-block scales) are empty for the
// other types
struct Layout {
    int64_t qs_off, qs_bytes, hi_off, hi_bytes, sc_off, sc_bytes, d_off, d_bytes, total;
};

// values and file bytes of one block (T_Q4KT planes are made from Q4_K blocks)
inline int block_values(int t) { return (q8_like(t) || q40_like(t)) ? 32 : kquant(t) ? 256 : 0; }
inline int block_bytes(int t) {
    return q40_like(t) ? 18 : q8_like(t) ? 34 : q4k_like(t) ? 144 : q5k_like(t) ? 176 : q6k_like(t) ? 210 : 0;
}

inline Layout layout(int t, int64_t n, int64_t k) {
    Layout L{};
    if (t == T_Q8_0) {
        L.qs_bytes = n * k;
        L.sc_bytes = n * (k / 32) * 2;
    } else if (t == T_Q4_0) {
        L.qs_bytes = n * (k / 2);
        L.sc_bytes = n * (k / 32) * 2;
    } else if (t == T_Q4_K) {
        L.qs_bytes = n * (k / 2);
        L.sc_bytes = n * (k / 256) * 16;
    } else if (t == T_Q5_K) {
        L.qs_bytes = n * (k / 2);
        L.hi_bytes = n * (k / 8);
        L.sc_bytes = n * (k / 256) * 16;
    } else if (t == T_I8T) {
        const int64_t np = (n + 15) / 16 * 16;
        L.qs_bytes = np * ((k + 63) / 64 * 64);
        L.sc_bytes = np * 4;
    } else if (t == T_Q8T) {
        const int64_t np = (n + 15) / 16 * 16, kp = (k + 63) / 64 * 64;
        L.qs_bytes = np * kp;
        L.sc_bytes = np * (kp / 16);
    } else if (t == T_Q40T) {
        const int64_t np = (n + 15) / 16 * 16, kp = (k + 127) / 128 * 128;
        L.qs_bytes = np * (kp / 2);
        L.sc_bytes = np * (kp / 16);
    } else if (t == T_Q5KT) {
        const int64_t np = (n + 15) / 16 * 16;
        L.qs_bytes = np * (k / 2);
        L.hi_bytes = np * (k / 8);
        L.sc_bytes = np * (k / 256) * 16;
    } else if (t == T_Q6KT) {
        const int64_t np = (n + 15) / 16 * 16;
        L.qs_bytes = np * (k / 2);
        L.hi_bytes = np * (k / 4);
        L.sc_bytes = np * (k / 16);
        L.d_bytes = np * (k / 256) * 2;
    } else if (t == T_Q4KT) {
        const int64_t np = (n + 15) / 16 * 16;
        L.qs_bytes = np * (k / 2);
        L.sc_bytes = np * (k / 256) * 16;
    } else {  // T_Q6_K
        L.qs_bytes = n * (k / 2);
        L.hi_bytes = n * (k / 4);
        L.sc_bytes = n * (k / 16);
        L.d_bytes = n * (k / 256) * 2;
    }
    L.qs_off = 0;
    L.hi_off = align256(L.qs_bytes);
    L.sc_off = align256(L.hi_off + L.hi_bytes);
    L.d_off = align256(L.sc_off + L.sc_bytes);
    L.total = align256(L.d_off + L.d_bytes);
    return L;
}

// Q5_K: where quant i (0..31) of a unit sits: low nibble as Q6_K's; high bit in qh byte i%4, bit 2 (i/8) + (i/4)%2
inline void q5k_slot(int i, int* lo_byte, int* lo_bit, int* hi_byte, int* hi_bit) {
    *lo_byte = 4 * (i >> 3) + (i & 3);
    *lo_bit = 4 * ((i >> 2) & 1);
    *hi_byte = i & 3;
    *hi_bit = 2 * (i >> 3) + ((i >> 2) & 1);
}

// Q6_K: where quant i (0..31) of a unit sits: low nibble in qs dword i/8, byte i%4, bits 4 ((i/4)%2) ..; high bits in
// qh dword i/16, byte i%4, bits 2 ((i/4)%4) ..
inline void q6k_slot(int i, int* lo_byte, int* lo_bit, int* hi_byte, int* hi_bit) {
    *lo_byte = 4 * (i >> 3) + (i & 3);
    *lo_bit = 4 * ((i >> 2) & 1);
    *hi_byte = 4 * (i >> 4) + (i & 3);
    *hi_bit = 2 * ((i >> 2) & 3);
}

// Q4_K, Q4_0: position of quant i (0..31) of a sub-block (block) inside its 16-byte unit: (dword index, bit offset)
inline void q4k_slot(int i, int* dword, int* bit) {
    const int e = i & 7;
    *dword = i >> 3;
    *bit = 16 * (e & 1) + 4 * (e >> 1);
}

}  // namespace mbq
