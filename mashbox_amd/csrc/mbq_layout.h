// Kernel-plane layout of one (N, K) weight, shared by the host repack and the device kernels.
//
// The GGUF blocks of a row are split into two planes so that every lane of a wave reads whole 16-byte vectors:
//
//   Q8_0 (ggml 8, 32 values / 34 B per block; reference src/mashbox/ops/reference.py:101-103)
//     qs   int8  (N, K)            the blocks' 32 quants, in file order
//     d    fp16  (N, K/32)         the blocks' scales
//   Q4_K (ggml 12, 256 values / 144 B per super-block; reference src/mashbox/ops/reference.py:132-149)
//     qs   (N, K/32, 16 B)         one 16-byte unit per sub-block of 32 quants; dword t of a unit holds quants
//                                  8t..8t+7 with quant 8t+2p in bits 4p..4p+3 and quant 8t+2p+1 in bits 16+4p..19+4p,
//                                  so ((dword >> 4p) & 0x000F000F) | 0x43004300 is the bfloat16 pair
//                                  (128 + q[8t+2p], 128 + q[8t+2p+1]) in one AND-OR
//     meta (N, K/256, 16 B)        the super-block's first 16 bytes as stored: d fp16, dmin fp16, 12 scale bytes
//
// Both planes start 256-byte aligned and the whole is rounded up to 256 bytes, so a stack of weights is a plain array
// of these records (mbq_plane_bytes apart). The byte count is the file's plus at most 511 bytes of zero padding.
#pragma once
#include <stdint.h>

namespace mbq {

enum : int { T_Q8_0 = 8, T_Q4_K = 12, T_INT8 = -8 };

constexpr int64_t align256(int64_t v) { return (v + 255) & ~int64_t(255); }

struct Layout {
    int64_t qs_off, qs_bytes, sc_off, sc_bytes, total;
};

inline int block_values(int t) { return t == T_Q8_0 ? 32 : t == T_Q4_K ? 256 : 0; }
inline int block_bytes(int t) { return t == T_Q8_0 ? 34 : t == T_Q4_K ? 144 : 0; }

inline Layout layout(int t, int64_t n, int64_t k) {
    Layout L{};
    if (t == T_Q8_0) {
        L.qs_bytes = n * k;
        L.sc_bytes = n * (k / 32) * 2;
    } else {  // T_Q4_K
        L.qs_bytes = n * (k / 2);
        L.sc_bytes = n * (k / 256) * 16;
    }
    L.qs_off = 0;
    L.sc_off = align256(L.qs_bytes);
    L.total = align256(L.sc_off + L.sc_bytes);
    return L;
}

// Q4_K: position of quant i (0..31) of a sub-block inside its 16-byte unit: (dword index, bit offset)
inline void q4k_slot(int i, int* dword, int* bit) {
    const int e = i & 7;
    *dword = i >> 3;
    *bit = 16 * (e & 1) + 4 * (e >> 1);
}

}  // namespace mbq
