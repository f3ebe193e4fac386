// Host repack of one weight into kernel planes (every GGUF type also into 16-row tiles), and its inverse (no HIP: also
// built alone, under the host sanitizers, by tests/test_host_sanitizers.py). Plane layouts: mbq_layout.h; file blocks: reference
// src/mashbox/ops/reference.py:66-70 (Q4_0), :101-103 (Q8_0), :132-149 (Q4_K), :150-159 (Q5_K), :164-173 (Q6_K);
// int8 per-channel weights: reference src/mashbox/models/qwen3_8_27b/model.py:72-82.
#pragma once
#include <stdint.h>

#include <algorithm>
#include <cstring>
#include <thread>
#include <vector>

#include "mbq_layout.h"

namespace mbq {

// run f(row_begin, row_end) over [0, rows) on up to `threads` host threads
template <class F>
inline void parallel_rows(int64_t rows, int threads, F f) {
    int hw = (int)std::thread::hardware_concurrency();
    if (threads <= 0) threads = hw > 0 ? hw : 1;
    threads = (int)std::min<int64_t>(threads, std::max<int64_t>(1, rows / 64));
    if (threads <= 1) {
        f(0, rows);
        return;
    }
    std::vector<std::thread> pool;
    const int64_t step = (rows + threads - 1) / threads;
    for (int i = 0; i < threads; ++i) {
        const int64_t a = i * step, b = std::min(rows, a + step);
        if (a >= b) break;
        pool.emplace_back(f, a, b);
    }
    for (auto& th : pool) th.join();
}

// Q6_K: the 6-bit quant i (0..31) of unit j (0..7) of a super-block, from the file's ql / qh bytes
// (reference src/mashbox/ops/reference.py:164-173: value 128g + 32r + i takes nibble r / 2 of ql[64g + 32 (r % 2) + i]
// and bits 2r, 2r + 1 of qh[32g + i])
inline uint32_t q6k_file_quant(const uint8_t* blk, int j, int i) {
    const int g = j >> 2, r = j & 3;
    const uint32_t lo = (blk[64 * g + 32 * (r & 1) + i] >> (4 * (r >> 1))) & 15u;
    const uint32_t hi = (blk[128 + 32 * g + i] >> (2 * r)) & 3u;
    return lo | (hi << 4);
}

// Q4_K planes (row-major, or T_Q4KT tiles): offset in the qs plane of byte b of row n's quants (b = value / 2; a
// 16-byte unit never straddles a 64-byte tile row), and in the meta plane of super-block sb's header
inline int64_t q4k_qs_at(int t, int64_t n, int64_t K, int64_t b) {
    return t == T_Q4KT ? q4kt_off(n, K) + (b / 64) * 1024 + b % 64 : n * (K / 2) + b;
}
inline int64_t q4k_meta_at(int t, int64_t n, int64_t K, int64_t sb) {
    return t == T_Q4KT ? q4kt_meta_off(n, K) + sb * 256 : (n * (K / 256) + sb) * 16;
}

// Q8_0 planes (row-major, or T_Q8T tiles): offset of block b of row n's first quant in the qs plane (T_Q8T: quants
// 8g .. 8g + 7 of the block at + 16 g) and of its fp16 scale in the d plane
inline int64_t q8_qs_at(int t, int64_t n, int64_t K, int64_t b) {
    return t == T_Q8T ? i8t_off(n, K, (32 * b) & ~int64_t(63)) + q8t_byte((int)((32 * b) % 64)) : n * K + 32 * b;
}
inline int64_t q8_d_at(int t, int64_t n, int64_t K, int64_t b) {
    return t == T_Q8T ? q8t_d_off(n, K) + (b / 2) * 64 + (b % 2) * 2 : (n * (K / 32) + b) * 2;
}

// Q4_0 planes (row-major, or T_Q40T tiles): block b of row n's 16-byte unit in the qs plane, and its fp16 scale
inline int64_t q40_q_at(int t, int64_t n, int64_t K, int64_t b) {
    return t == T_Q40T ? q40t_off(n, K) + (b >> 2) * 1024 + (b & 3) * 16 : n * (K / 2) + b * 16;
}
inline int64_t q40_d_at(int t, int64_t n, int64_t K, int64_t b) {
    return t == T_Q40T ? q40t_d_off(n, K) + (b >> 2) * 128 + (b & 3) * 2 : (n * (K / 32) + b) * 2;
}

// Q5_K planes (row-major, or T_Q5KT tiles) of row n: unit j of super-block b in the qs and qh planes, and the
// super-block's header
inline int64_t q5k_q_at(int t, int64_t n, int64_t K, int64_t b, int j) {
    return t == T_Q5KT ? q4kt_off(n, K) + (2 * b + (j >> 2)) * 1024 + (j & 3) * 16 : n * (K / 2) + b * 128 + j * 16;
}
inline int64_t q5k_h_at(int t, int64_t n, int64_t K, int64_t b, int j) {
    return t == T_Q5KT ? q5kt_h_off(n, K) + (2 * b + (j >> 2)) * 256 + (j & 3) * 4 : n * (K / 8) + b * 32 + j * 4;
}
inline int64_t q5k_meta_at(int t, int64_t n, int64_t K, int64_t b) {
    return t == T_Q5KT ? q4kt_meta_off(n, K) + b * 256 : (n * (K / 256) + b) * 16;
}

// Q6_K planes (row-major, or T_Q6KT tiles) of row n: unit j of super-block b in the qs and qh planes, half h (8 bytes)
// of the super-block's 16 sub-block scales, and its fp16 scale
struct Q6kAt {
    int t;
    int64_t n, K;
    uint8_t* p;
    const Layout& L;
    bool tiled() const { return t == T_Q6KT; }
    uint8_t* q(int64_t b, int j) const {
        return p + L.qs_off + (tiled() ? q4kt_off(n, K) + (2 * b + (j >> 2)) * 1024 + (j & 3) * 16 : n * (K / 2) + b * 128 + j * 16);
    }
    uint8_t* h(int64_t b, int j) const {
        return p + L.hi_off + (tiled() ? q6kt_h_off(n, K) + (2 * b + (j >> 2)) * 512 + (j & 3) * 8 : n * (K / 4) + b * 64 + j * 8);
    }
    uint8_t* sc(int64_t b, int hf) const {
        return p + L.sc_off + (tiled() ? q6kt_s_off(n, K) + (2 * b + hf) * 128 : n * (K / 16) + b * 16 + 8 * hf);
    }
    uint8_t* d(int64_t b) const { return p + L.d_off + (tiled() ? q6kt_d_off(n, K) + b * 32 : (n * (K / 256) + b) * 2); }
};

inline void repack_rows(int t, const uint8_t* raw, int64_t K, uint8_t* planes, const Layout& L, int64_t r0, int64_t r1) {
    const int64_t nb = K / block_values(t), bb = block_bytes(t), rb = nb * bb;
    for (int64_t n = r0; n < r1; ++n) {
        const uint8_t* row = raw + n * rb;
        if (q5k_like(t)) {
            // reference src/mashbox/ops/reference.py:150-159: value 32j + i takes nibble j % 2 of qs[32 (j / 2) + i]
            // (qs at byte 48) and bit j of qh[i] (qh at byte 16); T_Q5KT: at the tile offsets
            for (int64_t b = 0; b < nb; ++b) {
                const uint8_t* src = row + b * bb;
                memcpy(planes + L.sc_off + q5k_meta_at(t, n, K, b), src, 16);
                for (int j = 0; j < 8; ++j) {
                    uint8_t* qu = planes + L.qs_off + q5k_q_at(t, n, K, b, j);
                    uint8_t* hu = planes + L.hi_off + q5k_h_at(t, n, K, b, j);
                    memset(qu, 0, 16);
                    memset(hu, 0, 4);
                    for (int i = 0; i < 32; ++i) {
                        const uint32_t lo = (src[48 + 32 * (j >> 1) + i] >> (4 * (j & 1))) & 15u;
                        const uint32_t hi = (src[16 + i] >> j) & 1u;
                        int lb, lbit, hb, hbit;
                        q5k_slot(i, &lb, &lbit, &hb, &hbit);
                        qu[lb] |= (uint8_t)(lo << lbit);
                        hu[hb] |= (uint8_t)(hi << hbit);
                    }
                }
            }
        } else if (q6k_like(t)) {
            // Q6_K, row-major or in 16-row tiles (T_Q6KT): the same bytes of each plane at the layout's offsets
            const Q6kAt at{t, n, K, planes, L};
            for (int64_t b = 0; b < nb; ++b) {
                const uint8_t* src = row + b * bb;
                memcpy(at.sc(b, 0), src + 192, 8);
                memcpy(at.sc(b, 1), src + 200, 8);
                memcpy(at.d(b), src + 208, 2);
                for (int j = 0; j < 8; ++j) {
                    uint8_t* qu = at.q(b, j);
                    uint8_t* hu = at.h(b, j);
                    memset(qu, 0, 16);
                    memset(hu, 0, 8);
                    for (int i = 0; i < 32; ++i) {
                        const uint32_t v = q6k_file_quant(src, j, i);
                        int lb, lbit, hb, hbit;
                        q6k_slot(i, &lb, &lbit, &hb, &hbit);
                        qu[lb] |= (uint8_t)((v & 15u) << lbit);
                        hu[hb] |= (uint8_t)((v >> 4) << hbit);
                    }
                }
            }
        } else if (q8_like(t)) {
            // Q8_0, row-major or in 16-row tiles (T_Q8T: a block's 32 quants in four 8-byte groups 16 bytes apart)
            for (int64_t b = 0; b < nb; ++b) {
                memcpy(planes + L.sc_off + q8_d_at(t, n, K, b), row + b * bb, 2);
                for (int g = 0; g < (t == T_Q8T ? 4 : 1); ++g)
                    memcpy(planes + L.qs_off + q8_qs_at(t, n, K, b) + 16 * g, row + b * bb + 2 + 8 * g, t == T_Q8T ? 8 : 32);
            }
        } else if (q40_like(t)) {
            // reference src/mashbox/ops/reference.py:66-70: value i (i < 16) is the low nibble of qs[i], value 16 + i
            // its high nibble (qs at byte 2); T_Q40T: at the tile offsets
            for (int64_t b = 0; b < nb; ++b) {
                const uint8_t* src = row + b * bb;
                memcpy(planes + L.sc_off + q40_d_at(t, n, K, b), src, 2);
                uint32_t unit[4] = {0, 0, 0, 0};
                for (int i = 0; i < 32; ++i) {
                    const uint32_t v = (src[2 + (i & 15)] >> (4 * (i >> 4))) & 15u;
                    int dw, bit;
                    q4k_slot(i, &dw, &bit);
                    unit[dw] |= v << bit;
                }
                memcpy(planes + L.qs_off + q40_q_at(t, n, K, b), unit, 16);  // little-endian host, as the GPU
            }
        } else {
            // Q4_K, row-major or in 16-row tiles (T_Q4KT): the same units and headers at the layout's offsets
            for (int64_t b = 0; b < nb; ++b) {
                const uint8_t* src = row + b * bb;
                memcpy(planes + L.sc_off + q4k_meta_at(t, n, K, b), src, 16);
                const uint8_t* qs = src + 16;
                for (int j = 0; j < 8; ++j) {
                    uint32_t unit[4] = {0, 0, 0, 0};
                    for (int i = 0; i < 32; ++i) {
                        const uint8_t byte = qs[32 * (j >> 1) + i];
                        const uint32_t v = (j & 1) ? (byte >> 4) : (byte & 15u);
                        int dw, bit;
                        q4k_slot(i, &dw, &bit);
                        unit[dw] |= v << bit;
                    }
                    memcpy(planes + L.qs_off + q4k_qs_at(t, n, K, b * 128 + j * 16), unit, 16);  // little-endian host, as the GPU
                }
            }
        }
    }
}

// T_Q4KT: the rows of the last tile past N, zero (quants and headers)
inline void q4kt_zero_pad_rows(int64_t N, int64_t K, uint8_t* planes, const Layout& L) {
    for (int64_t n = N; n < (N + 15) / 16 * 16; ++n) {
        for (int64_t b = 0; b < K / 2; b += 64) memset(planes + L.qs_off + q4k_qs_at(T_Q4KT, n, K, b), 0, 64);
        for (int64_t sb = 0; sb < K / 256; ++sb) memset(planes + L.sc_off + q4k_meta_at(T_Q4KT, n, K, sb), 0, 16);
    }
}

inline void unpack_rows(int t, const uint8_t* planes, int64_t K, uint8_t* raw, const Layout& L, int64_t r0, int64_t r1) {
    const int64_t nb = K / block_values(t), bb = block_bytes(t), rb = nb * bb;
    for (int64_t n = r0; n < r1; ++n) {
        uint8_t* row = raw + n * rb;
        if (q5k_like(t)) {
            for (int64_t b = 0; b < nb; ++b) {
                uint8_t* dst = row + b * bb;
                memcpy(dst, planes + L.sc_off + q5k_meta_at(t, n, K, b), 16);
                memset(dst + 16, 0, 160);
                for (int j = 0; j < 8; ++j) {
                    const uint8_t* qu = planes + L.qs_off + q5k_q_at(t, n, K, b, j);
                    const uint8_t* hu = planes + L.hi_off + q5k_h_at(t, n, K, b, j);
                    for (int i = 0; i < 32; ++i) {
                        int lb, lbit, hb, hbit;
                        q5k_slot(i, &lb, &lbit, &hb, &hbit);
                        const uint8_t lo = (qu[lb] >> lbit) & 15u, hi = (hu[hb] >> hbit) & 1u;
                        dst[48 + 32 * (j >> 1) + i] |= (uint8_t)(lo << (4 * (j & 1)));
                        dst[16 + i] |= (uint8_t)(hi << j);
                    }
                }
            }
        } else if (q6k_like(t)) {
            const Q6kAt at{t, n, K, const_cast<uint8_t*>(planes), L};
            for (int64_t b = 0; b < nb; ++b) {
                uint8_t* dst = row + b * bb;
                memset(dst, 0, 192);
                memcpy(dst + 192, at.sc(b, 0), 8);
                memcpy(dst + 200, at.sc(b, 1), 8);
                memcpy(dst + 208, at.d(b), 2);
                for (int j = 0; j < 8; ++j) {
                    const uint8_t* qu = at.q(b, j);
                    const uint8_t* hu = at.h(b, j);
                    const int g = j >> 2, r = j & 3;
                    for (int i = 0; i < 32; ++i) {
                        int lb, lbit, hb, hbit;
                        q6k_slot(i, &lb, &lbit, &hb, &hbit);
                        const uint8_t lo = (qu[lb] >> lbit) & 15u, hi = (hu[hb] >> hbit) & 3u;
                        dst[64 * g + 32 * (r & 1) + i] |= (uint8_t)(lo << (4 * (r >> 1)));
                        dst[128 + 32 * g + i] |= (uint8_t)(hi << (2 * r));
                    }
                }
            }
        } else if (q8_like(t)) {
            for (int64_t b = 0; b < nb; ++b) {
                memcpy(row + b * bb, planes + L.sc_off + q8_d_at(t, n, K, b), 2);
                for (int g = 0; g < (t == T_Q8T ? 4 : 1); ++g)
                    memcpy(row + b * bb + 2 + 8 * g, planes + L.qs_off + q8_qs_at(t, n, K, b) + 16 * g, t == T_Q8T ? 8 : 32);
            }
        } else if (q40_like(t)) {
            for (int64_t b = 0; b < nb; ++b) {
                uint8_t* dst = row + b * bb;
                memcpy(dst, planes + L.sc_off + q40_d_at(t, n, K, b), 2);
                memset(dst + 2, 0, 16);
                uint32_t unit[4];
                memcpy(unit, planes + L.qs_off + q40_q_at(t, n, K, b), 16);
                for (int i = 0; i < 32; ++i) {
                    int dw, bit;
                    q4k_slot(i, &dw, &bit);
                    dst[2 + (i & 15)] |= (uint8_t)(((unit[dw] >> bit) & 15u) << (4 * (i >> 4)));
                }
            }
        } else {
            for (int64_t b = 0; b < nb; ++b) {
                uint8_t* dst = row + b * bb;
                memcpy(dst, planes + L.sc_off + q4k_meta_at(t, n, K, b), 16);
                uint8_t* qs = dst + 16;
                memset(qs, 0, 128);
                for (int j = 0; j < 8; ++j) {
                    uint32_t unit[4];
                    memcpy(unit, planes + L.qs_off + q4k_qs_at(t, n, K, b * 128 + j * 16), 16);
                    for (int i = 0; i < 32; ++i) {
                        int dw, bit;
                        q4k_slot(i, &dw, &bit);
                        const uint8_t v = (unit[dw] >> bit) & 15u;
                        qs[32 * (j >> 1) + i] |= (j & 1) ? (uint8_t)(v << 4) : v;
                    }
                }
            }
        }
    }
}

// calls f(offset, bytes) on every run of alignment padding between and after the planes; false if f fails
template <class F>
inline bool for_each_gap(const Layout& L, F f) {
    const int64_t ends[4][2] = {{L.qs_off + L.qs_bytes, L.hi_off}, {L.hi_off + L.hi_bytes, L.sc_off},
                                {L.sc_off + L.sc_bytes, L.d_off}, {L.d_off + L.d_bytes, L.total}};
    for (const auto& e : ends)
        if (e[1] > e[0] && !f(e[0], e[1] - e[0])) return false;
    return true;
}

// tiled int8 planes (mbq_layout.h): 16-row tiles [t0, t1) from the row-major (N, K) quants and (N,) scales; padding
// rows and columns zero
inline void i8t_pack_tiles(const int8_t* q, const float* s, int64_t N, int64_t K, uint8_t* planes, const Layout& L,
                           int64_t t0, int64_t t1) {
    const int64_t kc_n = (K + 63) / 64;
    for (int64_t rt = t0; rt < t1; ++rt) {
        for (int64_t kc = 0; kc < kc_n; ++kc) {
            uint8_t* blk = planes + L.qs_off + (rt * kc_n + kc) * 1024;
            for (int r = 0; r < 16; ++r) {
                const int64_t row = rt * 16 + r, c0 = kc * 64, n = row < N ? std::min<int64_t>(64, K - c0) : 0;
                if (n > 0) memcpy(blk + r * 64, q + row * K + c0, (size_t)n);
                if (n < 64) memset(blk + r * 64 + std::max<int64_t>(n, 0), 0, (size_t)(64 - std::max<int64_t>(n, 0)));
            }
        }
        for (int r = 0; r < 16; ++r) {
            const int64_t row = rt * 16 + r;
            const float v = row < N ? s[row] : 0.f;
            memcpy(planes + L.sc_off + row * 4, &v, 4);
        }
    }
}

inline void i8t_unpack_tiles(const uint8_t* planes, int64_t N, int64_t K, int8_t* q, float* s, const Layout& L,
                             int64_t t0, int64_t t1) {
    const int64_t kc_n = (K + 63) / 64;
    for (int64_t rt = t0; rt < t1; ++rt)
        for (int r = 0; r < 16; ++r) {
            const int64_t row = rt * 16 + r;
            if (row >= N) continue;
            for (int64_t kc = 0; kc < kc_n; ++kc)
                memcpy(q + row * K + kc * 64, planes + L.qs_off + (rt * kc_n + kc) * 1024 + r * 64, (size_t)std::min<int64_t>(64, K - kc * 64));
            memcpy(s + row, planes + L.sc_off + row * 4, 4);
        }
}

// whole weights: the padding zeroed, then the rows (16-row tiles for int8) on up to `threads` host threads (0: every
// hardware thread). The caller checks the shape and the buffer sizes.
inline void repack_host(int t, const uint8_t* raw, int64_t rows, int64_t cols, uint8_t* planes, int threads) {
    const Layout L = layout(t, rows, cols);
    if (t == T_Q8T || t == T_Q6KT || t == T_Q5KT || t == T_Q40T) memset(planes, 0, (size_t)L.total);   // padding rows (Q8_0: the half chunk past K)
    for_each_gap(L, [&](int64_t off, int64_t n) { memset(planes + off, 0, (size_t)n); return true; });
    parallel_rows(rows, threads, [&](int64_t a, int64_t b) { repack_rows(t, raw, cols, planes, L, a, b); });
    if (t == T_Q4KT) q4kt_zero_pad_rows(rows, cols, planes, L);
}

inline void unpack_host(int t, const uint8_t* planes, int64_t rows, int64_t cols, uint8_t* raw, int threads) {
    const Layout L = layout(t, rows, cols);
    parallel_rows(rows, threads, [&](int64_t a, int64_t b) { unpack_rows(t, planes, cols, raw, L, a, b); });
}

inline void i8t_repack_host(const int8_t* q, const float* s, int64_t rows, int64_t cols, uint8_t* planes, int threads) {
    const Layout L = layout(T_I8T, rows, cols);
    for_each_gap(L, [&](int64_t off, int64_t n) { memset(planes + off, 0, (size_t)n); return true; });
    parallel_rows((rows + 15) / 16, threads, [&](int64_t a, int64_t b) { i8t_pack_tiles(q, s, rows, cols, planes, L, a, b); });
}

inline void i8t_unpack_host(const uint8_t* planes, int64_t rows, int64_t cols, int8_t* q, float* s, int threads) {
    const Layout L = layout(T_I8T, rows, cols);
    parallel_rows((rows + 15) / 16, threads, [&](int64_t a, int64_t b) { i8t_unpack_tiles(planes, rows, cols, q, s, L, a, b); });
}

}  // namespace mbq
