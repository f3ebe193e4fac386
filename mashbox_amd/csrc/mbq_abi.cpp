// The C ABI of libmbq.so (declared in include/mbq.h): argument checks, the host repack, and dispatch to the kernels.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <string>
#include <thread>
#include <vector>

#include "../../include/mbq.h"
#include "mbq_launch.h"
#include "mbq_layout.h"

namespace mbq {

static thread_local std::string g_error;

int set_error(int code, const char* fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof buf, fmt, ap);
    va_end(ap);
    g_error = buf;
    return code;
}

static bool is_type(int t) { return t == T_Q8_0 || t == T_Q4_0 || kquant(t); }

static bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

// shape rules shared by every entry point of a ggml type
static int check_shape(int t, int64_t rows, int64_t cols) {
    if (!is_type(t)) return set_error(MBQ_BAD_ARG, "ggml type %d has no kernel planes (Q4_0 = 2, Q8_0 = 8, Q4_K = 12, Q5_K = 13, Q6_K = 14)", t);
    if (rows <= 0 || cols <= 0) return set_error(MBQ_BAD_ARG, "shape (%lld, %lld) is empty", (long long)rows, (long long)cols);
    if (cols % block_values(t))
        return set_error(MBQ_BAD_ARG, "a row of %lld values is not a multiple of the block size %d", (long long)cols,
                         block_values(t));
    if (rows > INT32_MAX || cols > INT32_MAX) return set_error(MBQ_BAD_ARG, "shape (%lld, %lld) too large", (long long)rows, (long long)cols);
    return 0;
}

// shape rules of an entry point that takes kernel planes: a ggml type's, or the tiled int8 planes' (T_I8T: any rows, a
// row of whole 16-value units)
static int check_planes_shape(int t, int64_t rows, int64_t cols) {
    if (t != T_I8T) return check_shape(t, rows, cols);
    if (rows <= 0 || cols <= 0 || rows > INT32_MAX || cols > INT32_MAX)
        return set_error(MBQ_BAD_ARG, "int8 shape (%lld, %lld)", (long long)rows, (long long)cols);
    if (cols % 16) return set_error(MBQ_BAD_ARG, "int8 K = %lld must be a multiple of 16", (long long)cols);
    return 0;
}

// run f(row_begin, row_end) over [0, rows) on up to `threads` host threads
template <class F>
static void parallel_rows(int64_t rows, int threads, F f) {
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
static inline uint32_t q6k_file_quant(const uint8_t* blk, int j, int i) {
    const int g = j >> 2, r = j & 3;
    const uint32_t lo = (blk[64 * g + 32 * (r & 1) + i] >> (4 * (r >> 1))) & 15u;
    const uint32_t hi = (blk[128 + 32 * g + i] >> (2 * r)) & 3u;
    return lo | (hi << 4);
}

static void repack_rows(int t, const uint8_t* raw, int64_t K, uint8_t* planes, const Layout& L, int64_t r0, int64_t r1) {
    const int64_t nb = K / block_values(t), bb = block_bytes(t), rb = nb * bb;
    for (int64_t n = r0; n < r1; ++n) {
        const uint8_t* row = raw + n * rb;
        if (t == T_Q5_K) {
            // reference src/mashbox/ops/reference.py:150-159: value 32j + i takes nibble j % 2 of qs[32 (j / 2) + i]
            // (qs at byte 48) and bit j of qh[i] (qh at byte 16)
            uint8_t* q = planes + L.qs_off + n * (K / 2);
            uint8_t* h = planes + L.hi_off + n * (K / 8);
            uint8_t* meta = planes + L.sc_off + n * nb * 16;
            for (int64_t b = 0; b < nb; ++b) {
                const uint8_t* src = row + b * bb;
                memcpy(meta + b * 16, src, 16);
                for (int j = 0; j < 8; ++j) {
                    uint8_t* qu = q + b * 128 + j * 16;
                    uint8_t* hu = h + b * 32 + j * 4;
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
        } else if (t == T_Q6_K) {
            uint8_t* q = planes + L.qs_off + n * (K / 2);
            uint8_t* h = planes + L.hi_off + n * (K / 4);
            uint8_t* sc = planes + L.sc_off + n * (K / 16);
            uint8_t* d = planes + L.d_off + n * nb * 2;
            for (int64_t b = 0; b < nb; ++b) {
                const uint8_t* src = row + b * bb;
                memcpy(sc + b * 16, src + 192, 16);
                memcpy(d + b * 2, src + 208, 2);
                for (int j = 0; j < 8; ++j) {
                    uint8_t* qu = q + b * 128 + j * 16;
                    uint8_t* hu = h + b * 64 + j * 8;
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
        } else if (t == T_Q8_0) {
            uint8_t* q = planes + L.qs_off + n * K;
            uint8_t* d = planes + L.sc_off + n * nb * 2;
            for (int64_t b = 0; b < nb; ++b) {
                memcpy(d + b * 2, row + b * bb, 2);
                memcpy(q + b * 32, row + b * bb + 2, 32);
            }
        } else if (t == T_Q4_0) {
            // reference src/mashbox/ops/reference.py:66-70: value i (i < 16) is the low nibble of qs[i], value 16 + i
            // its high nibble (qs at byte 2)
            uint8_t* q = planes + L.qs_off + n * (K / 2);
            uint8_t* d = planes + L.sc_off + n * nb * 2;
            for (int64_t b = 0; b < nb; ++b) {
                const uint8_t* src = row + b * bb;
                memcpy(d + b * 2, src, 2);
                uint32_t unit[4] = {0, 0, 0, 0};
                for (int i = 0; i < 32; ++i) {
                    const uint32_t v = (src[2 + (i & 15)] >> (4 * (i >> 4))) & 15u;
                    int dw, bit;
                    q4k_slot(i, &dw, &bit);
                    unit[dw] |= v << bit;
                }
                memcpy(q + b * 16, unit, 16);  // little-endian host, as the GPU
            }
        } else {
            uint8_t* q = planes + L.qs_off + n * (K / 2);
            uint8_t* meta = planes + L.sc_off + n * nb * 16;
            for (int64_t b = 0; b < nb; ++b) {
                const uint8_t* src = row + b * bb;
                memcpy(meta + b * 16, src, 16);
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
                    memcpy(q + b * 128 + j * 16, unit, 16);  // little-endian host, as the GPU
                }
            }
        }
    }
}

static void unpack_rows(int t, const uint8_t* planes, int64_t K, uint8_t* raw, const Layout& L, int64_t r0, int64_t r1) {
    const int64_t nb = K / block_values(t), bb = block_bytes(t), rb = nb * bb;
    for (int64_t n = r0; n < r1; ++n) {
        uint8_t* row = raw + n * rb;
        if (t == T_Q5_K) {
            const uint8_t* q = planes + L.qs_off + n * (K / 2);
            const uint8_t* h = planes + L.hi_off + n * (K / 8);
            const uint8_t* meta = planes + L.sc_off + n * nb * 16;
            for (int64_t b = 0; b < nb; ++b) {
                uint8_t* dst = row + b * bb;
                memcpy(dst, meta + b * 16, 16);
                memset(dst + 16, 0, 160);
                for (int j = 0; j < 8; ++j) {
                    const uint8_t* qu = q + b * 128 + j * 16;
                    const uint8_t* hu = h + b * 32 + j * 4;
                    for (int i = 0; i < 32; ++i) {
                        int lb, lbit, hb, hbit;
                        q5k_slot(i, &lb, &lbit, &hb, &hbit);
                        const uint8_t lo = (qu[lb] >> lbit) & 15u, hi = (hu[hb] >> hbit) & 1u;
                        dst[48 + 32 * (j >> 1) + i] |= (uint8_t)(lo << (4 * (j & 1)));
                        dst[16 + i] |= (uint8_t)(hi << j);
                    }
                }
            }
        } else if (t == T_Q6_K) {
            const uint8_t* q = planes + L.qs_off + n * (K / 2);
            const uint8_t* h = planes + L.hi_off + n * (K / 4);
            const uint8_t* sc = planes + L.sc_off + n * (K / 16);
            const uint8_t* d = planes + L.d_off + n * nb * 2;
            for (int64_t b = 0; b < nb; ++b) {
                uint8_t* dst = row + b * bb;
                memset(dst, 0, 192);
                memcpy(dst + 192, sc + b * 16, 16);
                memcpy(dst + 208, d + b * 2, 2);
                for (int j = 0; j < 8; ++j) {
                    const uint8_t* qu = q + b * 128 + j * 16;
                    const uint8_t* hu = h + b * 64 + j * 8;
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
        } else if (t == T_Q8_0) {
            const uint8_t* q = planes + L.qs_off + n * K;
            const uint8_t* d = planes + L.sc_off + n * nb * 2;
            for (int64_t b = 0; b < nb; ++b) {
                memcpy(row + b * bb, d + b * 2, 2);
                memcpy(row + b * bb + 2, q + b * 32, 32);
            }
        } else if (t == T_Q4_0) {
            const uint8_t* q = planes + L.qs_off + n * (K / 2);
            const uint8_t* d = planes + L.sc_off + n * nb * 2;
            for (int64_t b = 0; b < nb; ++b) {
                uint8_t* dst = row + b * bb;
                memcpy(dst, d + b * 2, 2);
                memset(dst + 2, 0, 16);
                uint32_t unit[4];
                memcpy(unit, q + b * 16, 16);
                for (int i = 0; i < 32; ++i) {
                    int dw, bit;
                    q4k_slot(i, &dw, &bit);
                    dst[2 + (i & 15)] |= (uint8_t)(((unit[dw] >> bit) & 15u) << (4 * (i >> 4)));
                }
            }
        } else {
            const uint8_t* q = planes + L.qs_off + n * (K / 2);
            const uint8_t* meta = planes + L.sc_off + n * nb * 16;
            for (int64_t b = 0; b < nb; ++b) {
                uint8_t* dst = row + b * bb;
                memcpy(dst, meta + b * 16, 16);
                uint8_t* qs = dst + 16;
                memset(qs, 0, 128);
                for (int j = 0; j < 8; ++j) {
                    uint32_t unit[4];
                    memcpy(unit, q + b * 128 + j * 16, 16);
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
static bool for_each_gap(const Layout& L, F f) {
    const int64_t ends[4][2] = {{L.qs_off + L.qs_bytes, L.hi_off}, {L.hi_off + L.hi_bytes, L.sc_off},
                                {L.sc_off + L.sc_bytes, L.d_off}, {L.d_off + L.d_bytes, L.total}};
    for (const auto& e : ends)
        if (e[1] > e[0] && !f(e[0], e[1] - e[0])) return false;
    return true;
}

static int check_out(int out_dtype) {
    if (out_dtype != MBQ_OUT_F32 && out_dtype != MBQ_OUT_BF16)
        return set_error(MBQ_BAD_ARG, "out_dtype %d is neither MBQ_OUT_F32 nor MBQ_OUT_BF16", out_dtype);
    return 0;
}

// resolves the planes of one weight of a stack: host layer -> base pointer; device layer -> kernel argument
static int plane_args(int t, const uint8_t* planes, int64_t layer, const int32_t* layer_dev, int64_t nlayers, int64_t N,
                      int64_t K, Args* a) {
    if (int rc = check_planes_shape(t, N, K)) return rc;
    if (!planes || !aligned16(planes)) return set_error(MBQ_BAD_ARG, "planes pointer is NULL or not 16-byte aligned");
    if (nlayers < 1 || nlayers > INT32_MAX) return set_error(MBQ_BAD_ARG, "nlayers %lld must be >= 1", (long long)nlayers);
    if (layer_dev == nullptr && (layer < 0 || layer >= nlayers))
        return set_error(MBQ_BAD_ARG, "layer %lld outside the stack of %lld", (long long)layer, (long long)nlayers);
    const Layout L = layout(t, N, K);
    a->stride = L.total;
    a->wbytes = L.total;
    a->base = planes + (layer_dev ? 0 : layer * L.total);
    a->layer_dev = layer_dev;
    a->nlayers = (int)nlayers;
    a->sc_off = L.sc_off;
    a->hi_off = L.hi_off;
    a->d_off = L.d_off;
    a->srow = nullptr;
    a->N = N;
    a->K = K;
    return 0;
}

// tiled int8 planes (mbq_layout.h): 16-row tiles [t0, t1) from the row-major (N, K) quants and (N,) scales; padding
// rows and columns zero
static void i8t_pack_tiles(const int8_t* q, const float* s, int64_t N, int64_t K, uint8_t* planes, const Layout& L,
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

static void i8t_unpack_tiles(const uint8_t* planes, int64_t N, int64_t K, int8_t* q, float* s, const Layout& L,
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

// launch_matmul over row chunks of x whose bytes stay within one buffer resource's range (a chunk of rows is an
// independent product; every row is computed exactly as in one launch)
static int launch_rows(int t, Args a, hipStream_t s) {
    const int64_t rows = std::max<int64_t>(1, BUF_MAX_BYTES / (a.K * 2));
    if (a.M <= rows) return launch_matmul(t, a, s);
    const int64_t M = a.M;
    const uint16_t* x = a.x;
    uint8_t* y = static_cast<uint8_t*>(a.y);
    const int64_t ybytes = a.out_bf16 ? 2 : 4;
    for (int64_t m0 = 0; m0 < M; m0 += rows) {
        a.M = std::min(rows, M - m0);
        a.x = x + m0 * a.K;
        a.y = y + m0 * a.N * ybytes;
        if (int rc = launch_matmul(t, a, s)) return rc;
    }
    return 0;
}

}  // namespace mbq

using namespace mbq;

static int matmul_call(int t, const uint8_t* planes_dev, int64_t layer, const int32_t* layer_dev, int64_t nlayers,
                       const uint16_t* x_dev, int64_t M, int64_t N, int64_t K, void* y_dev, int out_dtype, void* stream,
                       bool noalloc);

extern "C" {

int mbq_version(void) { return 100; }

const char* mbq_last_error(void) { return g_error.c_str(); }

int mbq_has_type(int t) { return is_type(t) ? 1 : 0; }

int64_t mbq_row_bytes(int t, int64_t cols) {
    if (!is_type(t)) return set_error(MBQ_BAD_ARG, "ggml type %d has no kernel planes", t);
    if (cols < 0 || cols % block_values(t))
        return set_error(MBQ_BAD_ARG, "a row of %lld values is not a multiple of the block size %d", (long long)cols,
                         block_values(t));
    return cols / block_values(t) * block_bytes(t);
}

// Every kernel addresses one weight's planes through a buffer resource (32-bit offsets): weights whose planes exceed
// BUF_MAX_BYTES are refused at every batch size, so they are not covered. Activations are cut into row chunks within
// that range by mbq_matmul, so every batch size of a covered weight runs.
int mbq_covers(int t, int64_t rows, int64_t cols) {
    if (check_planes_shape(t, rows, cols) != 0) return 0;
    return layout(t, rows, cols).total <= BUF_MAX_BYTES ? 1 : 0;
}

int64_t mbq_plane_bytes(int t, int64_t rows, int64_t cols) {
    if (int rc = check_planes_shape(t, rows, cols)) return rc;
    return layout(t, rows, cols).total;
}

int mbq_repack_host(int t, const uint8_t* raw, int64_t rows, int64_t cols, uint8_t* planes_host, size_t cap, int threads) {
    if (int rc = check_shape(t, rows, cols)) return rc;
    if (!raw || !planes_host) return set_error(MBQ_BAD_ARG, "NULL buffer");
    const Layout L = layout(t, rows, cols);
    if (cap < (size_t)L.total) return set_error(MBQ_E_CAP, "planes buffer of %zu bytes < %lld", cap, (long long)L.total);
    for_each_gap(L, [&](int64_t off, int64_t n) { memset(planes_host + off, 0, (size_t)n); return true; });
    parallel_rows(rows, threads, [&](int64_t a, int64_t b) { repack_rows(t, raw, cols, planes_host, L, a, b); });
    return MBQ_OK;
}

int mbq_unpack_host(int t, const uint8_t* planes_host, int64_t rows, int64_t cols, uint8_t* raw, size_t cap) {
    if (int rc = check_shape(t, rows, cols)) return rc;
    if (!raw || !planes_host) return set_error(MBQ_BAD_ARG, "NULL buffer");
    const int64_t rb = cols / block_values(t) * block_bytes(t);
    if (cap < (size_t)(rows * rb)) return set_error(MBQ_E_CAP, "raw buffer of %zu bytes < %lld", cap, (long long)(rows * rb));
    const Layout L = layout(t, rows, cols);
    parallel_rows(rows, 0, [&](int64_t a, int64_t b) { unpack_rows(t, planes_host, cols, raw, L, a, b); });
    return MBQ_OK;
}

int mbq_repack_dev(int t, const uint8_t* raw_dev, int64_t rows, int64_t cols, uint8_t* planes_dev, void* stream) {
    if (int rc = check_shape(t, rows, cols)) return rc;
    if (!raw_dev || !planes_dev || !aligned16(planes_dev)) return set_error(MBQ_BAD_ARG, "NULL or misaligned buffer");
    const Layout L = layout(t, rows, cols);
    hipStream_t s = reinterpret_cast<hipStream_t>(stream);
    // zero the alignment padding, then write every plane byte
    int rc = 0;
    if (!for_each_gap(L, [&](int64_t off, int64_t n) { return (rc = launch_zero(planes_dev + off, n, s)) == 0; })) return rc;
    return launch_repack(t, raw_dev, rows, cols, planes_dev, L, s);
}

int mbq_int8_repack_host(const int8_t* q, const float* s, int64_t rows, int64_t cols, uint8_t* planes_host, size_t cap,
                         int threads) {
    if (int rc = check_planes_shape(T_I8T, rows, cols)) return rc;
    if (!q || !s || !planes_host) return set_error(MBQ_BAD_ARG, "NULL buffer");
    const Layout L = layout(T_I8T, rows, cols);
    if (cap < (size_t)L.total) return set_error(MBQ_E_CAP, "planes buffer of %zu bytes < %lld", cap, (long long)L.total);
    for_each_gap(L, [&](int64_t off, int64_t n) { memset(planes_host + off, 0, (size_t)n); return true; });
    parallel_rows((rows + 15) / 16, threads, [&](int64_t a, int64_t b) { i8t_pack_tiles(q, s, rows, cols, planes_host, L, a, b); });
    return MBQ_OK;
}

int mbq_int8_unpack_host(const uint8_t* planes_host, int64_t rows, int64_t cols, int8_t* q, float* s) {
    if (int rc = check_planes_shape(T_I8T, rows, cols)) return rc;
    if (!q || !s || !planes_host) return set_error(MBQ_BAD_ARG, "NULL buffer");
    const Layout L = layout(T_I8T, rows, cols);
    parallel_rows((rows + 15) / 16, 0, [&](int64_t a, int64_t b) { i8t_unpack_tiles(planes_host, rows, cols, q, s, L, a, b); });
    return MBQ_OK;
}

int mbq_int8_repack_dev(const int8_t* q_dev, const float* s_dev, int64_t rows, int64_t cols, uint8_t* planes_dev, void* stream) {
    if (int rc = check_planes_shape(T_I8T, rows, cols)) return rc;
    if (!q_dev || !s_dev || !planes_dev || !aligned16(q_dev) || !aligned16(planes_dev))
        return set_error(MBQ_BAD_ARG, "q, s or planes is NULL, or q / planes not 16-byte aligned");
    const Layout L = layout(T_I8T, rows, cols);
    hipStream_t st = reinterpret_cast<hipStream_t>(stream);
    int rc = 0;
    if (!for_each_gap(L, [&](int64_t off, int64_t n) { return (rc = launch_zero(planes_dev + off, n, st)) == 0; })) return rc;
    return launch_i8t_repack(q_dev, s_dev, rows, cols, planes_dev, L, st);
}

int mbq_matmul(int t, const uint8_t* planes_dev, int64_t layer, const int32_t* layer_dev, int64_t nlayers,
               const uint16_t* x_dev, int64_t M, int64_t N, int64_t K, void* y_dev, int out_dtype, void* stream) {
    return matmul_call(t, planes_dev, layer, layer_dev, nlayers, x_dev, M, N, K, y_dev, out_dtype, stream, false);
}

// mbq_matmul with every split-K partial in the library's static scratch array instead of the allocated workspace: the
// same plans, kernels and results, and no allocation on any call
int mbq_matmul_noalloc(int t, const uint8_t* planes_dev, int64_t layer, const int32_t* layer_dev, int64_t nlayers,
                       const uint16_t* x_dev, int64_t M, int64_t N, int64_t K, void* y_dev, int out_dtype, void* stream) {
    return matmul_call(t, planes_dev, layer, layer_dev, nlayers, x_dev, M, N, K, y_dev, out_dtype, stream, true);
}

}  // extern "C"

static int matmul_call(int t, const uint8_t* planes_dev, int64_t layer, const int32_t* layer_dev, int64_t nlayers,
                       const uint16_t* x_dev, int64_t M, int64_t N, int64_t K, void* y_dev, int out_dtype, void* stream,
                       bool noalloc) {
    Args a{};
    a.noalloc = noalloc;
    if (int rc = plane_args(t, planes_dev, layer, layer_dev, nlayers, N, K, &a)) return rc;
    if (int rc = check_out(out_dtype)) return rc;
    if (M < 0 || M > INT32_MAX) return set_error(MBQ_BAD_ARG, "M = %lld", (long long)M);
    if (M == 0) return MBQ_OK;
    if (!x_dev || !y_dev || !aligned16(x_dev) || !aligned16(y_dev))
        return set_error(MBQ_BAD_ARG, "x or y is NULL or not 16-byte aligned");
    a.x = x_dev;
    a.M = M;
    a.y = y_dev;
    a.out_bf16 = out_dtype == MBQ_OUT_BF16;
    return launch_rows(t, a, reinterpret_cast<hipStream_t>(stream));
}

extern "C" {

int mbq_dequant(int t, const uint8_t* planes_dev, int64_t layer, const int32_t* layer_dev, int64_t nlayers, int64_t N,
                int64_t K, float* w_dev, void* stream) {
    if (t == T_I8T) return set_error(MBQ_BAD_ARG, "int8 planes have no dequant: their values are the int8 quants, scaled per row after the dot");
    Args a{};
    if (int rc = plane_args(t, planes_dev, layer, layer_dev, nlayers, N, K, &a)) return rc;
    if (!w_dev || !aligned16(w_dev)) return set_error(MBQ_BAD_ARG, "w is NULL or not 16-byte aligned");
    return launch_dequant(t, a, w_dev, nullptr, 0, reinterpret_cast<hipStream_t>(stream));
}

int mbq_dequant_rows(int t, const uint8_t* planes_dev, int64_t layer, const int32_t* layer_dev, int64_t nlayers,
                     int64_t N, int64_t K, const int32_t* rows_dev, int64_t count, float* w_dev, void* stream) {
    if (t == T_I8T) return set_error(MBQ_BAD_ARG, "int8 planes have no dequant: their values are the int8 quants, scaled per row after the dot");
    Args a{};
    if (int rc = plane_args(t, planes_dev, layer, layer_dev, nlayers, N, K, &a)) return rc;
    if (count < 0 || count > INT32_MAX) return set_error(MBQ_BAD_ARG, "%lld rows", (long long)count);
    if (count == 0) return MBQ_OK;
    if (!rows_dev || !w_dev || !aligned16(w_dev)) return set_error(MBQ_BAD_ARG, "rows or w is NULL, or w not 16-byte aligned");
    return launch_dequant(t, a, w_dev, rows_dev, count, reinterpret_cast<hipStream_t>(stream));
}

int mbq_dequant_raw(int t, const uint8_t* raw_dev, int64_t rows, int64_t cols, float* w_dev, void* stream) {
    if (int rc = check_shape(t, rows, cols)) return rc;
    if (!raw_dev || !w_dev || !aligned16(w_dev)) return set_error(MBQ_BAD_ARG, "raw is NULL or w is NULL / not 16-byte aligned");
    return launch_dequant_raw(t, raw_dev, rows, cols, w_dev, reinterpret_cast<hipStream_t>(stream));
}

int mbq_int8_linear(const int8_t* q_dev, const float* s_dev, const uint16_t* x_dev, int64_t M, int64_t N, int64_t K,
                    void* y_dev, int out_dtype, void* stream) {
    if (int rc = check_out(out_dtype)) return rc;
    if (N <= 0 || K <= 0 || N > INT32_MAX || K > INT32_MAX || M < 0 || M > INT32_MAX)
        return set_error(MBQ_BAD_ARG, "shape M=%lld N=%lld K=%lld", (long long)M, (long long)N, (long long)K);
    if (K % 16) return set_error(MBQ_BAD_ARG, "int8 K = %lld must be a multiple of 16", (long long)K);
    if (M == 0) return MBQ_OK;
    if (!q_dev || !s_dev || !x_dev || !y_dev || !aligned16(q_dev) || !aligned16(x_dev) || !aligned16(y_dev))
        return set_error(MBQ_BAD_ARG, "q, s, x or y is NULL or q, x, y not 16-byte aligned");
    Args a{};
    a.base = reinterpret_cast<const uint8_t*>(q_dev);
    a.stride = 0;
    a.wbytes = N * K;
    a.layer_dev = nullptr;
    a.nlayers = 1;
    a.sc_off = 0;
    a.srow = s_dev;
    a.x = x_dev;
    a.M = M;
    a.N = N;
    a.K = K;
    a.y = y_dev;
    a.out_bf16 = out_dtype == MBQ_OUT_BF16;
    return launch_rows(T_INT8, a, reinterpret_cast<hipStream_t>(stream));
}

int mbq_int8_embed(const int8_t* q_dev, const float* s_dev, int64_t N, int64_t D, const int32_t* toks_dev, int64_t T,
                   void* y_dev, int out_dtype, void* stream) {
    if (int rc = check_out(out_dtype)) return rc;
    if (N <= 0 || D <= 0 || T < 0 || N > INT32_MAX || D > INT32_MAX || T > 65535 * 64LL)
        return set_error(MBQ_BAD_ARG, "embedding table (%lld, %lld), %lld tokens", (long long)N, (long long)D, (long long)T);
    if (T == 0) return MBQ_OK;
    if (!q_dev || !s_dev || !toks_dev || !y_dev) return set_error(MBQ_BAD_ARG, "q, s, toks or y is NULL");
    hipStream_t st = reinterpret_cast<hipStream_t>(stream);
    for (int64_t t0 = 0; t0 < T; t0 += 65535) {                     // grid.y holds at most 65535 tokens
        const int64_t n = std::min<int64_t>(65535, T - t0);
        void* y = reinterpret_cast<uint8_t*>(y_dev) + t0 * D * (out_dtype == MBQ_OUT_BF16 ? 2 : 4);
        if (int rc = launch_int8_embed(q_dev, s_dev, N, D, toks_dev + t0, n, y, out_dtype == MBQ_OUT_BF16, st)) return rc;
    }
    return MBQ_OK;
}

int mbq_gemm_plan(int t, int64_t M, int64_t N, int64_t K, int* kernel, int* bm, int* bn, int* splits) {
    if (!kernel || !bm || !bn || !splits) return set_error(MBQ_BAD_ARG, "NULL output");
    if (t == T_INT8) {
        if (N <= 0 || K <= 0 || N > INT32_MAX || K > INT32_MAX || K % 16) return set_error(MBQ_BAD_ARG, "int8 shape (%lld, %lld)", (long long)N, (long long)K);
    } else if (int rc = check_planes_shape(t, N, K)) {
        return rc;
    }
    if (M < 0 || M > INT32_MAX) return set_error(MBQ_BAD_ARG, "M = %lld", (long long)M);
    if (M == 0) {
        *kernel = *bm = *bn = *splits = 0;                                   // nothing is launched
        return MBQ_OK;
    }
    Args a{};
    a.M = std::min<int64_t>(M, std::max<int64_t>(1, BUF_MAX_BYTES / (K * 2)));   // the row chunk mbq_matmul launches
    a.N = N;
    a.K = K;
    a.wbytes = t == T_INT8 ? N * K : layout(t, N, K).total;
    if (a.M <= GEMV_MAX_M && gemv_runs(t, a)) {
        *kernel = *bm = *bn = *splits = 0;
        return MBQ_OK;
    }
    return gemm_plan(t, a, kernel, bm, bn, splits);
}

int mbq_force_gemm_plan(int kernel, int bm, int bn, int splits) { return force_gemm_plan(kernel, bm, bn, splits); }

}  // extern "C"
