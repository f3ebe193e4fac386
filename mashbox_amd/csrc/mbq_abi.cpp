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
#include "mbq_host_repack.h"
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

// the ggml types with kernel planes
static bool is_type(int t) { return t == T_Q8_0 || t == T_Q4_0 || t == T_Q4_K || t == T_Q5_K || t == T_Q6_K; }
// plane types made from a ggml type's blocks: the ggml types' own, and each in 16-row tiles
static bool is_block_planes(int t) { return is_type(t) || t == T_Q4KT || t == T_Q8T || t == T_Q6KT || t == T_Q5KT || t == T_Q40T; }

static bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

// shape rules shared by every entry point of a ggml type's blocks (and of the tiled planes made from Q4_K, Q6_K and
// Q8_0 blocks)
static int check_shape(int t, int64_t rows, int64_t cols) {
    if (!is_block_planes(t))
        return set_error(MBQ_BAD_ARG, "type %d has no kernel planes (Q4_0 = 2, Q8_0 = 8, Q4_K = 12, Q5_K = 13, Q6_K = 14, "
                                      "tiled Q8_0 = -10, tiled Q4_0 = -11, tiled Q4_K = -12, tiled Q5_K = -13, tiled Q6_K = -14)", t);
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

int mbq_has_raw_type(int t) { return raw_type(t) ? 1 : 0; }

int64_t mbq_row_bytes(int t, int64_t cols) {
    const GgmlBlock b = ggml_block(t);
    if (b.values == 0) return set_error(MBQ_BAD_ARG, "%d is not a ggml type id", t);
    if (cols < 0 || cols % b.values)
        return set_error(MBQ_BAD_ARG, "a row of %lld values is not a multiple of the block size %d", (long long)cols,
                         b.values);
    return cols / b.values * b.bytes;
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
    repack_host(t, raw, rows, cols, planes_host, threads);
    return MBQ_OK;
}

int mbq_unpack_host(int t, const uint8_t* planes_host, int64_t rows, int64_t cols, uint8_t* raw, size_t cap) {
    if (int rc = check_shape(t, rows, cols)) return rc;
    if (!raw || !planes_host) return set_error(MBQ_BAD_ARG, "NULL buffer");
    const int64_t rb = cols / block_values(t) * block_bytes(t);
    if (cap < (size_t)(rows * rb)) return set_error(MBQ_E_CAP, "raw buffer of %zu bytes < %lld", cap, (long long)(rows * rb));
    unpack_host(t, planes_host, rows, cols, raw, 0);
    return MBQ_OK;
}

int mbq_repack_dev(int t, const uint8_t* raw_dev, int64_t rows, int64_t cols, uint8_t* planes_dev, void* stream) {
    if (int rc = check_shape(t, rows, cols)) return rc;
    if (!raw_dev || !planes_dev || !aligned16(planes_dev)) return set_error(MBQ_BAD_ARG, "NULL or misaligned buffer");
    const Layout L = layout(t, rows, cols);
    hipStream_t s = reinterpret_cast<hipStream_t>(stream);
    // zero the alignment padding, then write every plane byte (tiles: the last tile's padding rows, and Q8_0's half-chunk
    // past K, too)
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
    i8t_repack_host(q, s, rows, cols, planes_host, threads);
    return MBQ_OK;
}

int mbq_int8_unpack_host(const uint8_t* planes_host, int64_t rows, int64_t cols, int8_t* q, float* s) {
    if (int rc = check_planes_shape(T_I8T, rows, cols)) return rc;
    if (!q || !s || !planes_host) return set_error(MBQ_BAD_ARG, "NULL buffer");
    i8t_unpack_host(planes_host, rows, cols, q, s, 0);
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
    if (!raw_type(t)) {
        if (ggml_block(t).values == 0) return set_error(MBQ_BAD_ARG, "dequant_raw takes a ggml type's blocks, not type %d", t);
        return set_error(MBQ_BAD_ARG, "dequant_raw: ggml type %d decodes through gguf-py's code books, which this library "
                                      "does not carry", t);
    }
    const int bv = ggml_block(t).values;
    if (rows <= 0 || cols <= 0) return set_error(MBQ_BAD_ARG, "shape (%lld, %lld) is empty", (long long)rows, (long long)cols);
    if (cols % bv)
        return set_error(MBQ_BAD_ARG, "a row of %lld values is not a multiple of the block size %d", (long long)cols, bv);
    if (rows > INT32_MAX || cols > INT32_MAX || rows * cols > ((int64_t)1 << 40))
        return set_error(MBQ_BAD_ARG, "shape (%lld, %lld) too large", (long long)rows, (long long)cols);
    if (!raw_dev || !w_dev || !aligned16(w_dev)) return set_error(MBQ_BAD_ARG, "raw is NULL or w is NULL / not 16-byte aligned");
    if (!is_type(t) && reinterpret_cast<uintptr_t>(raw_dev) % raw_block_align(t))
        return set_error(MBQ_BAD_ARG, "dequant_raw: the blocks must start at a multiple of %d bytes", raw_block_align(t));
    return launch_dequant_raw(t, raw_dev, rows, cols, w_dev, reinterpret_cast<hipStream_t>(stream));
}

int mbq_matmul_raw(int t, const uint8_t* raw_dev, const uint16_t* x_dev, int64_t M, int64_t N, int64_t K, void* y_dev,
                   int out_dtype, void* stream) {
    if (!raw_type(t) || is_type(t))
        return set_error(MBQ_BAD_ARG, "matmul_raw takes the file blocks of an exact-path type without kernel planes, not type %d", t);
    if (out_dtype != MBQ_OUT_F32 && out_dtype != MBQ_OUT_BF16) return set_error(MBQ_BAD_ARG, "out_dtype %d", out_dtype);
    if (M == 0) return MBQ_OK;
    if (M < 0 || M > 8)
        return set_error(MBQ_BAD_ARG, "matmul_raw: M = %lld (1-8 rows; more rows: mbq_dequant_raw and a GEMM)", (long long)M);
    if (N <= 0 || K <= 0 || N > INT32_MAX || K > INT32_MAX || M * K > INT32_MAX || M * N > INT32_MAX)
        return set_error(MBQ_BAD_ARG, "matmul_raw: shape (%lld, %lld, %lld)", (long long)M, (long long)N, (long long)K);
    if (K % 32 || K % ggml_block(t).values)
        return set_error(MBQ_BAD_ARG, "matmul_raw: K = %lld must be a multiple of 32 and of the block size %d", (long long)K,
                         ggml_block(t).values);
    if (!raw_dev || !x_dev || !y_dev || !aligned16(x_dev) || (reinterpret_cast<uintptr_t>(y_dev) & 3u))
        return set_error(MBQ_BAD_ARG, "matmul_raw: raw, x or y is NULL, x not 16-byte or y not 4-byte aligned");
    if (reinterpret_cast<uintptr_t>(raw_dev) % raw_block_align(t))
        return set_error(MBQ_BAD_ARG, "matmul_raw: the blocks must start at a multiple of %d bytes", raw_block_align(t));
    return launch_raw_gemv(t, raw_dev, x_dev, M, N, K, y_dev, out_dtype == MBQ_OUT_BF16 ? 1 : 0,
                           reinterpret_cast<hipStream_t>(stream));
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

int mbq_probe_read(const void* p_dev, int64_t bytes, void* sink_dev, void* stream) {
    if (!p_dev || !sink_dev || bytes < 0) return set_error(MBQ_BAD_ARG, "read probe: NULL buffer or negative size");
    return launch_probe_read(static_cast<const uint8_t*>(p_dev), bytes, static_cast<uint32_t*>(sink_dev),
                             reinterpret_cast<hipStream_t>(stream));
}

int mbq_probe_bf16(void* diff_dev, void* stream) {
    if (!diff_dev) return set_error(MBQ_BAD_ARG, "bf16 probe: NULL output");
    return launch_probe_bf16(static_cast<unsigned long long*>(diff_dev), reinterpret_cast<hipStream_t>(stream));
}

int mbq_probe_mfma(int iters, void* sink_dev, int64_t* flops, void* stream) {
    if (iters < 1 || !sink_dev || !flops) return set_error(MBQ_BAD_ARG, "MFMA probe: iters < 1 or NULL output");
    return launch_probe_mfma(iters, static_cast<float*>(sink_dev), flops, reinterpret_cast<hipStream_t>(stream));
}

}  // extern "C"
