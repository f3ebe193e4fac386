// gfx950 (CDNA4) kernels of the quantized linear: dequant, device repack and the matmul dispatch (decode GEMV:
// mbq_gemv.hip; weight-stream GEMM: mbq_wsgemm.hip; LDS-tile MFMA GEMM: mbq_gemm.hip).
//
// Semantics follow reference src/mashbox/ops/__init__.py:594-632 (qmatmul: x @ W.T, float32 accumulation) with the
// weights of reference src/mashbox/ops/reference.py:66-70 (Q4_0), :101-103 (Q8_0), :132-149 (Q4_K), :150-159 (Q5_K) and
// :164-173 (Q6_K), and the int8 per-channel linear of reference src/mashbox/models/qwen3_8_27b/model.py:72-82. Plane layouts: mbq_layout.h.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <algorithm>
#include <atomic>

#include "mbq_device.h"
#include "mbq_launch.h"
#include "mbq_layout.h"

namespace mbq {


// ------------------------------------------------------------------------------------------------------- dequant
// One thread per 16-byte unit (K-quants and Q4_0: 32 values; Q8_0: half a block, 16 values). Bit for bit the reference
// dequantization: Q8_0 v = f32(q) * d, Q4_0 v = d * f32(q - 8), Q4_K and Q5_K v = (d*sc)*q - dmin*m and
// Q6_K v = (d*sc)*(q - 32), whose products are exact in float32 (Q4_0 and Q6_K keep the reference's order of the
// operands, which fixes the sign of a zero).
// With `rows` (out_rows device row ids) it writes row r of w from weight row rows[r] (plus N when negative, clamped to
// [0, N - 1], as jax.numpy indexes): the rows of a lookup, without the rest of the weight.
template <int T>
__global__ __launch_bounds__(256) void dequant_kernel(const uint8_t* __restrict__ base, int64_t stride,
                                                      const int32_t* __restrict__ layer_dev, int nlayers, int64_t sc_off,
                                                      int64_t hi_off, int64_t d_off, int N, int K, float* __restrict__ w,
                                                      const int32_t* __restrict__ rows, int64_t out_rows) {
    const int64_t uw = unit32(T) ? 32 : 16;
    const int64_t units = out_rows * (K / uw);
    const int64_t g = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (g >= units) return;
    const int64_t lo = layer_offset(stride, layer_dev, nlayers);
    const bool ok = lo >= 0;
    base += ok ? lo : 0;
    const int64_t o = g / (K / uw), u = g % (K / uw);
    int64_t n = o;
    if (rows != nullptr) {
        n = rows[o];
        n = n < 0 ? n + N : n;
        n = n < 0 ? 0 : (n >= N ? N - 1 : n);
    }
    float* out = w + o * K + u * uw;
    if (!ok) {
        for (int i = 0; i < uw; ++i) out[i] = __builtin_nanf("");
        return;
    }
    if constexpr (q6k_like(T)) {
        // T_Q6KT: unit u of chunk u / 4 in each tiled plane
        constexpr bool TL = T == T_Q6KT;
        const u32x4 q = ld16(base + (TL ? q4kt_off(n, K) + (u >> 2) * 1024 + (u & 3) * 16 : n * (K >> 1) + u * 16));
        const u32x2 h = *reinterpret_cast<const u32x2*>(base + hi_off + (TL ? q6kt_h_off(n, K) + (u >> 2) * 512 + (u & 3) * 8 : n * (K >> 2) + u * 8));
        const uint16_t scp = *reinterpret_cast<const uint16_t*>(base + sc_off + (TL ? q6kt_s_off(n, K) + (u >> 2) * 128 + (u & 3) * 2 : n * (K >> 4) + u * 2));
        const float d = f16f(*reinterpret_cast<const uint16_t*>(base + d_off + (TL ? q6kt_d_off(n, K) + (u >> 3) * 32 : (n * (K >> 8) + (u >> 3)) * 2)));
        const float ds0 = d * (float)(int8_t)(scp & 0xFFu), ds1 = d * (float)(int8_t)(scp >> 8);
#pragma unroll
        for (int t = 0; t < 4; ++t) {
            uint32_t lo, hi;
            q6k_bytes(q[t], h[t >> 1], t, &lo, &hi);
            const float ds = t < 2 ? ds0 : ds1;
            float v[8];
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                v[e] = ds * (float)((int)((lo >> (8 * e)) & 0xFFu) - 32);
                v[4 + e] = ds * (float)((int)((hi >> (8 * e)) & 0xFFu) - 32);
            }
            st16(out + t * 8, u32x4{__float_as_uint(v[0]), __float_as_uint(v[1]), __float_as_uint(v[2]), __float_as_uint(v[3])});
            st16(out + t * 8 + 4, u32x4{__float_as_uint(v[4]), __float_as_uint(v[5]), __float_as_uint(v[6]), __float_as_uint(v[7])});
        }
    } else if constexpr (q5k_like(T)) {
        constexpr bool TL = T == T_Q5KT;                         // unit u of chunk u / 4 in each tiled plane
        const u32x4 q = ld16(base + (TL ? q4kt_off(n, K) + (u >> 2) * 1024 + (u & 3) * 16 : n * (K >> 1) + u * 16));
        const uint32_t h = *reinterpret_cast<const uint32_t*>(base + hi_off + (TL ? q5kt_h_off(n, K) + (u >> 2) * 256 + (u & 3) * 4 : n * (K >> 3) + u * 4));
        const u32x4 mt = ld16(base + sc_off + (TL ? q4kt_meta_off(n, K) + (u >> 3) * 256 : (n * (K >> 8) + (u >> 3)) * 16));
        uint32_t sc, mn;
        q4k_scale_min(mt[1], mt[2], mt[3], (int)(u & 7), &sc, &mn);
        const float dsc = f16f(mt[0]) * (float)sc;
        const float dm = f16f(mt[0] >> 16) * (float)mn;
#pragma unroll
        for (int t = 0; t < 4; ++t) {
            uint32_t lo, hi;
            q5k_bytes(q[t], h, t, &lo, &hi);
            float v[8];
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                v[e] = dsc * (float)((lo >> (8 * e)) & 0xFFu) - dm;
                v[4 + e] = dsc * (float)((hi >> (8 * e)) & 0xFFu) - dm;
            }
            st16(out + t * 8, u32x4{__float_as_uint(v[0]), __float_as_uint(v[1]), __float_as_uint(v[2]), __float_as_uint(v[3])});
            st16(out + t * 8 + 4, u32x4{__float_as_uint(v[4]), __float_as_uint(v[5]), __float_as_uint(v[6]), __float_as_uint(v[7])});
        }
    } else if constexpr (q40_like(T)) {
        constexpr bool TL = T == T_Q40T;                         // block u: unit u % 4 of chunk u / 4 in the tiles
        const u32x4 q = ld16(base + (TL ? q40t_off(n, K) + (u >> 2) * 1024 + (u & 3) * 16 : n * (K >> 1) + u * 16));
        const float d = f16f(*reinterpret_cast<const uint16_t*>(base + sc_off + (TL ? q40t_d_off(n, K) + (u >> 2) * 128 + (u & 3) * 2 : (n * (K >> 5) + u) * 2)));
#pragma unroll
        for (int t = 0; t < 4; ++t) {
            float v[8];
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                const int bit = 16 * (e & 1) + 4 * (e >> 1);
                v[e] = d * (float)((int)((q[t] >> bit) & 15u) - 8);
            }
            st16(out + t * 8, u32x4{__float_as_uint(v[0]), __float_as_uint(v[1]), __float_as_uint(v[2]), __float_as_uint(v[3])});
            st16(out + t * 8 + 4, u32x4{__float_as_uint(v[4]), __float_as_uint(v[5]), __float_as_uint(v[6]), __float_as_uint(v[7])});
        }
    } else if constexpr (q4k_like(T)) {
        const u32x4 q = T == T_Q4KT ? ld16(base + q4kt_off(n, K) + (u >> 2) * 1024 + (u & 3) * 16) : ld16(base + n * (K >> 1) + u * 16);
        const u32x4 mt = T == T_Q4KT ? ld16(base + sc_off + q4kt_meta_off(n, K) + (u >> 3) * 256)
                                     : ld16(base + sc_off + (n * (K >> 8) + (u >> 3)) * 16);
        uint32_t sc, mn;
        q4k_scale_min(mt[1], mt[2], mt[3], (int)(u & 7), &sc, &mn);
        const float dsc = f16f(mt[0]) * (float)sc;
        const float dm = f16f(mt[0] >> 16) * (float)mn;
#pragma unroll
        for (int t = 0; t < 4; ++t) {
            float v[8];
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                const int bit = 16 * (e & 1) + 4 * (e >> 1);
                v[e] = dsc * (float)((q[t] >> bit) & 15u) - dm;
            }
            st16(out + t * 8, u32x4{__float_as_uint(v[0]), __float_as_uint(v[1]), __float_as_uint(v[2]), __float_as_uint(v[3])});
            st16(out + t * 8 + 4, u32x4{__float_as_uint(v[4]), __float_as_uint(v[5]), __float_as_uint(v[6]), __float_as_uint(v[7])});
        }
    } else {
        // Q8_0 (T_Q8T: unit u's two 8-byte groups at their tile offsets; the scale of block u / 2 in the tiled d plane)
        u32x4 q;
        if constexpr (T == T_Q8T) {
            const uint8_t* c = base + i8t_off(n, K, (u >> 2) * 64) + q8t_byte((int)(u & 3) * 16);
            const u32x2 lo = *reinterpret_cast<const u32x2*>(c), hi = *reinterpret_cast<const u32x2*>(c + 16);
            q = u32x4{lo[0], lo[1], hi[0], hi[1]};
        } else {
            q = ld16(base + n * K + u * 16);
        }
        const float d = f16f(*reinterpret_cast<const uint16_t*>(
            base + sc_off + (T == T_Q8T ? q8t_d_off(n, K) + (u >> 2) * 64 + ((u >> 1) & 1) * 2 : (n * (K >> 5) + (u >> 1)) * 2)));
#pragma unroll
        for (int t = 0; t < 4; ++t) {
            float v[4];
#pragma unroll
            for (int e = 0; e < 4; ++e) v[e] = (float)(int8_t)(q[t] >> (8 * e)) * d;
            st16(out + t * 4, u32x4{__float_as_uint(v[0]), __float_as_uint(v[1]), __float_as_uint(v[2]), __float_as_uint(v[3])});
        }
    }
}

// ------------------------------------------------------------------------------------------------- raw dequant
static int check_launch(const char* what);
// The file's blocks (rows, row_bytes) -> float32 (rows, cols), without planes: reference src/mashbox/ops/reference.py
// :398-409 (dequant) with :66-70 (Q4_0), :101-103 (Q8_0), :132-149 (Q4_K), :150-159 (Q5_K) and :164-173 (Q6_K), the
// rebuild of the exact path. One thread per 32 values (a Q4_0 / Q8_0 block, a Q4_K / Q5_K sub-block, two Q6_K
// sub-blocks); the blocks are 18 / 34 / 144 / 176 / 210 bytes apart, so bytes are read one at a time.
template <int T>
__global__ __launch_bounds__(256) void dequant_raw_kernel(const uint8_t* __restrict__ raw, int64_t rows, int K,
                                                          float* __restrict__ w) {
    const int64_t units = rows * (K / 32);
    const int64_t g = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (g >= units) return;
    const int64_t n = g / (K / 32), u = g % (K / 32);
    float* out = w + n * K + u * 32;
    if constexpr (T == T_Q8_0) {
        const uint8_t* b = raw + (n * (K / 32) + u) * 34;
        const float d = f16f((uint32_t)b[0] | ((uint32_t)b[1] << 8));
        for (int i = 0; i < 32; ++i) out[i] = (float)(int8_t)b[2 + i] * d;
    } else if constexpr (T == T_Q4_0) {
        // value i < 16: low nibble of qs[i]; value 16 + i: its high nibble (qs at byte 2)
        const uint8_t* b = raw + (n * (K / 32) + u) * 18;
        const float d = f16f((uint32_t)b[0] | ((uint32_t)b[1] << 8));
        for (int i = 0; i < 32; ++i) out[i] = d * (float)((int)((b[2 + (i & 15)] >> (4 * (i >> 4))) & 15u) - 8);
    } else if constexpr (T == T_Q5_K) {
        // value 32j + i of the super-block: nibble j % 2 of qs[32 (j / 2) + i] (qs at byte 48), bit j of qh[i] (byte 16)
        const uint8_t* b = raw + (n * (K / 256) + (u >> 3)) * 176;
        const int j = (int)(u & 7);
        const uint32_t s0 = b[4] | (b[5] << 8) | (b[6] << 16) | ((uint32_t)b[7] << 24);
        const uint32_t s1 = b[8] | (b[9] << 8) | (b[10] << 16) | ((uint32_t)b[11] << 24);
        const uint32_t s2 = b[12] | (b[13] << 8) | (b[14] << 16) | ((uint32_t)b[15] << 24);
        uint32_t sc, mn;
        q4k_scale_min(s0, s1, s2, j, &sc, &mn);
        const float dsc = f16f((uint32_t)b[0] | ((uint32_t)b[1] << 8)) * (float)sc;      // exact
        const float dm = f16f((uint32_t)b[2] | ((uint32_t)b[3] << 8)) * (float)mn;       // exact
        for (int i = 0; i < 32; ++i) {
            const uint32_t q = ((b[48 + 32 * (j >> 1) + i] >> (4 * (j & 1))) & 15u) | (((b[16 + i] >> j) & 1u) << 4);
            out[i] = dsc * (float)q - dm;
        }
    } else if constexpr (T == T_Q6_K) {
        // value 32j + i of the super-block (j = 4g + r): nibble r / 2 of ql[64g + 32 (r % 2) + i], bits 2r, 2r + 1 of
        // qh[32g + i], sub-block scale sc[2j + i / 16]
        const uint8_t* b = raw + (n * (K / 256) + (u >> 3)) * 210;
        const int j = (int)(u & 7), g = j >> 2, r = j & 3;
        const float d = f16f((uint32_t)b[208] | ((uint32_t)b[209] << 8));
        const float ds0 = d * (float)(int8_t)b[192 + 2 * j], ds1 = d * (float)(int8_t)b[193 + 2 * j];
        for (int i = 0; i < 32; ++i) {
            const int q = ((b[64 * g + 32 * (r & 1) + i] >> (4 * (r >> 1))) & 15) | (((b[128 + 32 * g + i] >> (2 * r)) & 3) << 4);
            out[i] = (i < 16 ? ds0 : ds1) * (float)(q - 32);
        }
    } else {
        const uint8_t* b = raw + (n * (K / 256) + (u >> 3)) * 144;
        const int j = (int)(u & 7);
        const uint32_t s0 = b[4] | (b[5] << 8) | (b[6] << 16) | ((uint32_t)b[7] << 24);
        const uint32_t s1 = b[8] | (b[9] << 8) | (b[10] << 16) | ((uint32_t)b[11] << 24);
        const uint32_t s2 = b[12] | (b[13] << 8) | (b[14] << 16) | ((uint32_t)b[15] << 24);
        uint32_t sc, mn;
        q4k_scale_min(s0, s1, s2, j, &sc, &mn);
        const float dsc = f16f((uint32_t)b[0] | ((uint32_t)b[1] << 8)) * (float)sc;      // exact
        const float dm = f16f((uint32_t)b[2] | ((uint32_t)b[3] << 8)) * (float)mn;       // exact
        const uint8_t* q = b + 16 + 32 * (j >> 1);                   // sub-block 2g: low nibbles, 2g+1: high nibbles
        const int sh = (j & 1) * 4;
        for (int i = 0; i < 32; ++i) out[i] = dsc * (float)((q[i] >> sh) & 15u) - dm;
    }
}

// ---------------------------------------------------------------------------- raw dequant, the other ggml types
// The exact path's rebuild for the ggml types that have no kernel planes here (reference src/mashbox/ops/reference.py,
// the line ranges at each type below). Every value is exact or rounded once, as in the reference: a product of an fp16
// scale and a small integer is exact in float32, so d * q + m (Q4_1, Q5_1) and dl * q - ml (Q2_K) round once whether
// or not the compiler fuses them; IQ4_XS's (d * s) * k rounds once in the second product, in that order.
__device__ __forceinline__ uint32_t le16(const uint8_t* p) { return (uint32_t)p[0] | ((uint32_t)p[1] << 8); }
__device__ __forceinline__ uint32_t le32(const uint8_t* p) { return le16(p) | (le16(p + 2) << 16); }
// value i (0..31) of a 32-value block's 16 nibble bytes: low nibbles first, then the high ones
__device__ __forceinline__ uint32_t nib32(const uint8_t* qs, int i) { return (qs[i & 15] >> (4 * (i >> 4))) & 15u; }
// ggml's kvalues_iq4nl (reference :348) and the FP4 (E2M1) values doubled, kvalues_mxfp4 (reference :195)
__constant__ float kIQ4[16] = {-127, -104, -83, -65, -49, -35, -22, -10, 1, 13, 25, 38, 53, 69, 89, 113};
__constant__ float kFP4[16] = {0, 1, 2, 3, 4, 6, 8, 12, 0, -1, -2, -3, -4, -6, -8, -12};

// MXFP4 (reference :198-219): k * 2^(e - 128) with the float32 bits built from integers, so results below the normal
// range are exact subnormals, results past it inf, and zero codes +0
__device__ __forceinline__ float mxfp4_value(uint32_t e, uint32_t q) {
    const uint32_t c = q & 7u;
    const int odd = (int)((0x31313110u >> (4 * c)) & 15u);     // |k| = odd * 2^p for c = 0..7: odd 0 1 1 3 1 3 1 3,
    const int p = (int)((0x23120100u >> (4 * c)) & 15u);       //                                 p   0 0 1 0 2 1 3 2
    if (odd == 0) return 0.f;
    const int x = p + (int)e - 128, E = odd == 3 ? x + 1 : x;
    uint32_t bits;
    if (E > 127) bits = 0x7F800000u;
    else if (E < -126) bits = (uint32_t)odd << (x + 149);                                // x >= -128: a shift of 21-22
    else bits = ((uint32_t)(E + 127) << 23) | (odd == 3 ? 1u << 22 : 0u);
    return __uint_as_float(bits | (q >= 8 ? 0x80000000u : 0u));
}

// NVFP4's block scale (reference :222-227): unsigned E4M3 of bits 0-6 (bias 7), halved; the bytes 0x00 and 0x7F give 0
__device__ __forceinline__ float ue4m3_half(uint32_t x) {
    if (x == 0u || x == 0x7Fu) return 0.f;
    const uint32_t e = (x >> 3) & 15u;
    const float man = (float)(x & 7u);
    const float raw = e == 0 ? man * 0x1p-9f : (1.f + man * 0.125f) * __uint_as_float((e + 120u) << 23);
    return raw * 0.5f;
}

// TQ1_0's code of value v (reference :176-185): the base-3 digit k of a byte, ((byte * 3^k mod 256) * 3) >> 8, over
// bytes 0-31 (values 0-159, k = v / 32), 32-47 (values 160-239) and 48-51 (values 240-255)
__device__ __forceinline__ int tq1_code(const uint8_t* b, int v) {
    int k, byte;
    if (v < 160) k = v >> 5, byte = b[v & 31];
    else if (v < 240) k = (v - 160) >> 4, byte = b[32 + ((v - 160) & 15)];
    else k = (v - 240) >> 2, byte = b[48 + ((v - 240) & 3)];
    const int pw = k == 0 ? 1 : k == 1 ? 3 : k == 2 ? 9 : k == 3 ? 27 : 81;
    return ((((byte * pw) & 255) * 3) >> 8) - 1;
}

// the alignment every block start of type T has when the blocks start at an address of that alignment: the largest
// power of two (at most 4) dividing the block bytes (Q2_K 84, Q4_1 20, Q5_1 24, IQ4_XS 136, NVFP4 36, F32: 4; Q3_K
// 110, Q5_0 22, IQ4_NL 18, TQ1_0 54, TQ2_0 66, F16, BF16: 2; MXFP4 17: 1). Told to the compiler, it lets it merge the
// byte reads of a block into wider loads.
template <int T>
__host__ __device__ constexpr int raw_align() { return raw_block_align(T); }
static_assert(raw_block_align(T_Q2_K) == 4 && raw_block_align(T_Q3_K) == 2 && raw_block_align(T_MXFP4) == 1 &&
              raw_block_align(T_F32) == 4 && raw_block_align(T_BF16) == 2, "block alignments");
template <int T>
__device__ __forceinline__ const uint8_t* blk(const uint8_t* p) {
    return static_cast<const uint8_t*>(__builtin_assume_aligned(p, raw_align<T>()));
}

// Values 32u .. 32u + 31 of one weight row in the file's blocks of type T (row: the row's first byte, aligned to
// raw_align<T>()): a block of the 32-value types, half an NVFP4 block, a 32-value group of a 256-value super-block; for
// the float types (one value per block) 32 consecutive values
template <int T>
__device__ __forceinline__ void raw_unit(const uint8_t* __restrict__ row, int u, float v[32]) {
    if constexpr (T == T_F32 || T == T_F16 || T == T_BF16) {            // reference :372-381
        constexpr int ES = T == T_F32 ? 4 : 2;
        const uint8_t* p = blk<T>(row + (int64_t)ES * 32 * u);
        for (int i = 0; i < 32; ++i)
            v[i] = T == T_F32 ? __uint_as_float(le32(p + 4 * i)) : T == T_F16 ? f16f(le16(p + 2 * i))
                                                                       : __uint_as_float(le16(p + 2 * i) << 16);
    } else if constexpr (T == T_Q4_1) {                                  // reference :73-77
        const uint8_t* b = blk<T>(row + (int64_t)u * 20);
        const float d = f16f(le16(b)), m = f16f(le16(b + 2));
        for (int i = 0; i < 32; ++i) v[i] = d * (float)nib32(b + 4, i) + m;
    } else if constexpr (T == T_Q5_0 || T == T_Q5_1) {                   // reference :85-98
        constexpr bool ONE = T == T_Q5_1;
        const uint8_t* b = blk<T>(row + (int64_t)u * (ONE ? 24 : 22));
        const float d = f16f(le16(b)), m = ONE ? f16f(le16(b + 2)) : 0.f;
        const uint32_t qh = le32(b + (ONE ? 4 : 2));
        const uint8_t* qs = b + (ONE ? 8 : 6);
        for (int i = 0; i < 32; ++i) {
            const int q = (int)(nib32(qs, i) | (((qh >> i) & 1u) << 4));
            v[i] = ONE ? d * (float)q + m : d * (float)(q - 16);
        }
    } else if constexpr (T == T_IQ4_NL) {                                // reference :351-356
        const uint8_t* b = blk<T>(row + (int64_t)u * 18);
        const float d = f16f(le16(b));
        for (int i = 0; i < 32; ++i) v[i] = d * kIQ4[nib32(b + 2, i)];
    } else if constexpr (T == T_MXFP4) {                                 // reference :198-219
        const uint8_t* b = blk<T>(row + (int64_t)u * 17);
        for (int i = 0; i < 32; ++i) v[i] = mxfp4_value(b[0], nib32(b + 1, i));
    } else if constexpr (T == T_NVFP4) {                                 // reference :230-236
        // half h of the 64-value block: sub-blocks 2h, 2h + 1 of 16 (scale byte s; codes: the low nibbles of bytes
        // 4 + 8s .. 11 + 8s, then their high nibbles)
        const uint8_t* b = blk<T>(row + (int64_t)(u >> 1) * 36);
        const int h = u & 1;
        for (int i = 0; i < 32; ++i) {
            const int s = 2 * h + (i >> 4), ii = i & 15;
            const uint32_t byte = b[4 + 8 * s + (ii & 7)];
            v[i] = ue4m3_half(b[s]) * kFP4[ii < 8 ? byte & 15u : byte >> 4];
        }
    } else {
        // 256-value super-blocks: group j (values 32j .. 32j + 31) of super-block u / 8
        const int j = u & 7, hh = j >> 2, si = j & 3;
        if constexpr (T == T_Q2_K) {                                     // reference :106-114
            const uint8_t* b = blk<T>(row + (int64_t)(u >> 3) * 84);
            const float d = f16f(le16(b + 80)), dmin = f16f(le16(b + 82));
            for (int half = 0; half < 2; ++half) {                       // sub-block 2j + half of 16 values
                const uint32_t s = b[2 * j + half];
                const float dl = d * (float)(s & 15u), ml = dmin * (float)(s >> 4);
                for (int l = 0; l < 16; ++l) {
                    const int i = 16 * half + l;
                    v[i] = dl * (float)((b[16 + 32 * hh + i] >> (2 * si)) & 3u) - ml;
                }
            }
        } else if constexpr (T == T_Q3_K) {                              // reference :117-129
            const uint8_t* b = blk<T>(row + (int64_t)(u >> 3) * 110);
            const float d = f16f(le16(b + 108));
            for (int half = 0; half < 2; ++half) {
                const int sb = 2 * j + half;                             // scale: low 4 bits from bytes 96-103, high 2 from 104-107
                const uint32_t lo = sb < 8 ? (b[96 + sb] & 15u) : (b[96 + sb - 8] >> 4);
                const uint32_t hi = (b[104 + (sb & 3)] >> (2 * (sb >> 2))) & 3u;
                const float dl = d * (float)((int)(lo | (hi << 4)) - 32);
                for (int l = 0; l < 16; ++l) {
                    const int i = 16 * half + l;
                    const int q = (int)((b[32 + 32 * hh + i] >> (2 * si)) & 3u) - (((b[i] >> j) & 1u) ? 0 : 4);
                    v[i] = dl * (float)q;
                }
            }
        } else if constexpr (T == T_IQ4_XS) {                            // reference :359-369
            const uint8_t* b = blk<T>(row + (int64_t)(u >> 3) * 136);
            const uint32_t lo = (b[4 + (j >> 1)] >> (4 * (j & 1))) & 15u, hi = (le16(b + 2) >> (2 * j)) & 3u;
            const float dl = f16f(le16(b)) * (float)((int)(lo | (hi << 4)) - 32);
            for (int i = 0; i < 32; ++i) v[i] = dl * kIQ4[nib32(b + 8 + 16 * j, i)];
        } else if constexpr (T == T_TQ1_0) {                             // reference :176-185
            const uint8_t* b = blk<T>(row + (int64_t)(u >> 3) * 54);
            const float d = f16f(le16(b + 52));
            for (int i = 0; i < 32; ++i) v[i] = d * (float)tq1_code(b, 32 * j + i);
        } else {                                                         // TQ2_0, reference :188-192
            static_assert(T == T_TQ2_0, "a raw type");
            const uint8_t* b = blk<T>(row + (int64_t)(u >> 3) * 66);
            const float d = f16f(le16(b + 64));
            for (int i = 0; i < 32; ++i) v[i] = d * (float)((int)((b[32 * hh + i] >> (2 * si)) & 3u) - 1);
        }
    }
}

// bytes of one row of K values in the file's blocks of type T
template <int T>
__host__ __device__ constexpr int64_t raw_row_bytes(int64_t K) {
    return T == T_F32 ? 4 * K : (T == T_F16 || T == T_BF16) ? 2 * K : T == T_Q4_1 ? K / 32 * 20 : T == T_Q5_0 ? K / 32 * 22
         : T == T_Q5_1 ? K / 32 * 24 : T == T_IQ4_NL ? K / 32 * 18 : T == T_MXFP4 ? K / 32 * 17 : T == T_NVFP4 ? K / 64 * 36
         : T == T_Q2_K ? K / 256 * 84 : T == T_Q3_K ? K / 256 * 110 : T == T_IQ4_XS ? K / 256 * 136
         : T == T_TQ1_0 ? K / 256 * 54 : K / 256 * 66;
}

// One thread per 32 values, as dequant_raw_kernel
template <int T>
__global__ __launch_bounds__(256) void dequant_raw_more_kernel(const uint8_t* __restrict__ raw, int64_t rows, int K,
                                                               float* __restrict__ w) {
    const int64_t units = rows * (K / 32);
    const int64_t g = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (g >= units) return;
    const int64_t n = g / (K / 32), u = g % (K / 32);
    float v[32];
    raw_unit<T>(raw + n * raw_row_bytes<T>(K), (int)u, v);
    float* out = w + n * K + u * 32;
#pragma unroll
    for (int i = 0; i < 32; i += 4)
        st16(out + i, u32x4{__float_as_uint(v[i]), __float_as_uint(v[i + 1]), __float_as_uint(v[i + 2]), __float_as_uint(v[i + 3])});
}

// The exact path's product for one to eight activation rows, fused: y (M, N) = x (M, K) @ W.T with W's rows rebuilt
// from the file's blocks in registers (raw_unit, bit for bit the values mbq_dequant_raw writes), float32 products and
// sums, each row read once from HBM instead of written as float32 and read back (reference src/mashbox/ops/__init__.py
// :574-576, 624-632: dequant, then a float32 dot). Lanes in groups of LPR take one weight row each (4 waves x 64 / LPR
// rows per block, rows over the grid), a lane the row's 32-value units u = lane % LPR, + LPR, ...; the group's sums
// meet by shuffles; with U2 a lane has two units' loads in flight. Up to RGV_MAX_M activation rows, one float32 sum
// each in registers.
constexpr int RGV_MAX_M = 8;
template <int T, int LPR, bool U2>
__global__ __launch_bounds__(256) void raw_gemv_kernel(const uint8_t* __restrict__ raw, const uint16_t* __restrict__ x,
                                                       int M, int N, int K, void* __restrict__ y, int out_bf16) {
    constexpr int RPB = 256 / LPR;                                       // rows per block
    const int lane = threadIdx.x & (LPR - 1);
    const int U = K >> 5;
    const int64_t rb = raw_row_bytes<T>(K);
    for (int64_t n = (int64_t)blockIdx.x * RPB + threadIdx.x / LPR; n < N; n += (int64_t)gridDim.x * RPB) {
        float acc[RGV_MAX_M];
#pragma unroll
        for (int m = 0; m < RGV_MAX_M; ++m) acc[m] = 0.f;
        const uint8_t* row = raw + n * rb;
        for (int u0 = lane; u0 < U; u0 += (U2 ? 2 : 1) * LPR)
#pragma unroll
        for (int uu = 0; uu < (U2 ? 2 : 1); ++uu) {
            const int u = u0 + uu * LPR;
            if (u >= U) break;
            float v[32];
            raw_unit<T>(row, u, v);
#pragma unroll
            for (int m = 0; m < RGV_MAX_M; ++m) {
                if (m < M) {
                    const u32x4* xp = reinterpret_cast<const u32x4*>(x + (int64_t)m * K + 32 * u);
#pragma unroll
                    for (int c = 0; c < 4; ++c) {
                        const u32x4 q = xp[c];
#pragma unroll
                        for (int e = 0; e < 4; ++e) {
                            acc[m] = __builtin_fmaf(__uint_as_float(q[e] << 16), v[8 * c + 2 * e], acc[m]);
                            acc[m] = __builtin_fmaf(__uint_as_float(q[e] & 0xFFFF0000u), v[8 * c + 2 * e + 1], acc[m]);
                        }
                    }
                }
            }
        }
#pragma unroll
        for (int m = 0; m < RGV_MAX_M; ++m)
#pragma unroll
            for (int off = LPR / 2; off >= 1; off >>= 1) acc[m] += __shfl_xor(acc[m], off, LPR);
        if (lane == 0) {
#pragma unroll
            for (int m = 0; m < RGV_MAX_M; ++m) {
                if (m < M) {
                    if (out_bf16) reinterpret_cast<uint16_t*>(y)[(int64_t)m * N + n] = (uint16_t)bf16_bits(acc[m]);
                    else reinterpret_cast<float*>(y)[(int64_t)m * N + n] = acc[m];
                }
            }
        }
    }
}

// F32, F16, BF16 (reference :372-381): one value per block, any row length; the rows are contiguous in the file and
// in w, so one thread takes 4 consecutive values of the whole (rows x K) array
template <int T>
__global__ __launch_bounds__(256) void dequant_raw_float_kernel(const uint8_t* __restrict__ raw, int64_t total,
                                                                float* __restrict__ w) {
    const int64_t i0 = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) * 4;
    const int64_t i1 = i0 + 4 < total ? i0 + 4 : total;
    for (int64_t i = i0; i < i1; ++i) {
        if constexpr (T == T_F32) w[i] = __uint_as_float(le32(raw + 4 * i));
        else if constexpr (T == T_F16) w[i] = f16f(le16(raw + 2 * i));
        else w[i] = __uint_as_float(le16(raw + 2 * i) << 16);
    }
}

int launch_dequant_raw(int t, const uint8_t* raw, int64_t rows, int64_t K, float* w, hipStream_t s) {
    if (t == T_F32 || t == T_F16 || t == T_BF16) {
        const int64_t total = rows * K;
        const dim3 grid((unsigned)((total + 1023) / 1024));
        if (t == T_F32) dequant_raw_float_kernel<T_F32><<<grid, 256, 0, s>>>(raw, total, w);
        else if (t == T_F16) dequant_raw_float_kernel<T_F16><<<grid, 256, 0, s>>>(raw, total, w);
        else dequant_raw_float_kernel<T_BF16><<<grid, 256, 0, s>>>(raw, total, w);
        return check_launch("dequant_raw");
    }
    const int64_t units = rows * (K / 32);
    const dim3 grid((unsigned)((units + 255) / 256));
    switch (t) {
        case T_Q4_0: dequant_raw_kernel<T_Q4_0><<<grid, 256, 0, s>>>(raw, rows, (int)K, w); break;
        case T_Q4_K: dequant_raw_kernel<T_Q4_K><<<grid, 256, 0, s>>>(raw, rows, (int)K, w); break;
        case T_Q5_K: dequant_raw_kernel<T_Q5_K><<<grid, 256, 0, s>>>(raw, rows, (int)K, w); break;
        case T_Q6_K: dequant_raw_kernel<T_Q6_K><<<grid, 256, 0, s>>>(raw, rows, (int)K, w); break;
        case T_Q8_0: dequant_raw_kernel<T_Q8_0><<<grid, 256, 0, s>>>(raw, rows, (int)K, w); break;
        case T_Q4_1: dequant_raw_more_kernel<T_Q4_1><<<grid, 256, 0, s>>>(raw, rows, (int)K, w); break;
        case T_Q5_0: dequant_raw_more_kernel<T_Q5_0><<<grid, 256, 0, s>>>(raw, rows, (int)K, w); break;
        case T_Q5_1: dequant_raw_more_kernel<T_Q5_1><<<grid, 256, 0, s>>>(raw, rows, (int)K, w); break;
        case T_Q2_K: dequant_raw_more_kernel<T_Q2_K><<<grid, 256, 0, s>>>(raw, rows, (int)K, w); break;
        case T_Q3_K: dequant_raw_more_kernel<T_Q3_K><<<grid, 256, 0, s>>>(raw, rows, (int)K, w); break;
        case T_IQ4_NL: dequant_raw_more_kernel<T_IQ4_NL><<<grid, 256, 0, s>>>(raw, rows, (int)K, w); break;
        case T_IQ4_XS: dequant_raw_more_kernel<T_IQ4_XS><<<grid, 256, 0, s>>>(raw, rows, (int)K, w); break;
        case T_TQ1_0: dequant_raw_more_kernel<T_TQ1_0><<<grid, 256, 0, s>>>(raw, rows, (int)K, w); break;
        case T_TQ2_0: dequant_raw_more_kernel<T_TQ2_0><<<grid, 256, 0, s>>>(raw, rows, (int)K, w); break;
        case T_MXFP4: dequant_raw_more_kernel<T_MXFP4><<<grid, 256, 0, s>>>(raw, rows, (int)K, w); break;
        case T_NVFP4: dequant_raw_more_kernel<T_NVFP4><<<grid, 256, 0, s>>>(raw, rows, (int)K, w); break;
        default: return set_error(MBQ_BAD_ARG, "dequant_raw: no kernel for ggml type %d", t);
    }
    return check_launch("dequant_raw");
}

// Lanes per row by the row's 32-value units U (MI355X, interleaved timings of 16, 32 and 64 lanes, with and without two
// units in flight, on Q2_K 9728 x 2560, Q3_K 17408 x 5120, IQ4_XS 5120 x 17408, Q5_0 6144 x 5120 at 4 rows and F16
// 4096 x 4096): short rows (U < 128) 16 lanes, so that a wave holds 4 rows (Q2_K 14.5 -> 10.8 us); the 256-value types,
// whose units cost the most vector work, 32 lanes up to U = 256 (Q3_K 51.3 -> 46.5 us); else 64, with two units in
// flight from U = 256 on (IQ4_XS 66.1 -> 60.8 us). Each choice was the fastest or within 2 % of it on those cases.
template <int T>
static void raw_gemv_t(const uint8_t* raw, const uint16_t* x, int64_t M, int64_t N, int64_t K, void* y, int out_bf16,
                       hipStream_t s) {
    const int64_t U = K / 32;
    constexpr bool HEAVY = ggml_block(T).values == 256;
    if (U < 128)
        raw_gemv_kernel<T, 16, false><<<dim3((unsigned)((N + 15) / 16)), 256, 0, s>>>(raw, x, (int)M, (int)N, (int)K, y, out_bf16);
    else if (HEAVY && U < 256)
        raw_gemv_kernel<T, 32, false><<<dim3((unsigned)((N + 7) / 8)), 256, 0, s>>>(raw, x, (int)M, (int)N, (int)K, y, out_bf16);
    else if (U < 256)
        raw_gemv_kernel<T, 64, false><<<dim3((unsigned)((N + 3) / 4)), 256, 0, s>>>(raw, x, (int)M, (int)N, (int)K, y, out_bf16);
    else
        raw_gemv_kernel<T, 64, true><<<dim3((unsigned)((N + 3) / 4)), 256, 0, s>>>(raw, x, (int)M, (int)N, (int)K, y, out_bf16);
}

int launch_raw_gemv(int t, const uint8_t* raw, const uint16_t* x, int64_t M, int64_t N, int64_t K, void* y, int out_bf16,
                    hipStream_t s) {
    switch (t) {
        case T_F32: raw_gemv_t<T_F32>(raw, x, M, N, K, y, out_bf16, s); break;
        case T_F16: raw_gemv_t<T_F16>(raw, x, M, N, K, y, out_bf16, s); break;
        case T_BF16: raw_gemv_t<T_BF16>(raw, x, M, N, K, y, out_bf16, s); break;
        case T_Q4_1: raw_gemv_t<T_Q4_1>(raw, x, M, N, K, y, out_bf16, s); break;
        case T_Q5_0: raw_gemv_t<T_Q5_0>(raw, x, M, N, K, y, out_bf16, s); break;
        case T_Q5_1: raw_gemv_t<T_Q5_1>(raw, x, M, N, K, y, out_bf16, s); break;
        case T_Q2_K: raw_gemv_t<T_Q2_K>(raw, x, M, N, K, y, out_bf16, s); break;
        case T_Q3_K: raw_gemv_t<T_Q3_K>(raw, x, M, N, K, y, out_bf16, s); break;
        case T_IQ4_NL: raw_gemv_t<T_IQ4_NL>(raw, x, M, N, K, y, out_bf16, s); break;
        case T_IQ4_XS: raw_gemv_t<T_IQ4_XS>(raw, x, M, N, K, y, out_bf16, s); break;
        case T_TQ1_0: raw_gemv_t<T_TQ1_0>(raw, x, M, N, K, y, out_bf16, s); break;
        case T_TQ2_0: raw_gemv_t<T_TQ2_0>(raw, x, M, N, K, y, out_bf16, s); break;
        case T_MXFP4: raw_gemv_t<T_MXFP4>(raw, x, M, N, K, y, out_bf16, s); break;
        case T_NVFP4: raw_gemv_t<T_NVFP4>(raw, x, M, N, K, y, out_bf16, s); break;
        default: return set_error(MBQ_BAD_ARG, "raw GEMV: no kernel for ggml type %d (kernel types run on their planes)", t);
    }
    return check_launch("raw GEMV");
}

// -------------------------------------------------------------------------------------------------- zero fill
// n bytes at p set to zero, one byte per thread (the planes' alignment padding: under 256 bytes a run). A kernel, not
// hipMemsetAsync, so that a repack recorded into a HIP graph replays correctly.
__global__ __launch_bounds__(256) void zero_kernel(uint8_t* __restrict__ p, int64_t n) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) p[i] = 0;
}

int launch_zero(uint8_t* p, int64_t n, hipStream_t s) {
    if (n <= 0) return 0;
    zero_kernel<<<dim3((unsigned)((n + 255) / 256)), 256, 0, s>>>(p, n);
    return check_launch("zero fill");
}

// ------------------------------------------------------------------------------------------------ device repack
// One thread per block: the file's bytes (unaligned, 18, 34, 144, 176 or 210 bytes apart) into the planes of
// mbq_layout.h.
template <int T>
__global__ __launch_bounds__(256) void repack_kernel(const uint8_t* __restrict__ raw, int N, int K, uint8_t* __restrict__ planes,
                                                     int64_t sc_off, int64_t hi_off, int64_t d_off) {
    const int bv = (q8_like(T) || q40_like(T)) ? 32 : 256;
    const int bb = q40_like(T) ? 18 : q8_like(T) ? 34 : q4k_like(T) ? 144 : q5k_like(T) ? 176 : 210;
    const int64_t nb = K / bv;
    const int64_t g = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    // tiles: the last tile's padding rows too, and for T_Q8T / T_Q40T the padding blocks of the last chunk (written zero)
    const int64_t rows = tiled_type(T) ? ((int64_t)N + 15) / 16 * 16 : N;
    const int64_t nbr = T == T_Q8T ? ((int64_t)K + 63) / 64 * 2 : T == T_Q40T ? ((int64_t)K + 127) / 128 * 4 : nb;
    if (g >= rows * nbr) return;
    const int64_t n = g / nbr, b = g % nbr;
    const bool live = n < N && b < nb;
    const uint8_t* src = raw + (live ? n * nb * bb + b * bb : 0);
    if constexpr (T == T_Q8T) {
        uint8_t* q = planes + i8t_off(n, K, (32 * b) & ~int64_t(63));
        for (int i = 0; i < 32; ++i) q[q8t_byte(32 * (int)(b & 1) + i)] = live ? src[2 + i] : 0;
        uint8_t* d = planes + sc_off + q8t_d_off(n, K) + (b / 2) * 64 + (b % 2) * 2;
        d[0] = live ? src[0] : 0;
        d[1] = live ? src[1] : 0;
    } else if constexpr (T == T_Q8_0) {
        uint8_t* q = planes + n * K + b * 32;
        for (int i = 0; i < 32; ++i) q[i] = src[2 + i];
        uint8_t* d = planes + sc_off + (n * nb + b) * 2;
        d[0] = src[0];
        d[1] = src[1];
    } else if constexpr (q40_like(T)) {
        // T_Q40T: at the tile offsets; rows past N and blocks past K (the last chunk's padding) written zero
        constexpr bool TL = T == T_Q40T;
        uint8_t* d = planes + sc_off + (TL ? q40t_d_off(n, K) + (b >> 2) * 128 + (b & 3) * 2 : (n * nb + b) * 2);
        d[0] = live ? src[0] : 0;
        d[1] = live ? src[1] : 0;
        uint32_t* dst = reinterpret_cast<uint32_t*>(planes + (TL ? q40t_off(n, K) + (b >> 2) * 1024 + (b & 3) * 16 : n * (K >> 1) + b * 16));
        for (int t = 0; t < 4; ++t) {
            uint32_t v = 0;
            for (int e = 0; e < 8 && live; ++e) {
                const int i = t * 8 + e;                               // slot of mbq_layout.h: dword i/8, bits 16 (e&1) + 4 (e/2)
                v |= ((uint32_t)(src[2 + (i & 15)] >> (4 * (i >> 4))) & 15u) << (16 * (e & 1) + 4 * (e >> 1));
            }
            dst[t] = v;
        }
    } else if constexpr (q5k_like(T)) {
        // T_Q5KT: at the tile offsets; the last tile's rows past N written zero
        constexpr bool TL = T == T_Q5KT;
        uint8_t* meta = planes + sc_off + (TL ? q4kt_meta_off(n, K) + b * 256 : (n * nb + b) * 16);
        for (int i = 0; i < 16; ++i) meta[i] = live ? src[i] : 0;
        for (int j = 0; j < 8; ++j) {
            uint32_t* qd = reinterpret_cast<uint32_t*>(planes + (TL ? q4kt_off(n, K) + (2 * b + (j >> 2)) * 1024 + (j & 3) * 16 : n * (K >> 1) + b * 128 + j * 16));
            uint32_t* hd = reinterpret_cast<uint32_t*>(planes + hi_off + (TL ? q5kt_h_off(n, K) + (2 * b + (j >> 2)) * 256 + (j & 3) * 4 : n * (K >> 3) + b * 32 + j * 4));
            uint32_t qw[4] = {0, 0, 0, 0}, hw = 0;
            for (int i = 0; i < 32 && live; ++i) {
                const uint32_t lo = (src[48 + 32 * (j >> 1) + i] >> (4 * (j & 1))) & 15u;
                const uint32_t hi = (src[16 + i] >> j) & 1u;
                // slots of mbq_layout.h: low nibble dword i/8, byte i%4, bits 4 ((i/4)%2); high bit byte i%4,
                // bit 2 (i/8) + (i/4)%2
                qw[i >> 3] |= lo << (8 * (i & 3) + 4 * ((i >> 2) & 1));
                hw |= hi << (8 * (i & 3) + 2 * (i >> 3) + ((i >> 2) & 1));
            }
            for (int t = 0; t < 4; ++t) qd[t] = qw[t];
            hd[0] = hw;
        }
    } else if constexpr (q6k_like(T)) {
        // T_Q6KT: every plane's bytes at their tile offsets; the last tile's rows past N written zero
        constexpr bool TL = T == T_Q6KT;
        for (int i = 0; i < 16; ++i)
            planes[sc_off + (TL ? q6kt_s_off(n, K) + (2 * b + (i >> 3)) * 128 + (i & 7) : n * (K >> 4) + b * 16 + i)] = live ? src[192 + i] : 0;
        uint8_t* d = planes + d_off + (TL ? q6kt_d_off(n, K) + b * 32 : (n * nb + b) * 2);
        d[0] = live ? src[208] : 0;
        d[1] = live ? src[209] : 0;
        for (int j = 0; j < 8; ++j) {
            uint32_t* qd = reinterpret_cast<uint32_t*>(planes + (TL ? q4kt_off(n, K) + (2 * b + (j >> 2)) * 1024 + (j & 3) * 16 : n * (K >> 1) + b * 128 + j * 16));
            uint32_t* hd = reinterpret_cast<uint32_t*>(planes + hi_off + (TL ? q6kt_h_off(n, K) + (2 * b + (j >> 2)) * 512 + (j & 3) * 8 : n * (K >> 2) + b * 64 + j * 8));
            const int g = j >> 2, r = j & 3;
            uint32_t qw[4] = {0, 0, 0, 0}, hw[2] = {0, 0};
            for (int i = 0; i < 32 && live; ++i) {
                const uint32_t lo = (src[64 * g + 32 * (r & 1) + i] >> (4 * (r >> 1))) & 15u;
                const uint32_t hi = (src[128 + 32 * g + i] >> (2 * r)) & 3u;
                // slots of mbq_layout.h: low nibble dword i/8, byte i%4, bits 4 ((i/4)%2); high bits dword i/16,
                // byte i%4, bits 2 ((i/4)%4)
                qw[i >> 3] |= lo << (8 * (i & 3) + 4 * ((i >> 2) & 1));
                hw[i >> 4] |= hi << (8 * (i & 3) + 2 * ((i >> 2) & 3));
            }
            for (int t = 0; t < 4; ++t) qd[t] = qw[t];
            hd[0] = hw[0];
            hd[1] = hw[1];
        }
    } else if constexpr (T == T_Q4KT) {
        // the Q4_K units and header of row n at their tile offsets (mbq_layout.h); the rows of the last tile past the
        // weight's own (n >= N) are written zero
        uint8_t* meta = planes + sc_off + q4kt_meta_off(n, K) + b * 256;
        for (int i = 0; i < 16; ++i) meta[i] = live ? src[i] : 0;
        const uint8_t* qs = src + 16;
        for (int j = 0; j < 8; ++j) {
            uint32_t* dst = reinterpret_cast<uint32_t*>(planes + q4kt_off(n, K) + (2 * b + (j >> 2)) * 1024 + (j & 3) * 16);
            for (int t = 0; t < 4; ++t) {
                uint32_t v = 0;
                for (int e = 0; e < 8 && live; ++e) {
                    const int i = t * 8 + e;
                    const uint32_t byte = qs[32 * (j >> 1) + i];
                    const uint32_t q = (j & 1) ? (byte >> 4) : (byte & 15u);
                    v |= q << (16 * (e & 1) + 4 * (e >> 1));
                }
                dst[t] = v;
            }
        }
    } else {
        uint8_t* meta = planes + sc_off + (n * nb + b) * 16;
        for (int i = 0; i < 16; ++i) meta[i] = src[i];
        const uint8_t* qs = src + 16;
        uint32_t* dst = reinterpret_cast<uint32_t*>(planes + n * (K >> 1) + b * 128);
        for (int j = 0; j < 8; ++j)
            for (int t = 0; t < 4; ++t) {
                uint32_t v = 0;
                for (int e = 0; e < 8; ++e) {
                    const int i = t * 8 + e;
                    const uint32_t byte = qs[32 * (j >> 1) + i];
                    const uint32_t q = (j & 1) ? (byte >> 4) : (byte & 15u);
                    v |= q << (16 * (e & 1) + 4 * (e >> 1));
                }
                dst[j * 4 + t] = v;
            }
    }
}

// ------------------------------------------------------------------------------------------- tiled int8 repack
// One thread per 16 bytes of the quant plane (mbq_layout.h, T_I8T): thread g fills bytes 16 (g % 4) .. of row g / 4 % 16
// of block g / 64, from the row-major quants, or zero past N or K; the first NP threads also write the scale plane.
// HBM-bound, load-time only.
__global__ __launch_bounds__(256) void i8t_repack_kernel(const int8_t* __restrict__ q, const float* __restrict__ sc, int64_t N,
                                                         int64_t K, uint8_t* __restrict__ planes, int64_t sc_off, int64_t chunks,
                                                         int64_t np) {
    const int64_t g = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    const int64_t kc_n = (K + 63) / 64;
    if (g < chunks) {
        const int64_t blk = g >> 6, c = g & 63, r = c >> 2, part = c & 3;
        const int64_t row = (blk / kc_n) * 16 + r, col = (blk % kc_n) * 64 + 16 * part;
        u32x4 v = {0u, 0u, 0u, 0u};
        if (row < N && col < K) v = ld16(q + row * K + col);           // K % 16 == 0: whole 16-byte pieces
        st16(planes + blk * 1024 + r * 64 + 16 * part, v);
    }
    if (g < np) reinterpret_cast<float*>(planes + sc_off)[g] = g < N ? sc[g] : 0.f;
}

int launch_i8t_repack(const int8_t* q, const float* sc, int64_t N, int64_t K, uint8_t* planes, const Layout& L, hipStream_t s) {
    const int64_t chunks = L.qs_bytes / 16, np = (N + 15) / 16 * 16;
    const int64_t threads = std::max(chunks, np);
    i8t_repack_kernel<<<dim3((unsigned)((threads + 255) / 256)), 256, 0, s>>>(q, sc, N, K, planes, L.sc_off, chunks, np);
    return check_launch("int8 repack");
}

// ------------------------------------------------------------------------------------------ int8 embedding rows
// y[t, :] = f32(q[r, :]) * s[r] (then rounded to bfloat16 when out_bf16), r = toks[t] (+ N when negative, clamped to
// [0, N - 1]): reference src/mashbox/models/qwen3_8_27b/model.py:132-139 (embed, whose int8_rows at :117-129 equals the
// plain gather bit for bit). HBM-bound: D bytes read and 2 D (4 D) written per token. VEC: D % 16 == 0, one thread per
// 16 values (one 16-byte load, two or four 16-byte stores); else one thread per value.
template <bool VEC>
__global__ __launch_bounds__(256) void embed_kernel(const int8_t* __restrict__ q, const float* __restrict__ s, int64_t N,
                                                    int64_t D, const int32_t* __restrict__ toks, void* __restrict__ y,
                                                    int out_bf16) {
    const int64_t t = blockIdx.y;
    int64_t r = toks[t];
    r = r < 0 ? r + N : r;
    r = r < 0 ? 0 : (r >= N ? N - 1 : r);
    const float sc = s[r];
    const int64_t per = VEC ? 16 : 1;
    const int64_t c = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) * per;
    if (c >= D) return;
    if constexpr (VEC) {
        const u32x4 w = ld16(q + r * D + c);
        float v[16];
#pragma unroll
        for (int e = 0; e < 16; ++e) v[e] = (float)(int8_t)(w[e >> 2] >> (8 * (e & 3))) * sc;
        if (out_bf16) {
            uint16_t* o = reinterpret_cast<uint16_t*>(y) + t * D + c;
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                u32x4 p;
#pragma unroll
                for (int e = 0; e < 4; ++e) p[e] = bf16_bits(v[8 * h + 2 * e]) | (bf16_bits(v[8 * h + 2 * e + 1]) << 16);
                st16(o + 8 * h, p);
            }
        } else {
            float* o = reinterpret_cast<float*>(y) + t * D + c;
#pragma unroll
            for (int h = 0; h < 4; ++h)
                st16(o + 4 * h, u32x4{__float_as_uint(v[4 * h]), __float_as_uint(v[4 * h + 1]), __float_as_uint(v[4 * h + 2]),
                                      __float_as_uint(v[4 * h + 3])});
        }
    } else {
        store_y(y, t * D + c, (float)q[r * D + c] * sc, out_bf16);
    }
}

int launch_int8_embed(const int8_t* q, const float* s, int64_t N, int64_t D, const int32_t* toks, int64_t T, void* y,
                      int out_bf16, hipStream_t st) {
    const bool vec = D % 16 == 0 && (reinterpret_cast<uintptr_t>(q) & 15) == 0 && (reinterpret_cast<uintptr_t>(y) & 15) == 0;
    const int64_t per = vec ? 16 : 1, threads = (D + per - 1) / per;
    const dim3 grid((unsigned)((threads + 255) / 256), (unsigned)T);
    if (vec)
        embed_kernel<true><<<grid, 256, 0, st>>>(q, s, N, D, toks, y, out_bf16);
    else
        embed_kernel<false><<<grid, 256, 0, st>>>(q, s, N, D, toks, y, out_bf16);
    return check_launch("int8 embed");
}

// -------------------------------------------------------------------------------------------------- launchers
static int check_launch(const char* what) {
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return set_error(MBQ_LAUNCH_FAIL, "%s: %s", what, hipGetErrorString(e));
    return 0;
}

// Decode batches (M <= GEMV_MAX_M) run the GEMV when it has a plan for the shape; a row too long for the activation
// rows' registers (e.g. K = 17408 at 3-4 rows, or a Q8_0 / int8 K over 24576) runs the weight-stream kernel instead,
// which takes any K (launch_gemm routes M <= GEMV_MAX_M there).
template <int T>
static int launch_t(const Args& a, hipStream_t s) {
    return a.M <= GEMV_MAX_M && gemv_runs(T, a) ? launch_gemv(T, a, s) : launch_gemm(T, a, s);
}

int cus_of_device() {
    static std::atomic<int> cache[64];
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
    int n = cache[dev].load(std::memory_order_relaxed);
    if (n == 0) {
        if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) n = 256;
        cache[dev].store(n, std::memory_order_relaxed);
    }
    return n;
}

int launch_matmul(int t, const Args& a, hipStream_t s) {
    switch (t) {
        case T_Q4_0: return launch_t<T_Q4_0>(a, s);
        case T_Q8_0: return launch_t<T_Q8_0>(a, s);
        case T_Q4_K: return launch_t<T_Q4_K>(a, s);
        case T_Q5_K: return launch_t<T_Q5_K>(a, s);
        case T_Q6_K: return launch_t<T_Q6_K>(a, s);
        case T_INT8: return launch_t<T_INT8>(a, s);
        case T_I8T: return launch_t<T_I8T>(a, s);
        case T_Q4KT: return launch_t<T_Q4KT>(a, s);
        case T_Q8T: return launch_t<T_Q8T>(a, s);
        case T_Q6KT: return launch_t<T_Q6KT>(a, s);
        case T_Q5KT: return launch_t<T_Q5KT>(a, s);
        case T_Q40T: return launch_t<T_Q40T>(a, s);
    }
    return set_error(MBQ_BAD_ARG, "no kernel for type %d", t);
}

int launch_dequant(int t, const Args& a, float* w, const int32_t* rows, int64_t out_rows, hipStream_t s) {
    const int64_t uw = unit32(t) ? 32 : 16;
    const int64_t units = (rows ? out_rows : a.N) * (a.K / uw);
    if (units == 0) return 0;
    const dim3 grid((unsigned)((units + 255) / 256));
    auto run = [&](auto kern) {
        kern<<<grid, 256, 0, s>>>(a.base, a.stride, a.layer_dev, a.nlayers, a.sc_off, a.hi_off, a.d_off, (int)a.N, (int)a.K, w,
                                  rows, rows ? out_rows : a.N);
    };
    if (t == T_Q4_0) run(dequant_kernel<T_Q4_0>);
    else if (t == T_Q4_K) run(dequant_kernel<T_Q4_K>);
    else if (t == T_Q4KT) run(dequant_kernel<T_Q4KT>);
    else if (t == T_Q8T) run(dequant_kernel<T_Q8T>);
    else if (t == T_Q6KT) run(dequant_kernel<T_Q6KT>);
    else if (t == T_Q5KT) run(dequant_kernel<T_Q5KT>);
    else if (t == T_Q40T) run(dequant_kernel<T_Q40T>);
    else if (t == T_Q5_K) run(dequant_kernel<T_Q5_K>);
    else if (t == T_Q6_K) run(dequant_kernel<T_Q6_K>);
    else run(dequant_kernel<T_Q8_0>);
    return check_launch("dequant");
}

int launch_repack(int t, const uint8_t* raw, int64_t N, int64_t K, uint8_t* planes, const Layout& L, hipStream_t s) {
    const int64_t blocks = t == T_Q8T ? (N + 15) / 16 * 16 * ((K + 63) / 64 * 2)
                           : t == T_Q40T ? (N + 15) / 16 * 16 * ((K + 127) / 128 * 4)
                                      : (tiled_type(t) ? (N + 15) / 16 * 16 : N) * (K / block_values(t));
    const dim3 grid((unsigned)((blocks + 255) / 256));
    auto run = [&](auto kern) { kern<<<grid, 256, 0, s>>>(raw, (int)N, (int)K, planes, L.sc_off, L.hi_off, L.d_off); };
    if (t == T_Q4_0) run(repack_kernel<T_Q4_0>);
    else if (t == T_Q4_K) run(repack_kernel<T_Q4_K>);
    else if (t == T_Q4KT) run(repack_kernel<T_Q4KT>);
    else if (t == T_Q8T) run(repack_kernel<T_Q8T>);
    else if (t == T_Q6KT) run(repack_kernel<T_Q6KT>);
    else if (t == T_Q5KT) run(repack_kernel<T_Q5KT>);
    else if (t == T_Q40T) run(repack_kernel<T_Q40T>);
    else if (t == T_Q5_K) run(repack_kernel<T_Q5_K>);
    else if (t == T_Q6_K) run(repack_kernel<T_Q6_K>);
    else run(repack_kernel<T_Q8_0>);
    return check_launch("repack");
}

}  // namespace mbq
