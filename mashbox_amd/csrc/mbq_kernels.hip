// gfx950 (CDNA4) kernels of the quantized linear: dequant, device repack and the matmul dispatch (decode GEMV:
// mbq_gemv.hip; weight-stream GEMM: mbq_wsgemm.hip; LDS-tile MFMA GEMM: mbq_gemm.hip).
//
// Semantics follow reference src/mashbox/ops/__init__.py:594-632 (qmatmul: x @ W.T, float32 accumulation) with the
// weights of reference src/mashbox/ops/reference.py:101-103 (Q8_0) and :132-149 (Q4_K), and the int8 per-channel
// linear of reference src/mashbox/models/qwen3_8_27b/model.py:72-82. Plane layouts: mbq_layout.h.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <algorithm>

#include "mbq_device.h"
#include "mbq_launch.h"
#include "mbq_layout.h"

namespace mbq {


// ------------------------------------------------------------------------------------------------------- dequant
// One thread per 16-byte unit (Q4_K: a sub-block of 32 values; Q8_0: half a block, 16 values). Bit for bit the
// reference dequantization: Q8_0 v = f32(q) * d and Q4_K v = (d*sc)*q - dmin*m, whose products are exact in float32.
template <int T>
__global__ __launch_bounds__(256) void dequant_kernel(const uint8_t* __restrict__ base, int64_t stride,
                                                      const int32_t* __restrict__ layer_dev, int nlayers, int64_t sc_off,
                                                      int N, int K, float* __restrict__ w) {
    const int64_t uw = (T == T_Q4_K) ? 32 : 16;
    const int64_t units = (int64_t)N * (K / uw);
    const int64_t g = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (g >= units) return;
    const int64_t lo = layer_offset(stride, layer_dev, nlayers);
    const bool ok = lo >= 0;
    base += ok ? lo : 0;
    const int64_t n = g / (K / uw), u = g % (K / uw);
    float* out = w + n * K + u * uw;
    if (!ok) {
        for (int i = 0; i < uw; ++i) out[i] = __builtin_nanf("");
        return;
    }
    if constexpr (T == T_Q4_K) {
        const u32x4 q = ld16(base + n * (K >> 1) + u * 16);
        const u32x4 mt = ld16(base + sc_off + (n * (K >> 8) + (u >> 3)) * 16);
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
        const u32x4 q = ld16(base + n * K + u * 16);
        const float d = f16f(*reinterpret_cast<const uint16_t*>(base + sc_off + (n * (K >> 5) + (u >> 1)) * 2));
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
// :398-409 (dequant) with :101-103 (Q8_0) and :132-149 (Q4_K), the rebuild of the exact path. One thread per 32 values
// (a Q8_0 block, a Q4_K sub-block); the blocks are 34 / 144 bytes apart, so bytes are read one at a time.
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

int launch_dequant_raw(int t, const uint8_t* raw, int64_t rows, int64_t K, float* w, hipStream_t s) {
    const int64_t units = rows * (K / 32);
    const dim3 grid((unsigned)((units + 255) / 256));
    if (t == T_Q4_K)
        dequant_raw_kernel<T_Q4_K><<<grid, 256, 0, s>>>(raw, rows, (int)K, w);
    else
        dequant_raw_kernel<T_Q8_0><<<grid, 256, 0, s>>>(raw, rows, (int)K, w);
    return check_launch("dequant_raw");
}

// ------------------------------------------------------------------------------------------------ device repack
// One thread per block: the file's bytes (unaligned, 34 or 144 bytes apart) into the planes of mbq_layout.h.
template <int T>
__global__ __launch_bounds__(256) void repack_kernel(const uint8_t* __restrict__ raw, int N, int K, uint8_t* __restrict__ planes,
                                                     int64_t sc_off) {
    const int bv = (T == T_Q4_K) ? 256 : 32, bb = (T == T_Q4_K) ? 144 : 34;
    const int64_t nb = K / bv;
    const int64_t g = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (g >= (int64_t)N * nb) return;
    const int64_t n = g / nb, b = g % nb;
    const uint8_t* src = raw + n * nb * bb + b * bb;
    if constexpr (T == T_Q8_0) {
        uint8_t* q = planes + n * K + b * 32;
        for (int i = 0; i < 32; ++i) q[i] = src[2 + i];
        uint8_t* d = planes + sc_off + (n * nb + b) * 2;
        d[0] = src[0];
        d[1] = src[1];
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

// -------------------------------------------------------------------------------------------------- launchers
static int check_launch(const char* what) {
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return set_error(MBQ_LAUNCH_FAIL, "%s: %s", what, hipGetErrorString(e));
    return 0;
}

template <int T>
static int launch_t(const Args& a, hipStream_t s) {
    return a.M <= GEMV_MAX_M ? launch_gemv(T, a, s) : launch_gemm(T, a, s);
}

int launch_matmul(int t, const Args& a, hipStream_t s) {
    switch (t) {
        case T_Q8_0: return launch_t<T_Q8_0>(a, s);
        case T_Q4_K: return launch_t<T_Q4_K>(a, s);
        case T_INT8: return launch_t<T_INT8>(a, s);
    }
    return set_error(MBQ_BAD_ARG, "no kernel for type %d", t);
}

int launch_dequant(int t, const Args& a, float* w, hipStream_t s) {
    const int64_t uw = (t == T_Q4_K) ? 32 : 16;
    const int64_t units = a.N * (a.K / uw);
    const dim3 grid((unsigned)((units + 255) / 256));
    if (t == T_Q4_K)
        dequant_kernel<T_Q4_K><<<grid, 256, 0, s>>>(a.base, a.stride, a.layer_dev, a.nlayers, a.sc_off, (int)a.N, (int)a.K, w);
    else
        dequant_kernel<T_Q8_0><<<grid, 256, 0, s>>>(a.base, a.stride, a.layer_dev, a.nlayers, a.sc_off, (int)a.N, (int)a.K, w);
    return check_launch("dequant");
}

int launch_repack(int t, const uint8_t* raw, int64_t N, int64_t K, uint8_t* planes, int64_t sc_off, hipStream_t s) {
    const int64_t blocks = N * (K / block_values(t));
    const dim3 grid((unsigned)((blocks + 255) / 256));
    if (t == T_Q4_K)
        repack_kernel<T_Q4_K><<<grid, 256, 0, s>>>(raw, (int)N, (int)K, planes, sc_off);
    else
        repack_kernel<T_Q8_0><<<grid, 256, 0, s>>>(raw, (int)N, (int)K, planes, sc_off);
    return check_launch("repack");
}

}  // namespace mbq
