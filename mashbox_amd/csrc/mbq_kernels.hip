// gfx950 (CDNA4) kernels of the quantized linear: decode GEMV, MFMA GEMM, dequant and device repack.
//
// Semantics follow reference src/mashbox/ops/__init__.py:594-632 (qmatmul: x @ W.T, float32 accumulation) with the
// weights of reference src/mashbox/ops/reference.py:101-103 (Q8_0) and :132-149 (Q4_K), and the int8 per-channel
// linear of reference src/mashbox/models/qwen3_8_27b/model.py:72-82. Plane layouts: mbq_layout.h.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "mbq_launch.h"
#include "mbq_layout.h"

namespace mbq {

typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

// ----------------------------------------------------------------------------------------------------- helpers
__device__ __forceinline__ u32x4 ld16(const void* p) { return *reinterpret_cast<const u32x4*>(p); }
__device__ __forceinline__ void st16(void* p, u32x4 v) { *reinterpret_cast<u32x4*>(p) = v; }

// fp16 bits -> float32, exact (subnormal, inf and NaN kept): reference src/mashbox/ops/reference.py:49-51
__device__ __forceinline__ float f16f(uint32_t h) { return (float)__builtin_bit_cast(_Float16, (uint16_t)(h & 0xFFFFu)); }

// float32 -> bfloat16 bits, round to nearest even; NaN stays NaN (quiet)
__device__ __forceinline__ uint32_t bf16_bits(float f) {
    const uint32_t u = __float_as_uint(f);
    if ((u & 0x7FFFFFFFu) > 0x7F800000u) return (u >> 16) | 0x40u;
    return (u + 0x7FFFu + ((u >> 16) & 1u)) >> 16;
}

__device__ __forceinline__ float dot2(uint32_t a, uint32_t b, float c) {
    return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, a), __builtin_bit_cast(bf16x2_t, b), c, false);
}

// Q4_K unit dword -> bfloat16 pair (128 + q[8t+2p], 128 + q[8t+2p+1]); exact (mbq_layout.h)
__device__ __forceinline__ uint32_t nib_pair(uint32_t w, int p) { return ((w >> (4 * p)) & 0x000F000Fu) | 0x43004300u; }

// int8 bytes 2p, 2p+1 of w -> bfloat16 pair, exact (every int8 is a bfloat16)
__device__ __forceinline__ uint32_t i8_pair(uint32_t w, int p) {
    const float f0 = (float)(int8_t)(w >> (16 * p));
    const float f1 = (float)(int8_t)(w >> (16 * p + 8));
    return __builtin_amdgcn_perm(__float_as_uint(f1), __float_as_uint(f0), 0x07060302u);
}

// Q4_K: scale and min of sub-block j from the super-block's scale dwords s0 (bytes 0-3), s1 (4-7), s2 (8-11):
// reference src/mashbox/ops/reference.py:132-139 (_scale_min_k4)
__device__ __forceinline__ void q4k_scale_min(uint32_t s0, uint32_t s1, uint32_t s2, int j, uint32_t* sc, uint32_t* mn) {
    const int sh = 8 * (j & 3);
    if (j < 4) {
        *sc = (s0 >> sh) & 63u;
        *mn = (s1 >> sh) & 63u;
    } else {
        *sc = ((s2 >> sh) & 15u) | (((s0 >> (sh + 6)) & 3u) << 4);
        *mn = ((s2 >> (sh + 4)) & 15u) | (((s1 >> (sh + 6)) & 3u) << 4);
    }
}

// byte offset of the layer a kernel reads; -1 when layer_dev names no layer of the stack
__device__ __forceinline__ int64_t layer_offset(int64_t stride, const int32_t* layer_dev, int nlayers) {
    if (layer_dev == nullptr) return 0;
    const int l = *layer_dev;
    if (l < 0 || l >= nlayers) return -1;
    return (int64_t)l * stride;
}

__device__ __forceinline__ void store_y(void* y, int64_t i, float v, int out_bf16) {
    if (out_bf16)
        reinterpret_cast<uint16_t*>(y)[i] = (uint16_t)bf16_bits(v);
    else
        reinterpret_cast<float*>(y)[i] = v;
}

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off, 64);
    return v;
}

constexpr uint32_t BF16_ONES = 0x3F803F80u;  // bfloat16 pair (1, 1)

// ---------------------------------------------------------------------------------------------------- decode GEMV
// One wave owns R consecutive weight rows and the whole K; its 64 lanes stride over the rows' 16-byte units
// (Q4_K: a 32-quant sub-block; Q8_0 / int8: 16 quants). Every load is a 128-bit vector load and a wave's loads of one
// row are 1 KiB contiguous. Quants become bfloat16 pairs in registers (exact) and meet x through v_dot2_f32_bf16 with
// float32 accumulation; block scales are applied once per unit in float32; the lanes' partial sums are reduced across
// the wave at the end. Up to M = 4 activation rows share each weight load.
template <int T, int M, int R>
__global__ __launch_bounds__(256) void gemv_kernel(const uint8_t* __restrict__ base, int64_t stride,
                                                   const int32_t* __restrict__ layer_dev, int nlayers, int64_t sc_off,
                                                   const float* __restrict__ srow, const uint16_t* __restrict__ x,
                                                   int N, int K, void* __restrict__ y, int out_bf16) {
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int n0 = (blockIdx.x * 4 + wave) * R;
    if (n0 >= N) return;
    const int64_t lo = layer_offset(stride, layer_dev, nlayers);
    const bool ok = lo >= 0;
    base += ok ? lo : 0;
    float acc[R][M];
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
        for (int m = 0; m < M; ++m) acc[r][m] = 0.f;

    if (ok) {
        if constexpr (T == T_Q4_K) {
            const int U = K >> 5;
            const int64_t rq = K >> 1;
            const int nsb = K >> 8;
            const int j = lane & 7;  // sub-block of the super-block: lane-constant since units advance by 64
            for (int u = lane; u < U; u += 64) {
                u32x4 xv[M][4];
                float xs[M];
#pragma unroll
                for (int m = 0; m < M; ++m) {
#pragma unroll
                    for (int i = 0; i < 4; ++i) xv[m][i] = ld16(x + (int64_t)m * K + (int64_t)u * 32 + i * 8);
                    float s = 0.f;
#pragma unroll
                    for (int i = 0; i < 4; ++i)
#pragma unroll
                        for (int p = 0; p < 4; ++p) s = dot2(xv[m][i][p], BF16_ONES, s);
                    xs[m] = s;
                }
#pragma unroll
                for (int r = 0; r < R; ++r) {
                    const int64_t n = min(n0 + r, N - 1);
                    const u32x4 w = ld16(base + n * rq + (int64_t)u * 16);
                    const u32x4 mt = ld16(base + sc_off + (n * nsb + (u >> 3)) * 16);
                    uint32_t sc, mn;
                    q4k_scale_min(mt[1], mt[2], mt[3], j, &sc, &mn);
                    const float dsc = f16f(mt[0]) * (float)sc;          // exact
                    const float dm = f16f(mt[0] >> 16) * (float)mn;      // exact
                    const float c = 128.f * dsc + dm;
#pragma unroll
                    for (int m = 0; m < M; ++m) {
                        float P = 0.f;
#pragma unroll
                        for (int t = 0; t < 4; ++t)
#pragma unroll
                            for (int p = 0; p < 4; ++p) P = dot2(nib_pair(w[t], p), xv[m][t][p], P);
                        acc[r][m] += dsc * P - c * xs[m];
                    }
                }
            }
        } else {  // Q8_0 and int8: 16-quant units
            const int U = K >> 4;
            for (int u = lane; u < U; u += 64) {
                u32x4 xv[M][2];
#pragma unroll
                for (int m = 0; m < M; ++m)
#pragma unroll
                    for (int i = 0; i < 2; ++i) xv[m][i] = ld16(x + (int64_t)m * K + (int64_t)u * 16 + i * 8);
#pragma unroll
                for (int r = 0; r < R; ++r) {
                    const int64_t n = min(n0 + r, N - 1);
                    const u32x4 w = ld16(base + n * K + (int64_t)u * 16);
                    float d = 1.f;
                    if constexpr (T == T_Q8_0)
                        d = f16f(*reinterpret_cast<const uint16_t*>(base + sc_off + (n * (K >> 5) + (u >> 1)) * 2));
#pragma unroll
                    for (int m = 0; m < M; ++m) {
                        float P = 0.f;
#pragma unroll
                        for (int t = 0; t < 4; ++t)
#pragma unroll
                            for (int p = 0; p < 2; ++p) P = dot2(i8_pair(w[t], p), xv[m][t >> 1][((t & 1) << 1) + p], P);
                        if constexpr (T == T_Q8_0)
                            acc[r][m] += d * P;
                        else
                            acc[r][m] += P;
                    }
                }
            }
        }
    }
#pragma unroll
    for (int r = 0; r < R; ++r) {
        const int n = n0 + r;
        const float s = (T == T_INT8 && n < N) ? srow[n] : 1.f;
#pragma unroll
        for (int m = 0; m < M; ++m) {
            float v = wave_sum(acc[r][m]);
            if (lane == 0 && n < N) {
                v = ok ? v * s : __builtin_nanf("");
                store_y(y, (int64_t)m * N + n, v, out_bf16);
            }
        }
    }
}

// ------------------------------------------------------------------------------------------------------ MFMA GEMM
// Block tile 64 x 64 x 64, 4 waves (2 x 2), each wave 32 x 32 = 2 x 2 tiles of v_mfma_f32_16x16x32_bf16.
// x tiles are copied to LDS; weight tiles are dequantized into LDS as bfloat16 (int8: exact; Q8_0 / Q4_K: the float32
// dequantized value rounded to nearest even), then both feed the MFMA with float32 accumulation.
constexpr int GB_M = 64, GB_N = 64, GB_K = 64, G_LDS = GB_K + 8;

template <int T>
__device__ __forceinline__ void load_b_tile(uint16_t (*Bs)[G_LDS], const uint8_t* __restrict__ base, int64_t sc_off,
                                            int n0, int k0, int N, int K, int tid) {
    const int row = tid >> 2;
    const int gn = n0 + row;
    if constexpr (T == T_Q4_K) {
        const int sub = (tid >> 1) & 1, half = tid & 1;
        const int sbk = (k0 >> 5) + sub;  // sub-block index within the row
        uint32_t out[16];
        if (gn < N) {
            const u32x2 w = *reinterpret_cast<const u32x2*>(base + (int64_t)gn * (K >> 1) + (int64_t)sbk * 16 + half * 8);
            const u32x4 mt = ld16(base + sc_off + ((int64_t)gn * (K >> 8) + (sbk >> 3)) * 16);
            uint32_t sc, mn;
            q4k_scale_min(mt[1], mt[2], mt[3], sbk & 7, &sc, &mn);
            const float dsc = f16f(mt[0]) * (float)sc;
            const float dm = f16f(mt[0] >> 16) * (float)mn;
#pragma unroll
            for (int tt = 0; tt < 2; ++tt)
#pragma unroll
                for (int e = 0; e < 8; e += 2) {
                    const int p = e >> 1;
                    const float q0 = (float)((w[tt] >> (4 * p)) & 15u);
                    const float q1 = (float)((w[tt] >> (16 + 4 * p)) & 15u);
                    const float v0 = dsc * q0 - dm, v1 = dsc * q1 - dm;
                    out[tt * 4 + p] = bf16_bits(v0) | (bf16_bits(v1) << 16);
                }
        } else {
#pragma unroll
            for (int i = 0; i < 8; ++i) out[i] = 0u;
        }
        uint16_t* dst = &Bs[row][sub * 32 + half * 16];
        st16(dst, u32x4{out[0], out[1], out[2], out[3]});
        st16(dst + 8, u32x4{out[4], out[5], out[6], out[7]});
    } else {
        const int c = tid & 3;
        const int gk = k0 + c * 16;
        uint32_t out[8];
        if (gn < N && gk < K) {
            const u32x4 w = ld16(base + (int64_t)gn * K + gk);
            if constexpr (T == T_Q8_0) {
                const float d = f16f(*reinterpret_cast<const uint16_t*>(base + sc_off + ((int64_t)gn * (K >> 5) + (gk >> 5)) * 2));
#pragma unroll
                for (int t = 0; t < 4; ++t)
#pragma unroll
                    for (int p = 0; p < 2; ++p) {
                        const float v0 = (float)(int8_t)(w[t] >> (16 * p)) * d;
                        const float v1 = (float)(int8_t)(w[t] >> (16 * p + 8)) * d;
                        out[t * 2 + p] = bf16_bits(v0) | (bf16_bits(v1) << 16);
                    }
            } else {
#pragma unroll
                for (int t = 0; t < 4; ++t)
#pragma unroll
                    for (int p = 0; p < 2; ++p) out[t * 2 + p] = i8_pair(w[t], p);
            }
        } else {
#pragma unroll
            for (int i = 0; i < 8; ++i) out[i] = 0u;
        }
        uint16_t* dst = &Bs[row][c * 16];
        st16(dst, u32x4{out[0], out[1], out[2], out[3]});
        st16(dst + 8, u32x4{out[4], out[5], out[6], out[7]});
    }
}

template <int T>
__global__ __launch_bounds__(256) void gemm_kernel(const uint8_t* __restrict__ base, int64_t stride,
                                                   const int32_t* __restrict__ layer_dev, int nlayers, int64_t sc_off,
                                                   const float* __restrict__ srow, const uint16_t* __restrict__ x,
                                                   int M, int N, int K, void* __restrict__ y, int out_bf16) {
    __shared__ __attribute__((aligned(16))) uint16_t As[GB_M][G_LDS];
    __shared__ __attribute__((aligned(16))) uint16_t Bs[GB_N][G_LDS];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int m0 = blockIdx.y * GB_M, n0 = blockIdx.x * GB_N;
    const int64_t lo = layer_offset(stride, layer_dev, nlayers);
    const bool ok = lo >= 0;
    base += ok ? lo : 0;
    const int wm = wave >> 1, wn = wave & 1;
    f32x4_t acc[2][2];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int jn = 0; jn < 2; ++jn) acc[i][jn] = f32x4_t{0.f, 0.f, 0.f, 0.f};

    if (ok) {
        for (int k0 = 0; k0 < K; k0 += GB_K) {
#pragma unroll
            for (int i = 0; i < 2; ++i) {
                const int e = tid + 256 * i, row = e >> 3, ch = e & 7;
                const int gm = m0 + row, gk = k0 + ch * 8;
                u32x4 v = {0u, 0u, 0u, 0u};
                if (gm < M && gk < K) v = ld16(x + (int64_t)gm * K + gk);
                st16(&As[row][ch * 8], v);
            }
            load_b_tile<T>(Bs, base, sc_off, n0, k0, N, K, tid);
            __syncthreads();
#pragma unroll
            for (int ks = 0; ks < GB_K / 32; ++ks) {
                bf16x8_t a[2], b[2];
                const int kk = ks * 32 + (lane >> 4) * 8;
#pragma unroll
                for (int i = 0; i < 2; ++i) a[i] = *reinterpret_cast<const bf16x8_t*>(&As[wm * 32 + i * 16 + (lane & 15)][kk]);
#pragma unroll
                for (int jn = 0; jn < 2; ++jn) b[jn] = *reinterpret_cast<const bf16x8_t*>(&Bs[wn * 32 + jn * 16 + (lane & 15)][kk]);
#pragma unroll
                for (int i = 0; i < 2; ++i)
#pragma unroll
                    for (int jn = 0; jn < 2; ++jn)
                        acc[i][jn] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a[i], b[jn], acc[i][jn], 0, 0, 0);
            }
            __syncthreads();
        }
    }
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int jn = 0; jn < 2; ++jn) {
            const int n = n0 + wn * 32 + jn * 16 + (lane & 15);
            if (n >= N) continue;
            const float s = (T == T_INT8) ? srow[n] : 1.f;
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int m = m0 + wm * 32 + i * 16 + (lane >> 4) * 4 + r;
                if (m < M) store_y(y, (int64_t)m * N + n, ok ? acc[i][jn][r] * s : __builtin_nanf(""), out_bf16);
            }
        }
}

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

template <int T, int M>
static void launch_gemv_m(const Args& a, hipStream_t s) {
    constexpr int R = 2;
    const dim3 grid((unsigned)((a.N + 4 * R - 1) / (4 * R)));
    gemv_kernel<T, M, R><<<grid, 256, 0, s>>>(a.base, a.stride, a.layer_dev, a.nlayers, a.sc_off, a.srow, a.x, (int)a.N,
                                              (int)a.K, a.y, a.out_bf16);
}

template <int T>
static int launch_t(const Args& a, hipStream_t s) {
    if (a.M <= GEMV_MAX_M) {
        switch (a.M) {
            case 1: launch_gemv_m<T, 1>(a, s); break;
            case 2: launch_gemv_m<T, 2>(a, s); break;
            case 3: launch_gemv_m<T, 3>(a, s); break;
            default: launch_gemv_m<T, 4>(a, s); break;
        }
        return check_launch("gemv");
    }
    const dim3 grid((unsigned)((a.N + GB_N - 1) / GB_N), (unsigned)((a.M + GB_M - 1) / GB_M));
    gemm_kernel<T><<<grid, 256, 0, s>>>(a.base, a.stride, a.layer_dev, a.nlayers, a.sc_off, a.srow, a.x, (int)a.M,
                                        (int)a.N, (int)a.K, a.y, a.out_bf16);
    return check_launch("gemm");
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
