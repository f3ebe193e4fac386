// gfx950 (CDNA4) kernels of the quantized linear: decode GEMV, dequant and device repack (the MFMA GEMM: mbq_gemm.hip).
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


// ---------------------------------------------------------------------------------------------------- decode GEMV
// One wave owns one weight row and the whole K; the block's 8 waves own 8 consecutive rows and share x, staged once
// into LDS as bfloat16. The 64 lanes of a wave stride over the row's 16-byte units (Q4_K: a sub-block of 32 quants;
// Q8_0 / int8: 16 quants), so each wave-wide load reads 1 KiB of the row contiguously. Loads run in double-buffered
// stages of CH units per lane: the next stage's loads are in flight while the current stage computes, so several HBM
// round trips overlap in every wave. Quants become bfloat16 pairs in registers (exact) and meet x through
// v_dot2_f32_bf16 with float32 accumulation; block scales apply once per unit in float32; the lanes' partial sums are
// reduced across the wave at the end. Up to M = 4 activation rows share each weight load.
constexpr int GV_WAVES = 8;

template <int T> struct GvUnit;
template <> struct GvUnit<T_Q4_K> { u32x4 q, meta; };
template <> struct GvUnit<T_Q8_0> { u32x4 q; uint32_t d; };
template <> struct GvUnit<T_INT8> { u32x4 q; };

// unit loads from a row's planes: q and sr are wave-uniform bases (scalar registers), v the lane's unit index
template <int T>
__device__ __forceinline__ void gv_load(GvUnit<T>& g, const uint8_t* __restrict__ q, const uint8_t* __restrict__ sr, uint32_t v) {
    g.q = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(q + v * 16u));
    if constexpr (T == T_Q4_K) g.meta = ld16(sr + (v >> 3) * 16u);
    if constexpr (T == T_Q8_0) g.d = *reinterpret_cast<const uint16_t*>(sr + (v >> 1) * 2u);
}

// 16-byte chunk t of unit u of activation row m. In LDS (XL) the chunks are stored chunk-major, [m][t][u], so the
// lanes of a wave (consecutive units) read consecutive 16-byte words without bank conflicts; from global memory
// they are read in place, row-major.
template <bool XL, int UW>
__device__ __forceinline__ u32x4 x_chunk(const uint16_t* xs, int K, int U, int m, int t, int u) {
    if constexpr (XL)
        return ld16(xs + ((int64_t)(m * (UW / 8) + t) * U + u) * 8);
    else
        return ld16(xs + (int64_t)m * K + (int64_t)u * UW + t * 8);
}

// adds unit u's contribution for the M activation rows to acc (act = false: the lane has no unit here and adds an
// exact zero: its scale is zeroed, the quants it holds are a valid unit's). xs: the activations (x_chunk); xsum: M rows
// of the per-unit sums of x (float32), precomputed by the block, which take the +128 offset of the quant pairs back
// out. The dot2 chains are split in two independent accumulators.
template <int T, int M, bool XL>
__device__ __forceinline__ void gv_compute(const GvUnit<T>& g, const uint16_t* xs, const float* xsum, int K, int U, int u,
                                           bool act, const Q4kSel& sel, uint32_t kmask, uint32_t kmagic, float* acc) {
    if constexpr (T == T_Q4_K) {
        uint32_t sc, mn;
        q4k_scale_min_sel(g.meta[1], g.meta[2], g.meta[3], sel, &sc, &mn);
        float dsc = f16f(g.meta[0]) * (float)sc;        // exact
        const float dm = f16f(g.meta[0] >> 16) * (float)mn;    // exact
        float c = 128.f * dsc + dm;
        dsc = act ? dsc : 0.f;
        c = act ? c : 0.f;
#pragma unroll
        for (int m = 0; m < M; ++m) {
            float P0 = 0.f, P1 = 0.f;
#pragma unroll
            for (int t = 0; t < 4; t += 2) {
                const u32x4 xa = x_chunk<XL, 32>(xs, K, U, m, t, u), xb = x_chunk<XL, 32>(xs, K, U, m, t + 1, u);
#pragma unroll
                for (int p = 0; p < 4; ++p) {
                    P0 = dot2((((g.q[t] >> (4 * p)) & kmask) | kmagic), xa[p], P0);
                    P1 = dot2((((g.q[t + 1] >> (4 * p)) & kmask) | kmagic), xb[p], P1);
                }
            }
            acc[m] += dsc * (P0 + P1) - c * xsum[m * U + u];
        }
    } else {
        float d = 1.f;
        if constexpr (T == T_Q8_0) d = f16f(g.d);
        d = act ? d : 0.f;
        u32x4 q;
#pragma unroll
        for (int t = 0; t < 4; ++t) q[t] = g.q[t] ^ 0x80808080u;
#pragma unroll
        for (int m = 0; m < M; ++m) {
            const u32x4 x0 = x_chunk<XL, 16>(xs, K, U, m, 0, u), x1 = x_chunk<XL, 16>(xs, K, U, m, 1, u);
            float P0 = 0.f, P1 = 0.f;
#pragma unroll
            for (int t = 0; t < 2; ++t)
#pragma unroll
                for (int p = 0; p < 2; ++p) {
                    P0 = dot2(u8_pair(q[t], p), x0[(t << 1) + p], P0);
                    P1 = dot2(u8_pair(q[t + 2], p), x1[(t << 1) + p], P1);
                }
            acc[m] += d * ((P0 + P1) - 128.f * xsum[m * U + u]);
        }
    }
}

// Persistent decode GEMV: the grid is exactly the blocks the GPU holds at once, so there is no second round of
// blocks. Block b owns rows [b*N/P, (b+1)*N/P); each row is cut into S parts of at most 64*CH units, so one part is
// one wave-wide batch of CH 16-byte loads per lane. The block's waves take the (row, part) items round-robin, with
// the next item's loads in flight while the current one computes; each item's partial sums are reduced across the
// wave with DPP into LDS, and the block adds the S parts of each row at the end. Item bookkeeping is wave-uniform
// (scalar registers); lanes only form 32-bit unit offsets.
template <int T, int M, int CH, bool XL>
__global__ __launch_bounds__(64 * GV_WAVES, 2) void gemv_kernel(const uint8_t* __restrict__ base, int64_t stride,
                                                            const int32_t* __restrict__ layer_dev, int nlayers,
                                                            int64_t sc_off, const float* __restrict__ srowscale,
                                                            const uint16_t* __restrict__ x, int N, int K, int S,
                                                            void* __restrict__ y, int out_bf16) {
    extern __shared__ __attribute__((aligned(16))) uint16_t lds[];   // [x: M x K bf16] [xsum: M x U f32] [parts]
    constexpr int UW = (T == T_Q4_K) ? 32 : 16;
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int P = gridDim.x;
    const int r0 = (int)((int64_t)blockIdx.x * N / P), r1 = (int)((int64_t)(blockIdx.x + 1) * N / P);
    const int64_t lo = layer_offset(stride, layer_dev, nlayers);
    const bool ok = lo >= 0;
    base += ok ? lo : 0;
    const int U = K / UW;
    const int PU = (U + S - 1) / S;           // units per part (<= 64 * CH)
    const int items = (r1 - r0) * S;
    const int64_t qstride = (int64_t)U * 16;
    const int64_t sstride = (T == T_Q4_K) ? (int64_t)(K >> 8) * 16 : (int64_t)(K >> 5) * 2;
    float* xsum = reinterpret_cast<float*>(lds + (XL ? M * K : 0));
    float* parts = xsum + M * U;              // (r1 - r0) x S x M

    const uint32_t kmask = in_vgpr(0x000F000Fu), kmagic = in_vgpr(0x43004300u);
    GvUnit<T> A[CH], B[CH];
    // item it (wave-uniform) -> row, first unit u0, unit count nu
    auto load = [&](GvUnit<T>* G, int it) {
        const int row = r0 + it / S, u0 = (it % S) * PU, nu = min(PU, U - u0);
        const uint8_t* q = base + row * qstride;
        const uint8_t* sr = base + sc_off + row * sstride;
#pragma unroll
        for (int i = 0; i < CH; ++i) {
            if (64 * i >= nu) break;           // wave-uniform: no lane has a unit in this slot
            const int li = (lane + 64 * i < nu) ? lane + 64 * i : 0;
            gv_load<T>(G[i], q, sr, (uint32_t)(u0 + li));
        }
    };

    const bool any = ok && wave < items;
    if (any) load(A, wave);

    // per-unit sums of x (float32), and in LDS mode the activations themselves, chunk-major [m][t][u]
    for (int e = threadIdx.x; e < M * U; e += 64 * GV_WAVES) {
        const int m = e / U, u = e - m * U;
        const uint16_t* xu = x + (int64_t)m * K + (int64_t)u * UW;
        float sum = 0.f;
#pragma unroll
        for (int t = 0; t < UW / 8; ++t) {
            const u32x4 v = ld16(xu + t * 8);
            if constexpr (XL) st16(lds + ((m * (UW / 8) + t) * U + u) * 8, v);
#pragma unroll
            for (int p = 0; p < 4; ++p) sum = dot2(v[p], BF16_ONES, sum);
        }
        xsum[e] = sum;
    }
    __syncthreads();
    const uint16_t* xa = XL ? lds : x;

    auto finish = [&](const GvUnit<T>* G, int it) {
        const int rl = it / S, p = it % S, u0 = p * PU, nu = min(PU, U - u0);
        float acc[CH][M];
#pragma unroll
        for (int i = 0; i < CH; ++i)
#pragma unroll
            for (int m = 0; m < M; ++m) acc[i][m] = 0.f;
        const Q4kSel sel = q4k_sel((u0 + lane) & 7);   // units advance by 64: the lane's sub-block slot is fixed
#pragma unroll
        for (int i = 0; i < CH; ++i) {
            if (64 * i >= nu) break;           // wave-uniform
            const bool act = lane + 64 * i < nu;
            const int u = act ? u0 + lane + 64 * i : u0 + lane;   // inactive: a unit of the same slot, scale zeroed
            gv_compute<T, M, XL>(G[i], xa, xsum, K, U, u < U ? u : u0, act, sel, kmask, kmagic, acc[i]);
        }
#pragma unroll
        for (int m = 0; m < M; ++m) {
            float v = 0.f;
#pragma unroll
            for (int i = 0; i < CH; ++i) v += acc[i][m];
            v = wave_sum_dpp(v);
            if (lane == 0) parts[(rl * S + p) * M + m] = v;
        }
    };
    if (any) {
        for (int it = wave; it < items; it += 2 * GV_WAVES) {
            const int nx = it + GV_WAVES;
            if (nx < items) load(B, nx);
            finish(A, it);
            if (nx + GV_WAVES < items) load(A, nx + GV_WAVES);
            if (nx < items) finish(B, nx);
        }
    }
    __syncthreads();
    for (int e = threadIdx.x; e < (r1 - r0) * M; e += 64 * GV_WAVES) {
        const int rl = e / M, m = e - rl * M, n = r0 + rl;
        float v = 0.f;
        for (int p = 0; p < S; ++p) v += parts[(rl * S + p) * M + m];
        const float sc = (T == T_INT8) ? srowscale[n] : 1.f;
        store_y(y, (int64_t)m * N + n, ok ? v * sc : __builtin_nanf(""), out_bf16);
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

// blocks of a GEMV kernel the GPU holds at once (cached per kernel and LDS size)
template <class K>
static int resident_blocks(K kernel, size_t lds) {
    static thread_local struct { const void* k; size_t lds; int n; } cache[32];
    static thread_local int used = 0;
    for (int i = 0; i < used; ++i)
        if (cache[i].k == (const void*)kernel && cache[i].lds == lds) return cache[i].n;
    int dev = 0, cus = 0, per = 0;
    if (hipGetDevice(&dev) != hipSuccess || hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
        hipOccupancyMaxActiveBlocksPerMultiprocessor(&per, kernel, 64 * GV_WAVES, lds) != hipSuccess || per < 1)
        return -1;
    const int n = cus * per;
    if (used < 32) cache[used++] = {(const void*)kernel, lds, n};
    return n;
}

template <int T, int M>
static int launch_gemv_m(const Args& a, hipStream_t s) {
    constexpr int CH = (T == T_Q4_K) ? (M == 1 ? 4 : 2) : (M <= 2 ? 4 : 2);
    const int64_t UW = (T == T_Q4_K) ? 32 : 16;
    const int64_t U = a.K / UW;
    const int S = (int)((U + 64 * CH - 1) / (64 * CH));
    const size_t xbytes = (size_t)M * a.K * 2, sums = (size_t)M * U * 4;
    const bool xl = xbytes + sums <= (size_t)GEMV_MAX_LDS;
    auto kern = xl ? gemv_kernel<T, M, CH, true> : gemv_kernel<T, M, CH, false>;
    // parts: rows per block x S x M floats; the block count depends on the LDS, so settle it in two steps
    size_t lds = (xl ? xbytes : 0) + sums;
    int P = resident_blocks(kern, lds + 4096);
    if (P < 1) return set_error(MBQ_LAUNCH_FAIL, "GEMV occupancy query failed");
    P = (int)std::min<int64_t>(P, a.N);
    const int64_t rows_max = (a.N + P - 1) / P;
    lds += (size_t)rows_max * S * M * 4;
    if (lds > 160 * 1024) return set_error(MBQ_BAD_ARG, "GEMV K = %lld, N = %lld needs too much LDS", (long long)a.K, (long long)a.N);
    kern<<<dim3((unsigned)P), 64 * GV_WAVES, lds, s>>>(a.base, a.stride, a.layer_dev, a.nlayers, a.sc_off, a.srow, a.x,
                                                      (int)a.N, (int)a.K, S, a.y, a.out_bf16);
    return 0;
}

template <int T>
static int launch_t(const Args& a, hipStream_t s) {
    if (a.M <= GEMV_MAX_M) {
        int rc;
        switch (a.M) {
            case 1: rc = launch_gemv_m<T, 1>(a, s); break;
            case 2: rc = launch_gemv_m<T, 2>(a, s); break;
            case 3: rc = launch_gemv_m<T, 3>(a, s); break;
            default: rc = launch_gemv_m<T, 4>(a, s); break;
        }
        return rc ? rc : check_launch("gemv");
    }
    return launch_gemm(T, a, s);
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
