// gfx950 (CDNA4) kernels of the quantized linear: decode GEMV, MFMA GEMM, dequant and device repack.
//
// Semantics follow reference src/mashbox/ops/__init__.py:594-632 (qmatmul: x @ W.T, float32 accumulation) with the
// weights of reference src/mashbox/ops/reference.py:101-103 (Q8_0) and :132-149 (Q4_K), and the int8 per-channel
// linear of reference src/mashbox/models/qwen3_8_27b/model.py:72-82. Plane layouts: mbq_layout.h.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <algorithm>

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

// bytes 2p, 2p+1 of w (int8 already offset to unsigned by ^0x80) -> bfloat16 pair (q + 128), exact
__device__ __forceinline__ uint32_t u8_pair(uint32_t w, int p) {
    const float f0 = (float)((w >> (16 * p)) & 0xFFu);
    const float f1 = (float)((w >> (16 * p + 8)) & 0xFFu);
    return __builtin_amdgcn_perm(__float_as_uint(f1), __float_as_uint(f0), 0x07060302u);
}

// a value the compiler keeps in a VGPR (gfx9 VOP3 instructions take no literal operands, so v_and_or_b32 and v_bfi_b32
// need their constants in registers)
__device__ __forceinline__ uint32_t in_vgpr(uint32_t v) {
    asm volatile("" : "+v"(v));
    return v;
}

// Q4_K scale/min extraction parameters of sub-block j (0..7) of a super-block, computed once per lane
struct Q4kSel {
    bool hi;                 // j >= 4
    uint32_t sh_lo, w_lo, sh_lo_m, sh_hi, w_hi;
};
__device__ __forceinline__ Q4kSel q4k_sel(int j) {
    Q4kSel r;
    const uint32_t sh = 8u * (uint32_t)(j & 3);
    r.hi = j >= 4;
    r.sh_lo = sh;
    r.w_lo = r.hi ? 4u : 6u;
    r.sh_lo_m = sh + (r.hi ? 4u : 0u);
    r.sh_hi = sh + 6u;
    r.w_hi = r.hi ? 2u : 0u;
    return r;
}
// the same values as q4k_scale_min, without branches
__device__ __forceinline__ void q4k_scale_min_sel(uint32_t s0, uint32_t s1, uint32_t s2, const Q4kSel& q, uint32_t* sc,
                                                  uint32_t* mn) {
    *sc = __builtin_amdgcn_ubfe(q.hi ? s2 : s0, q.sh_lo, q.w_lo) | (__builtin_amdgcn_ubfe(s0, q.sh_hi, q.w_hi) << 4);
    *mn = __builtin_amdgcn_ubfe(q.hi ? s2 : s1, q.sh_lo_m, q.w_lo) | (__builtin_amdgcn_ubfe(s1, q.sh_hi, q.w_hi) << 4);
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

template <int CTRL, int ROW_MASK>
__device__ __forceinline__ float dpp_f(float v) {
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, ROW_MASK, 0xF, false));
}

// sum over the 64 lanes of a wave through DPP; the total is returned in every lane (read from lane 63)
__device__ __forceinline__ float wave_sum_dpp(float v) {
    v += dpp_f<0xB1, 0xF>(v);    // quad_perm [1,0,3,2]
    v += dpp_f<0x4E, 0xF>(v);    // quad_perm [2,3,0,1]: every lane holds its quad's sum
    v += dpp_f<0x114, 0xF>(v);   // row_shr:4
    v += dpp_f<0x118, 0xF>(v);   // row_shr:8: lane 15 of each row holds the row's sum
    v += dpp_f<0x142, 0xA>(v);   // row_bcast:15 into rows 1 and 3
    v += dpp_f<0x143, 0xC>(v);   // row_bcast:31 into rows 2 and 3: lane 63 holds the wave's sum
    return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 63));
}

constexpr uint32_t BF16_ONES = 0x3F803F80u;  // bfloat16 pair (1, 1)

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
