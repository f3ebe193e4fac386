// gfx950 decode GEMV of the quantized linear at one activation row on 16-row tile planes: y (1, N) = x (1, K) @ W.T
// with float32 accumulation, reference src/mashbox/ops/__init__.py:594-632 (qmatmul) on the weights of reference
// src/mashbox/ops/reference.py:66-70 (Q4_0), :101-103 (Q8_0), :132-149 (Q4_K), :150-159 (Q5_K) and :164-173 (Q6_K),
// and the int8 per-channel linear of reference src/mashbox/models/qwen3_8_27b/model.py:72-82 (dot, then * s), with the
// weights repacked once at load into the 16-row tiles of mbq_layout.h (MBQ_Q4KT, MBQ_Q5KT, MBQ_Q6KT, MBQ_Q40T,
// MBQ_Q8T, MBQ_I8T planes: ops.prepare's default layout). Batches of 2 rows and more run the K-group kernel
// (mbq_kgemm.hip) on the same planes.
//
// HBM-bound, as the row-major GEMV (mbq_gemv.hip): every weight byte is read once, 16 bytes per lane, each wave-wide
// load one KiB (non-temporal).
//
// Work split. A block owns whole tiles, TB = ceil(tiles / CUs) of them (the last block fewer), so no lane of a load
// holds a row of another block. The block's units (tile, chunk) in tile-major order are cut into W equal contiguous
// ranges, one per wave: consecutive chunks of a tile are consecutive KiB of the planes, so every wave streams one
// contiguous run, and the waves of a block carry the same number of units. Lane l of a wave takes row l / 4 of the
// tile and quarter l % 4 of the chunk: 16 bytes of quants, one 32-value unit of the nibble types, 2 x 8 values of Q8_0
// (one per block of the chunk), 16 values of int8. D units are in flight per wave (registers; every load is issued,
// past the wave's range at an offset out of the buffer's range: zero, no traffic, so the compiler's vmcnt waits count
// exactly the units ahead). x sits in LDS for the whole block (read once from L2), with the sums of its 32-value
// units for the nibble types' offsets; a lane reads its unit's x one unit ahead. When a wave's range leaves a tile,
// each row's sum over its 4 lanes (a DPP quad) goes to LDS; at the end the block adds a row's parts in wave order (a
// fixed order: the result does not depend on timing) and stores it. No block exchanges anything with another: no
// workspace, so mbq_matmul_noalloc runs it as it is.
//
// Arithmetic: per unit the row-major GEMV's (float32 accumulation with v_dot2_f32_bf16):
//   Q4_K, Q5_K   (128 + q) as bfloat16 pairs; y += (d sc) * sum(x (128 + q)) - (128 d sc + dmin m) * sum(x)
//   Q4_0         the Q4_K pairs; y += d * sum(x (128 + q)) - 136 d * sum(x)
//   Q6_K         per 16-value half (one scale): y += (d sc) * sum(x (128 + q)) - 160 (d sc) * sum(x)
//   Q8_0, int8   exact bfloat16 pairs of the int8 quants; Q8_0 y += d * sum(x q) per block, int8 the row scale at the end
//
// Measured on MI355X (Q4_K tiles, one 27B-class layer at one row, graph-replayed): q 7.5, k 5.2, o 8.1, gate 12.9,
// down 14.9 us against 9.0, 7.0, 11.0, 15.2 and 17.1 us on the K-group kernel, and 7.4, 4.3, 6.7, 12.7 and 14.2 us for
// the row-major GEMV on row-major planes. Deeper pipelines were slower (8 units in flight: +5-20 %), and so were blocks
// of one tile (more blocks than CUs).
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <algorithm>
#include <type_traits>
#include <utility>

#include "mbq_device.h"
#include "mbq_launch.h"
#include "mbq_layout.h"

namespace mbq {

template <int T> constexpr int tg_cw() { return (T == T_Q8T || T == T_I8T) ? 64 : 128; }   // K values per chunk
constexpr int TG_XB = 4;                       // 16-byte pieces of x per thread per staging batch
constexpr size_t TG_LDS_MAX = 160 * 1024 - 1024;

struct TgArgs {
    const uint8_t* base;        // planes (host layer applied)
    int64_t stride;             // bytes between stacked weights (layer_dev)
    const int32_t* layer_dev;
    int nlayers;
    int64_t sc_off, hi_off, d_off;
    int64_t wbytes;             // bytes of one weight's planes
    const uint16_t* x;
    int N, K, KP, TB;           // rows, columns, columns padded to whole chunks, tiles per block
    void* y;
    int out_bf16;
};

template <class F, int... P>
__device__ __forceinline__ void tg_each(F&& f, std::integer_sequence<int, P...>) {
    (f(std::integral_constant<int, P>{}), ...);
}

// 4 int8 quants (one dword) -> 2 bfloat16 pairs, exact
__device__ __forceinline__ void tg_i8x4(uint32_t w, uint32_t* lo, uint32_t* hi) {
    *lo = pack_bf16((float)(int8_t)(w & 0xFFu), (float)(int8_t)((w >> 8) & 0xFFu));
    *hi = pack_bf16((float)(int8_t)((w >> 16) & 0xFFu), (float)(int8_t)(w >> 24));
}

template <int T, int W, int D>
__global__ __launch_bounds__(64 * W, 1) void tgemv_kernel(const TgArgs g) {
    extern __shared__ __attribute__((aligned(16))) uint8_t tg_lds[];
    constexpr int NT = 64 * W, CW = tg_cw<T>();
    constexpr bool Q4K = T == T_Q4KT, Q5 = T == T_Q5KT, Q6 = T == T_Q6KT, Q40 = T == T_Q40T, Q8 = T == T_Q8T;
    constexpr bool NIB = Q4K || Q5 || Q6 || Q40;          // nibble units of 32 values (x sums needed)
    const int N = g.N, K = g.K, KP = g.KP;
    const int lane = threadIdx.x & 63, tid = threadIdx.x;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int rl = lane >> 2, pu = lane & 3;              // the lane's row of the tile, quarter of the chunk
    const int tiles = (N + 15) >> 4;
    const int t0 = blockIdx.x * g.TB, nt = max(0, min(g.TB, tiles - t0));
    const int r0 = 16 * t0, r1 = min(N, 16 * (t0 + nt));
    const int KC = KP / CW, SB = K >> 8, U = nt * KC;
    const int ua = wave * U / W, ub = (wave + 1) * U / W;  // this wave's units [ua, ub)

    const int64_t lo = layer_offset(g.stride, g.layer_dev, g.nlayers);
    const bool ok = lo >= 0;
    const uint8_t* wb = g.base + (ok ? lo : 0);
    const rsrc_t wr = make_rsrc(wb, (uint32_t)g.wbytes);
    const rsrc_t xr = make_rsrc(g.x, (uint32_t)K * 2u);
    uint16_t* xl = reinterpret_cast<uint16_t*>(tg_lds);                     // KP values of x (zero past K)
    float* us = reinterpret_cast<float*>(tg_lds + 2 * (size_t)KP);          // per 32-value unit: its sum (Q6_K: the
                                                                             // sums of its two halves)
    float* parts = us + KP / 16;                                             // TB x W x 16 row parts

    // the weight stream: unit u of the block = (tile t0 + u / KC, chunk u % KC); its bytes for lane l
    struct Raw { u32x4 q; u32x4 h; u32x2 h2; uint32_t s, d; };
    int lt = ua / KC, lc = ua - lt * KC;                                     // next unit to load
    auto load = [&](Raw& R, int u) __attribute__((always_inline)) {
        const bool live = ok && u < ub;                                      // wave-uniform
        const uint32_t t = (uint32_t)(t0 + lt), tc = t * (uint32_t)KC + (uint32_t)lc;
        auto v = [&](uint32_t off) { return live ? off : OOB_VOFF; };
        R.q = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(wr, v((uint32_t)lane * 16u), tc * 1024u, 2));
        if constexpr (Q4K || Q5)                                             // the row's super-block header
            R.h = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(
                      wr, v((uint32_t)rl * 16u), (uint32_t)g.sc_off + (t * (uint32_t)SB + ((uint32_t)lc >> 1)) * 256u, 0));
        if constexpr (Q5)                                                    // the unit's high-bit word
            R.s = (uint32_t)__builtin_amdgcn_raw_buffer_load_b32(wr, v((uint32_t)rl * 16u + (uint32_t)pu * 4u),
                                                                  (uint32_t)g.hi_off + tc * 256u, 2);
        if constexpr (Q6) {                                                  // high bits, 2 sub-block scales, d
            R.h2 = __builtin_bit_cast(u32x2, __builtin_amdgcn_raw_buffer_load_b64(
                       wr, v((uint32_t)rl * 32u + (uint32_t)pu * 8u), (uint32_t)g.hi_off + tc * 512u, 2));
            R.s = bload2(wr, v((uint32_t)rl * 8u + (uint32_t)pu * 2u), (uint32_t)g.sc_off + tc * 128u);
            R.d = bload2(wr, v((uint32_t)rl * 2u), (uint32_t)g.d_off + (t * (uint32_t)SB + ((uint32_t)lc >> 1)) * 32u);
        }
        if constexpr (Q40) R.d = bload2(wr, v((uint32_t)rl * 8u + (uint32_t)pu * 2u), (uint32_t)g.sc_off + tc * 128u);
        if constexpr (Q8)                                                    // the row's two block scales
            R.d = (uint32_t)__builtin_amdgcn_raw_buffer_load_b32(wr, v((uint32_t)rl * 4u), (uint32_t)g.sc_off + tc * 64u, 0);
        if (++lc == KC) { lc = 0; ++lt; }
    };

    // x into LDS with the sums of its 32-value units (four adjacent pieces: a lane quad; Q6_K the sums of the units'
    // halves, two pieces each), one barrier. The first batch of x loads is issued before the first units' weights, so
    // its wait does not cover them.
    const int npc = KP >> 3;                                                 // 16-byte pieces of x
    auto stage_x = [&](const u32x4* xin, int b) __attribute__((always_inline)) {
#pragma unroll
        for (int i = 0; i < TG_XB; ++i) {
            const int p = tid + NT * (TG_XB * b + i);                        // p & 3 == lane & 3
            float s = 0.f, h = 0.f;
            if constexpr (NIB) {
#pragma unroll
                for (int e = 0; e < 4; ++e) s = dot2(xin[i][e], BF16_ONES, s);
                s += dpp_f<0xB1, 0xF>(s);                                    // pieces 2j, 2j + 1: a half
                h = dpp_f<0x4E, 0xF>(s);                                     // the quad's other half
            }
            if (p < npc) {
                *reinterpret_cast<u32x4*>(xl + 8 * p) = xin[i];
                if (NIB && (p & 3) == 0) {
                    if constexpr (Q6) *reinterpret_cast<float2*>(us + 2 * (p >> 2)) = float2{s, h};
                    else us[p >> 2] = s + h;
                }
            }
        }
    };
    auto load_x = [&](u32x4* xin, int b) __attribute__((always_inline)) {
#pragma unroll
        for (int i = 0; i < TG_XB; ++i) {
            const int p = tid + NT * (TG_XB * b + i);
            xin[i] = bload16(xr, p < npc ? (uint32_t)p * 16u : OOB_VOFF, 0);   // past K: zero
        }
    };
    u32x4 xin[TG_XB];
    load_x(xin, 0);
    Raw R[D];
    tg_each([&](auto J) __attribute__((always_inline)) {
        if constexpr (decltype(J)::value < D - 1) load(R[decltype(J)::value], ua + decltype(J)::value);
    }, std::make_integer_sequence<int, D>{});
    stage_x(xin, 0);
    for (int b = 1; TG_XB * NT * b < npc; ++b) {
        load_x(xin, b);
        stage_x(xin, b);
    }
    __syncthreads();

    // x of the unit being computed, read one unit ahead: nibble types 32 values (4 pieces) and their sum (Q6_K the
    // sums of the two halves); Q8_0 8 values of each block; int8 16 values
    constexpr int XP = NIB ? 4 : 2;
    u32x4 xv[XP];
    float xa = 0.f;
    float2 x2 = float2{0.f, 0.f};
    auto read_x = [&](int c) __attribute__((always_inline)) {
        if constexpr (NIB) {
            const uint16_t* xp = xl + CW * c + 32 * pu;
#pragma unroll
            for (int i = 0; i < 4; ++i) xv[i] = *reinterpret_cast<const u32x4*>(xp + 8 * i);
            if constexpr (Q6) x2 = *reinterpret_cast<const float2*>(us + 2 * (4 * c + pu));
            else xa = us[4 * c + pu];
        } else if constexpr (Q8) {
            xv[0] = *reinterpret_cast<const u32x4*>(xl + 64 * c + 8 * pu);
            xv[1] = *reinterpret_cast<const u32x4*>(xl + 64 * c + 32 + 8 * pu);
        } else {
            xv[0] = *reinterpret_cast<const u32x4*>(xl + 64 * c + 16 * pu);
            xv[1] = *reinterpret_cast<const u32x4*>(xl + 64 * c + 16 * pu + 8);
        }
    };
    int ct = ua / KC, cc = ua - ct * KC;                                     // unit being computed (tile, chunk)
    read_x(cc);
    const Q4kSel sel0 = q4k_sel(pu), sel1 = q4k_sel(4 + pu);                // sub-block pu of an even / odd chunk
    const uint32_t kmask = in_vgpr(0x000F000Fu), kmagic = in_vgpr(0x43004300u), c43 = in_vgpr(0x43434343u);
    float acc = 0.f;
    auto flush = [&]() __attribute__((always_inline)) {                     // the rows' sums of tile ct, this wave
        float v = acc + dpp_f<0xB1, 0xF>(acc);
        v += dpp_f<0x4E, 0xF>(v);
        if (pu == 0) parts[(ct * W + wave) * 16 + rl] = v;
        acc = 0.f;
    };
    auto process = [&](const Raw& Wr) __attribute__((always_inline)) {
        u32x4 x[XP];
#pragma unroll
        for (int i = 0; i < XP; ++i) x[i] = xv[i];
        const float sx = xa;
        const float2 sh = x2;
        read_x(cc + 1 == KC ? 0 : cc + 1);                                   // the next unit's x (a chunk in range)
        if constexpr (Q4K || Q5 || Q40) {
            float dsc, cst;
            if constexpr (Q40) {
                dsc = f16f(Wr.d);
                cst = 136.f * dsc;                                           // (128 + q) d - 136 d = (q - 8) d
            } else {
                uint32_t sc, mn;
                q4k_scale_min_sel(Wr.h[1], Wr.h[2], Wr.h[3], (cc & 1) ? sel1 : sel0, &sc, &mn);
                dsc = f16f(Wr.h[0]) * (float)sc;                             // exact
                cst = 128.f * dsc + f16f(Wr.h[0] >> 16) * (float)mn;
            }
            float P0 = 0.f, P1 = 0.f;
            if constexpr (Q5) {
#pragma unroll
                for (int t = 0; t < 4; ++t) {
                    uint32_t lo8, hi8;
                    q5k_bytes(Wr.q[t], Wr.s, t, &lo8, &hi8);
                    P0 = dot2(b128_pair(lo8, c43, 0), x[t][0], P0);
                    P0 = dot2(b128_pair(lo8, c43, 1), x[t][1], P0);
                    P1 = dot2(b128_pair(hi8, c43, 0), x[t][2], P1);
                    P1 = dot2(b128_pair(hi8, c43, 1), x[t][3], P1);
                }
            } else {
#pragma unroll
                for (int t = 0; t < 4; ++t)
#pragma unroll
                    for (int pp = 0; pp < 4; ++pp) {
                        const uint32_t pr = ((Wr.q[t] >> (4 * pp)) & kmask) | kmagic;
                        float& Pm = (pp & 1) ? P1 : P0;
                        Pm = dot2(pr, x[t][pp], Pm);
                    }
            }
            acc = __builtin_fmaf(dsc, P0 + P1, __builtin_fmaf(-cst, sx, acc));
        } else if constexpr (Q6) {
            const float d = f16f(Wr.d);
            const float ds0 = d * (float)(int8_t)(Wr.s & 0xFFu), ds1 = d * (float)(int8_t)((Wr.s >> 8) & 0xFFu);   // exact
            float A0 = 0.f, B0 = 0.f, A1 = 0.f, B1 = 0.f;                    // halves 0 / 1, quant bytes lo / hi
#pragma unroll
            for (int t = 0; t < 4; ++t) {
                uint32_t lo8, hi8;
                q6k_bytes(Wr.q[t], Wr.h2[t >> 1], t, &lo8, &hi8);
                float& A = t < 2 ? A0 : A1;
                float& B = t < 2 ? B0 : B1;
                A = dot2(b128_pair(lo8, c43, 0), x[t][0], A);
                A = dot2(b128_pair(lo8, c43, 1), x[t][1], A);
                B = dot2(b128_pair(hi8, c43, 0), x[t][2], B);
                B = dot2(b128_pair(hi8, c43, 1), x[t][3], B);
            }
            acc = __builtin_fmaf(ds0, A0 + B0, __builtin_fmaf(-160.f * ds0, sh.x, acc));
            acc = __builtin_fmaf(ds1, A1 + B1, __builtin_fmaf(-160.f * ds1, sh.y, acc));
        } else {
            // Q8_0: dwords 0-1 the lane's 8 values of the chunk's first block, 2-3 of its second; int8: 16 values
            float P0 = 0.f, P1 = 0.f;
#pragma unroll
            for (int t = 0; t < 4; ++t) {
                uint32_t b0, b1;
                tg_i8x4(Wr.q[t], &b0, &b1);
                float& Pm = (t < 2) ? P0 : P1;
                Pm = dot2(b0, x[t >> 1][2 * (t & 1)], Pm);
                Pm = dot2(b1, x[t >> 1][2 * (t & 1) + 1], Pm);
            }
            if constexpr (Q8) acc = __builtin_fmaf(f16f(Wr.d >> 16), P1, __builtin_fmaf(f16f(Wr.d), P0, acc));
            else acc += P0 + P1;
        }
        if (++cc == KC) {
            flush();
            cc = 0;
            ++ct;
        }
    };
    // unit k + j computes from register set j while the set of unit k + j - 1 refills with unit k + j + D - 1
    for (int k = ua; k < ub; k += D) {
        tg_each([&](auto J) __attribute__((always_inline)) {
            constexpr int j = decltype(J)::value;
            load(R[(j + D - 1) % D], k + j + D - 1);
            if (k + j < ub) process(R[j]);
        }, std::make_integer_sequence<int, D>{});
    }
    if (cc != 0) flush();                                                    // the range ends inside a tile
    __syncthreads();

    // each row: the parts of the waves whose ranges meet its tile, in wave order, times the int8 row scale
    for (int r = r0 + tid; r < r1; r += NT) {
        const int tl = (r >> 4) - t0;
        float v = 0.f;
        for (int w = 0; w < W; ++w) {
            const int wa = w * U / W, wz = (w + 1) * U / W;
            if (wa < (tl + 1) * KC && wz > tl * KC) v += parts[(tl * W + w) * 16 + (r & 15)];
        }
        if constexpr (T == T_I8T) v *= row_scale<T>(nullptr, wb, g.sc_off, r);
        store_y(g.y, r, ok ? v : __builtin_nanf(""), g.out_bf16);
    }
}

// ------------------------------------------------------------------------------------------------------ launchers
// The launch of one call: tiles per block, and the block shape. Blocks of 16 waves with 3 units in flight each when
// the blocks cover at most 70 % of the CUs and hold at least 64 units (MI355X, Q4_K tiles: 5120 rows, K = 6144 8.5 ->
// 8.1 us, K = 17408 16.4 -> 14.9 us), else 8 waves with 5 in flight (6144 x 5120 7.5 us against 7.7, 17408 x 5120 12.9
// against 13.5, 1024 x 5120 5.2 against 5.8).
struct TgPlan { int TB, P, W, KP; size_t lds; };
static bool tg_plan(int t, const Args& a, TgPlan* p) {
    if (a.M != 1 || a.N < 1 || a.K < 1 || a.wbytes > BUF_MAX_BYTES || a.K * 2 > BUF_MAX_BYTES) return false;
    const int cw = (t == T_Q8T || t == T_I8T) ? 64 : 128;
    const int64_t KP = (a.K + cw - 1) / cw * cw, KC = KP / cw;
    const int64_t tiles = (a.N + 15) / 16, cus = cus_of_device();
    const int64_t TB = (tiles + cus - 1) / cus, P = (tiles + TB - 1) / TB;
    const bool wide = 10 * P <= 7 * cus && TB * KC >= 64;
    const int W = wide ? 16 : 8;
    const size_t lds = (size_t)KP * 2 + (size_t)KP / 16 * 4 + (size_t)TB * W * 16 * 4;
    if (lds > TG_LDS_MAX) return false;
    *p = TgPlan{(int)TB, (int)P, W, (int)KP, lds};
    return true;
}

template <int T, int W, int D>
static int tg_launch(const Args& a, const TgPlan& p, hipStream_t s) {
    auto kern = tgemv_kernel<T, W, D>;
    static std::atomic<uint64_t> lds_set{0};
    if (set_lds_limit((const void*)kern, p.lds, lds_set) != hipSuccess)
        return set_error(MBQ_LAUNCH_FAIL, "tile GEMV: %zu bytes of LDS refused", p.lds);
    TgArgs g{a.base, a.stride, a.layer_dev, a.nlayers, a.sc_off, a.hi_off, a.d_off, a.wbytes, a.x,
             (int)a.N, (int)a.K, p.KP, p.TB, a.y, a.out_bf16};
    kern<<<dim3((unsigned)p.P), 64 * W, p.lds, s>>>(g);
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return set_error(MBQ_LAUNCH_FAIL, "tile GEMV: %s", hipGetErrorString(e));
    return 0;
}

template <int T>
static int tg_launch_t(const Args& a, hipStream_t s) {
    TgPlan p;
    if (!tg_plan(T, a, &p)) return set_error(MBQ_BAD_ARG, "tile GEMV: no plan for %lld x %lld at %lld rows", (long long)a.N,
                                             (long long)a.K, (long long)a.M);
    return p.W == 16 ? tg_launch<T, 16, 3>(a, p, s) : tg_launch<T, 8, 5>(a, p, s);
}

bool tgemv_runs(int t, const Args& a) {
    TgPlan p;
    return tiled_type(t) && forced_gemm_kernel() == K_AUTO && tg_plan(t, a, &p);
}

int launch_tgemv(int t, const Args& a, hipStream_t s) {
    switch (t) {
        case T_Q4KT: return tg_launch_t<T_Q4KT>(a, s);
        case T_Q5KT: return tg_launch_t<T_Q5KT>(a, s);
        case T_Q6KT: return tg_launch_t<T_Q6KT>(a, s);
        case T_Q40T: return tg_launch_t<T_Q40T>(a, s);
        case T_Q8T: return tg_launch_t<T_Q8T>(a, s);
        case T_I8T: return tg_launch_t<T_I8T>(a, s);
    }
    return set_error(MBQ_BAD_ARG, "tile GEMV: type %d is not a tiled plane type", t);
}

}  // namespace mbq
