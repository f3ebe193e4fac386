// gfx950 decode GEMV of the quantized linear (M <= GEMV_MAX_M activation rows).
//
// y (M, N) = x (M, K) @ W.T with float32 accumulation: reference src/mashbox/ops/__init__.py:594-632 (qmatmul) on the
// weights of reference src/mashbox/ops/reference.py:66-70 (Q4_0), :101-103 (Q8_0), :132-149 (Q4_K), :150-159 (Q5_K) and
// :164-173 (Q6_K), and the int8 per-channel
// linear of reference src/mashbox/models/qwen3_8_27b/model.py:72-82 (dot, then * s). Plane layouts: mbq_layout.h.
//
// HBM-bound: every weight byte is read once, 16 bytes per lane, each wave-wide load 1 KiB of one row (non-temporal).
//
// Work split. A persistent grid; block b owns rows [b N / P, (b + 1) N / P). A row's U units (a unit: 16 bytes of quants
// = 16 int8 values, or 32 Q4_0 / K-quant values) are cut into S parts of PU units, at most 64 CH: one part of one row is
// an item of CH chunks, one chunk = one 16-byte load per lane (lane l takes unit 64 i + l of the part). Wave w always
// takes part w % S (of rows j, j + n, j + 2 n, ... with j = w / S and n the number of waves of that part, 8 / S when S
// divides 8): the x values its lanes
// multiply are the same for every row and are held in registers for the whole kernel (read once from L2; no LDS in
// the inner loop). Rows of few units (K = 2560: 80 units, a second chunk with 16 of 64 lanes busy) are packed R to an
// item instead (S = 1, R in {2, 4}, R U a multiple of 64): R consecutive rows are one run of R U units in every plane,
// lane l of chunk i takes unit f = 64 i + l of the run (row f / U, whose sums the lane adds to that row's), and the
// x a lane multiplies is still the same for every item. The next item's loads (DEPTH - 1 items) are in flight while an item computes; every load is
// unconditional (lanes past a part's end, chunks past it and items past a wave's last row read out of the buffer's
// range: zero, and no memory traffic), so the compiler's vmcnt waits count exactly the next item's loads. An item's sums are reduced across the wave with DPP; with S > 1 the block
// adds a row's parts through LDS at the end.
//
// Arithmetic, float32 accumulation with v_dot2_f32_bf16:
//   int8 / Q8_0   a signed byte convert (one SDWA op per value) and a pack give exact bfloat16 pairs; Q8_0 scales the
//                 unit's sum by d.
//   Q4_K          ((w >> 4p) & 0x000F000F) | 0x43004300 is the bfloat16 pair (128 + q, 128 + q'); per unit
//                 y += (d sc) * sum(x (128 + q)) - (128 d sc + dmin m) * sum(x); the per-unit sums of x are computed
//                 once per wave from its x registers.
//   Q4_0          the Q4_K pairs; per unit (one block) y += d * sum(x (128 + q)) - 136 d * sum(x).
//   Q5_K          q5k_bytes (a rotate and a bit-field insert per four values) then one byte permute per pair make
//                 (128 + q, 128 + q'); per unit the Q4_K sum.
//   Q6_K          an AND, an AND-OR and at most one shift per four values leave the 6-bit quants as bytes
//                 (q6k_bytes), and one byte permute per pair makes the bfloat16 pair (128 + q, 128 + q'); per half unit
//                 (16 values, one scale) y += (d sc) * sum(x (128 + q)) - 160 (d sc) * sum(x).
// A lane that holds no unit of a part (the part's last chunk) reads zero and has its scale zeroed.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <algorithm>
#include <type_traits>

#include "mbq_device.h"
#include "mbq_launch.h"
#include "mbq_layout.h"

namespace mbq {

constexpr int GV_WAVES = 8, GV_THREADS = 64 * GV_WAVES;
// grid: one block per CU, two when every wave of the two still gets enough items (part rows): at least 16 at one
// activation row, 8 at 2-4 rows, 3.5 with 3 parts per row (gv_two_blocks). Measured on MI355X, one block against two:
// a 151936-row output head at one row 10-14 % faster with two; 17408 x 5120 at 2 rows (2 parts, 8.5 items per wave)
// 0-7 % faster, at 3-4 rows (3 parts, 12.8) 12-14 %; 5120-6144 rows at 3-4 rows (3 parts, 3.8-4.5) 0-11 %; at 2-3
// items per wave (2 parts: 4096-6144 rows at 2-3 rows) 5-10 % slower. With 3 parts a block's 8 waves take them 3 / 3 /
// 2, so the waves of the third part carry half the rows each: a second block per CU fills in behind them.
constexpr int GV_ITEMS_2BPC = 16, GV_ITEMS_2BPC_M = 8;
inline bool gv_two_blocks(int64_t N, int S, int M, int cus) {
    const int64_t items = N * S, waves2 = 2 * (int64_t)cus * GV_WAVES;   // part rows; waves of two blocks per CU
    return items >= waves2 * GV_ITEMS_2BPC || (M > 1 && items >= waves2 * GV_ITEMS_2BPC_M) || (S == 3 && 2 * items >= waves2 * 7);
}
constexpr int GV_ITEM_CHUNKS = 3;     // parts of at most 3 chunks: items of 2-3 KiB (measured best on MI355X)

template <int T> constexpr int gv_uw() { return unit32(T) ? 32 : 16; }   // values per 16-byte unit
template <int T> constexpr int gv_tpu() { return gv_uw<T>() / 8; }            // 16-byte x chunks per unit
// chunks per item that the registers hold (x of M rows for CH chunks, and two items' loads in flight)
template <int T> constexpr int gv_chmax(int M) {
    return unit32(T) ? (M == 1 ? 5 : M == 2 ? 2 : 1) : T == T_Q8_0 ? (M == 1 ? 5 : M == 2 ? 3 : 2) : (M == 1 ? 6 : M == 2 ? 4 : M == 3 ? 3 : 2);
}

struct GvArgs {
    const uint8_t* base;        // planes (host layer applied)
    int64_t stride;             // bytes between stacked weights (layer_dev)
    const int32_t* layer_dev;
    int nlayers;
    int64_t sc_off;             // scale plane offset
    int64_t hi_off, d_off;      // Q6_K high-bit and super-block scale planes
    int64_t wbytes;             // bytes of one weight's planes (int8: N x K)
    const float* srow;          // int8 per-row scales
    const uint16_t* x;
    int N, K, S, PU;            // rows, columns, parts per row (divides 8), units per part
    void* y;
    int out_bf16;
};

// 4 int8 quants (one dword) -> 2 bfloat16 pairs, exact
__device__ __forceinline__ void gv_i8x4(uint32_t w, uint32_t* lo, uint32_t* hi) {
    *lo = pack_bf16((float)(int8_t)(w & 0xFFu), (float)(int8_t)((w >> 8) & 0xFFu));
    *hi = pack_bf16((float)(int8_t)((w >> 16) & 0xFFu), (float)(int8_t)(w >> 24));
}

template <int T, int M, int CH, int DEPTH = 2, int R = 1>
__global__ __launch_bounds__(GV_THREADS, 2) void gemv_kernel(const GvArgs g) {
    extern __shared__ float parts[];                                  // S > 1: (r1 - r0) x S x M
    constexpr int UW = gv_uw<T>(), TPU = gv_tpu<T>();
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int N = g.N, K = g.K, S = g.S, PU = g.PU;
    const int P = gridDim.x;
    // block b owns rows [r0, r1): N / P of them, whole groups of R rows (the last group may end past N)
    const int G = (N + R - 1) / R;
    const int r0 = R * (int)((int64_t)blockIdx.x * G / P), r1 = min(N, R * (int)((int64_t)(blockIdx.x + 1) * G / P));
    const int64_t lo = layer_offset(g.stride, g.layer_dev, g.nlayers);
    const bool ok = lo >= 0;
    const rsrc_t wr = make_rsrc(g.base + (ok ? lo : 0), (uint32_t)g.wbytes);
    const rsrc_t xr = make_rsrc(g.x, (uint32_t)((int64_t)M * K * 2));
    const int U = K / UW;
    const uint32_t qstride = (uint32_t)U * 16u;
    const uint32_t sstride = (T == T_Q4_K || T == T_Q5_K) ? (uint32_t)(K >> 8) * 16u : (T == T_Q6_K) ? (uint32_t)(K >> 4) : (uint32_t)(K >> 5) * 2u;

    // this wave's part and its units
    const int part = wave % S, rstep = (GV_WAVES - part + S - 1) / S;   // the waves that take this part
    const int u0 = part * PU, nu = max(0, min(PU, U - u0));
    const int lastc = max(0, (nu - 1) >> 6);                         // last chunk with a unit of the part
    const int nrows = r1 - r0, first = wave / S, ngroups = (nrows + R - 1) / R;
    const int nit = first < ngroups ? (ngroups - 1 - first) / rstep + 1 : 0;   // rows (groups of R rows) this wave takes
    const bool any = ok && nit > 0 && nu > 0;

    struct Raw { u32x4 q[CH]; u32x4 meta[CH]; uint32_t d[CH]; u32x2 h[CH]; uint32_t s[CH]; };
    // Lane offsets of a load. The lanes past the part's last unit (in its last chunk), the chunks past that one and the
    // items past the wave's last row take an offset beyond the buffer's range: such a load returns zero without
    // touching memory, so no byte is fetched twice, and the load stays unconditional.
    const bool lane_in = 64 * lastc + lane < nu;                       // the lane's unit of the last chunk exists
    const uint32_t vq = (uint32_t)lane * 16u, vq_last = lane_in ? vq : OOB_VOFF;
    const uint32_t vd = (uint32_t)(lane >> 1) * 2u, vd_last = lane_in ? vd : OOB_VOFF;
    const uint32_t vm = (uint32_t)(lane >> 3) * 16u, vm_last = lane_in ? vm : OOB_VOFF;
    const uint32_t vh = (uint32_t)lane * 8u, vh_last = lane_in ? vh : OOB_VOFF;          // Q6_K high bits
    const uint32_t vs = (uint32_t)lane * 2u, vs_last = lane_in ? vs : OOB_VOFF;          // Q6_K scale pairs, Q4_0 scales
    const uint32_t vd6 = (uint32_t)(lane >> 3) * 2u, vd6_last = lane_in ? vd6 : OOB_VOFF;  // Q6_K super-block scales
    const uint32_t vh5 = (uint32_t)lane * 4u, vh5_last = lane_in ? vh5 : OOB_VOFF;        // Q5_K high bits
    auto load = [&](Raw& W, int k) {                                  // the k-th item of the wave (clamped)
        const bool live = k < nit;                                    // wave-uniform
        const int row = r0 + (first + min(k, nit - 1) * rstep) * R;   // the item's first row
        const int nv = R > 1 ? min(R, r1 - row) * U : 0;              // R > 1: the item's units
        const uint32_t qs = (uint32_t)row * qstride + (uint32_t)u0 * 16u;
        const uint32_t ss = (uint32_t)g.sc_off + (uint32_t)row * sstride;
#pragma unroll
        for (int i = 0; i < CH; ++i) {
            const uint32_t c = (uint32_t)(R > 1 ? i : min(i, lastc));   // wave-uniform
            auto off = [&](uint32_t full, uint32_t last) {
                if constexpr (R > 1) return (!live || 64 * i + lane >= nv) ? OOB_VOFF : full;
                else return (!live || i > lastc) ? OOB_VOFF : (i < lastc ? full : last);
            };
            W.q[i] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(wr, off(vq, vq_last), qs + 1024u * c, 2));
            if constexpr (T == T_Q8_0) W.d[i] = bload2(wr, off(vd, vd_last), ss + (uint32_t)u0 + 64u * c);
            if constexpr (T == T_Q4_0) W.d[i] = bload2(wr, off(vs, vs_last), ss + (uint32_t)u0 * 2u + 128u * c);
            if constexpr (T == T_Q4_K || T == T_Q5_K) W.meta[i] = bload16(wr, off(vm, vm_last), ss + (uint32_t)u0 * 2u + 128u * c);
            if constexpr (T == T_Q5_K)
                W.s[i] = (uint32_t)__builtin_amdgcn_raw_buffer_load_b32(
                    wr, off(vh5, vh5_last), (uint32_t)g.hi_off + (uint32_t)row * (qstride >> 2) + (uint32_t)u0 * 4u + 256u * c, 2);
            if constexpr (T == T_Q6_K) {
                W.h[i] = __builtin_bit_cast(u32x2, __builtin_amdgcn_raw_buffer_load_b64(
                    wr, off(vh, vh_last), (uint32_t)g.hi_off + (uint32_t)row * (qstride >> 1) + (uint32_t)u0 * 8u + 512u * c, 2));
                W.s[i] = bload2(wr, off(vs, vs_last), ss + (uint32_t)u0 * 2u + 128u * c);
                W.d[i] = bload2(wr, off(vd6, vd6_last), (uint32_t)g.d_off + (uint32_t)row * (uint32_t)(K >> 7) + ((uint32_t)u0 >> 2) + 16u * c);
            }
        }
    };

    // x of the lane's units (clamped to the row), per activation row, and for Q4_K the per-unit sums of x. The x loads
    // are issued before the first item's weights: loads complete in order, so the sums of x then wait for x only, with
    // the weights still in flight.
    u32x4 xv[CH][M][TPU];
    float xs[CH][M], xs2[CH][M];                                      // Q6_K: sums of x over each half unit
    int rsel[CH];                                                     // R > 1: the item row of the lane's unit
#pragma unroll
    for (int i = 0; i < CH; ++i) {
        const int u = R > 1 ? (64 * i + lane) % U : min(u0 + lane + 64 * i, U - 1);
        rsel[i] = (64 * i + lane) / U;
#pragma unroll
        for (int m = 0; m < M; ++m)
#pragma unroll
            for (int t = 0; t < TPU; ++t) xv[i][m][t] = bload16(xr, (uint32_t)(((int64_t)m * K + (int64_t)u * UW + t * 8) * 2), 0);
    }
    Raw A, B, C;
    if (any) {
        load(A, 0);
        if constexpr (DEPTH == 3) load(B, 1);
    }
#pragma unroll
    for (int i = 0; i < CH; ++i) {
#pragma unroll
        for (int m = 0; m < M; ++m) {
            float sum = 0.f, sum2 = 0.f;
            if constexpr (unit32(T)) {
#pragma unroll
                for (int t = 0; t < TPU; ++t)
#pragma unroll
                    for (int p = 0; p < 4; ++p) {
                        if (T == T_Q6_K && t >= 2) sum2 = dot2(xv[i][m][t][p], BF16_ONES, sum2);
                        else sum = dot2(xv[i][m][t][p], BF16_ONES, sum);
                    }
            }
            xs[i][m] = sum;
            xs2[i][m] = sum2;
        }
    }
    const Q4kSel sel = q4k_sel((u0 + lane) & 7);                     // units advance by 64: the lane's slot is fixed
    const uint32_t kmask = in_vgpr(0x000F000Fu), kmagic = in_vgpr(0x43004300u);
    const uint32_t c43 = in_vgpr(0x43434343u);

    auto finish = [&](const Raw& W, int k) {
        const int rl = first + k * rstep;                             // R > 1: the item's group
        const int nuk = R > 1 ? min(R, r1 - (r0 + rl * R)) * U : nu;  // units of the item
        float acc[M], accr[R][M];
#pragma unroll
        for (int m = 0; m < M; ++m) {
            acc[m] = 0.f;
#pragma unroll
            for (int r = 0; r < R; ++r) accr[r][m] = 0.f;
        }
        // chunk i; FULL: every lane holds a unit of the part (no zeroed scale)
        auto chunk = [&](auto FULL_, int i) {
            constexpr bool FULL = decltype(FULL_)::value;
            const bool act = FULL || lane + 64 * i < nuk;
            if constexpr (T == T_Q6_K) {
                const float d = f16f(W.d[i]);
                float ds0 = d * (float)(int8_t)(W.s[i] & 0xFFu), ds1 = d * (float)(int8_t)((W.s[i] >> 8) & 0xFFu);   // exact
                if constexpr (!FULL) {
                    ds0 = act ? ds0 : 0.f;
                    ds1 = act ? ds1 : 0.f;
                }
                float A0[M], B0[M], A1[M], B1[M];                         // halves 0 / 1, quant bytes lo / hi
#pragma unroll
                for (int t = 0; t < 4; ++t) {
                    uint32_t lo, hi;
                    q6k_bytes(W.q[i][t], W.h[i][t >> 1], t, &lo, &hi);
#pragma unroll
                    for (int m = 0; m < M; ++m) {
                        float& A = t < 2 ? A0[m] : A1[m];
                        float& B = t < 2 ? B0[m] : B1[m];
                        A = dot2(b128_pair(lo, c43, 0), xv[i][m][t][0], (t & 1) ? A : 0.f);
                        A = dot2(b128_pair(lo, c43, 1), xv[i][m][t][1], A);
                        B = dot2(b128_pair(hi, c43, 0), xv[i][m][t][2], (t & 1) ? B : 0.f);
                        B = dot2(b128_pair(hi, c43, 1), xv[i][m][t][3], B);
                    }
                }
#pragma unroll
                for (int m = 0; m < M; ++m) {
                    acc[m] = __builtin_fmaf(ds0, A0[m] + B0[m], __builtin_fmaf(-160.f * ds0, xs[i][m], acc[m]));
                    acc[m] = __builtin_fmaf(ds1, A1[m] + B1[m], __builtin_fmaf(-160.f * ds1, xs2[i][m], acc[m]));
                }
            } else if constexpr (T == T_Q5_K) {
                uint32_t sc, mn;
                q4k_scale_min_sel(W.meta[i][1], W.meta[i][2], W.meta[i][3], sel, &sc, &mn);
                float dsc = f16f(W.meta[i][0]) * (float)sc;             // exact
                const float dm = f16f(W.meta[i][0] >> 16) * (float)mn;  // exact
                float c = 128.f * dsc + dm;
                if constexpr (!FULL) {
                    dsc = act ? dsc : 0.f;
                    c = act ? c : 0.f;
                }
                float P0[M], P1[M];                                       // quant bytes lo / hi
#pragma unroll
                for (int t = 0; t < 4; ++t) {
                    uint32_t lo, hi;
                    q5k_bytes(W.q[i][t], W.s[i], t, &lo, &hi);
#pragma unroll
                    for (int m = 0; m < M; ++m) {
                        P0[m] = dot2(b128_pair(lo, c43, 0), xv[i][m][t][0], t ? P0[m] : 0.f);
                        P0[m] = dot2(b128_pair(lo, c43, 1), xv[i][m][t][1], P0[m]);
                        P1[m] = dot2(b128_pair(hi, c43, 0), xv[i][m][t][2], t ? P1[m] : 0.f);
                        P1[m] = dot2(b128_pair(hi, c43, 1), xv[i][m][t][3], P1[m]);
                    }
                }
#pragma unroll
                for (int m = 0; m < M; ++m) acc[m] = __builtin_fmaf(dsc, P0[m] + P1[m], __builtin_fmaf(-c, xs[i][m], acc[m]));
            } else if constexpr (nib4(T)) {
                float dsc, c;
                if constexpr (T == T_Q4_0) {
                    dsc = f16f(W.d[i]);
                    c = 136.f * dsc;                                    // (128 + q) d - 136 d = (q - 8) d
                } else {
                    uint32_t sc, mn;
                    q4k_scale_min_sel(W.meta[i][1], W.meta[i][2], W.meta[i][3], sel, &sc, &mn);
                    dsc = f16f(W.meta[i][0]) * (float)sc;               // exact
                    const float dm = f16f(W.meta[i][0] >> 16) * (float)mn;  // exact
                    c = 128.f * dsc + dm;
                }
                if constexpr (!FULL) {
                    dsc = act ? dsc : 0.f;
                    c = act ? c : 0.f;
                }
                float P0[M], P1[M];
#pragma unroll
                for (int t = 0; t < 4; ++t)
#pragma unroll
                    for (int pp = 0; pp < 4; ++pp) {
                        const uint32_t pr = ((W.q[i][t] >> (4 * pp)) & kmask) | kmagic;
#pragma unroll
                        for (int m = 0; m < M; ++m) {
                            float& Pm = (pp & 1) ? P1[m] : P0[m];
                            Pm = dot2(pr, xv[i][m][t][pp], (t == 0 && pp < 2) ? 0.f : Pm);
                        }
                    }
#pragma unroll
                for (int m = 0; m < M; ++m) acc[m] = __builtin_fmaf(dsc, P0[m] + P1[m], __builtin_fmaf(-c, xs[i][m], acc[m]));
            } else {
                float d = 1.f;
                if constexpr (T == T_Q8_0) d = f16f(W.d[i]);
                if constexpr (!FULL) d = act ? d : 0.f;
                float P0[M], P1[M];
#pragma unroll
                for (int t = 0; t < 4; ++t) {
                    uint32_t b0, b1;
                    gv_i8x4(W.q[i][t], &b0, &b1);
#pragma unroll
                    for (int m = 0; m < M; ++m) {
                        float& Pm = (t & 1) ? P1[m] : P0[m];
                        Pm = dot2(b0, xv[i][m][t >> 1][2 * (t & 1)], t < 2 ? 0.f : Pm);
                        Pm = dot2(b1, xv[i][m][t >> 1][2 * (t & 1) + 1], Pm);
                    }
                }
#pragma unroll
                for (int m = 0; m < M; ++m) acc[m] = __builtin_fmaf(d, P0[m] + P1[m], acc[m]);
            }
        };
        using Full = std::integral_constant<bool, true>;
        using Part = std::integral_constant<bool, false>;
#pragma unroll
        for (int i = 0; i < CH; ++i) {
            if (64 * (i + 1) <= nuk) chunk(Full{}, i);                 // wave-uniform
            else if (64 * i < nuk) chunk(Part{}, i);
            if constexpr (R > 1) {                                    // the chunk's sums to the lanes' rows
#pragma unroll
                for (int m = 0; m < M; ++m) {
#pragma unroll
                    for (int r = 0; r < R; ++r) accr[r][m] += rsel[i] == r ? acc[m] : 0.f;
                    acc[m] = 0.f;
                }
            }
        }
        if constexpr (R > 1) {
#pragma unroll
            for (int r = 0; r < R; ++r)
#pragma unroll
                for (int m = 0; m < M; ++m) {
                    const float v = wave_sum_dpp(accr[r][m]);
                    const int n = r0 + rl * R + r;
                    if (lane == 0 && n < r1) store_y(g.y, (int64_t)m * N + n, v * ((T == T_INT8) ? g.srow[n] : 1.f), g.out_bf16);
                }
        } else {
#pragma unroll
            for (int m = 0; m < M; ++m) {
                const float v = wave_sum_dpp(acc[m]);
                if (lane == 0) {
                    if (S == 1) {
                        const int n = r0 + rl;
                        const float sc = (T == T_INT8) ? g.srow[n] : 1.f;
                        store_y(g.y, (int64_t)m * N + n, v * sc, g.out_bf16);
                    } else {
                        parts[(rl * S + part) * M + m] = v;
                    }
                }
            }
        }
    };
    if (any) {
        if constexpr (DEPTH == 3) {
            // while item k computes, items k + 1 and k + 2 load
            for (int k = 0; k < nit; k += 3) {
                load(C, k + 2);
                finish(A, k);
                load(A, k + 3);
                if (k + 1 < nit) finish(B, k + 1);
                load(B, k + 4);
                if (k + 2 < nit) finish(C, k + 2);
            }
        } else {
            // while item k computes, item k + 1 loads
            for (int k = 0; k < nit; k += 2) {
                load(B, k + 1);
                finish(A, k);
                load(A, k + 2);
                if (k + 1 < nit) finish(B, k + 1);
            }
        }
    }
    if (S > 1 || !ok) {
        __syncthreads();
        for (int e = threadIdx.x; e < nrows * M; e += GV_THREADS) {
            const int rl = e / M, m = e - rl * M, n = r0 + rl;
            float v = 0.f;
            if (S > 1)
                for (int p = 0; p < S && p * PU < U; ++p) v += parts[(rl * S + p) * M + m];   // parts past K hold nothing
            const float sc = (T == T_INT8) ? g.srow[n] : 1.f;
            store_y(g.y, (int64_t)m * N + n, ok ? v * sc : __builtin_nanf(""), g.out_bf16);
        }
    }
}

// ------------------------------------------------------------------------------------------------------ launchers
// blocks of a GEMV kernel the current GPU holds at once: its CUs (cached per device) times the kernel's blocks per CU
// (cached per kernel and LDS size)
template <class Kern>
static int resident_blocks(Kern kernel, size_t lds) {
    static thread_local struct { const void* k; size_t lds; int per; } cache[64];
    static thread_local int used = 0;
    for (int i = 0; i < used; ++i)
        if (cache[i].k == (const void*)kernel && cache[i].lds == lds) return cus_of_device() * cache[i].per;
    int per = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per, kernel, GV_THREADS, lds) != hipSuccess || per < 1) return -1;
    if (used < 64) cache[used++] = {(const void*)kernel, lds, per};
    return cus_of_device() * per;
}

// Parts per row: the fewest S in {1, 2, 4, 8} whose parts take at most GV_ITEM_CHUNKS chunks and fit the registers
// (at M = 1: K <= 24576 int8 / Q8_0, 49152 Q4_0 / K-quants); PU rounded to the scale granularity (Q8_0 scales cover
// 2 units, Q4_K meta 8, Q4_0 scales 1). S = 3 instead when it raises the share of busy lanes by 20 points or more: its parts have 3, 3 and 2 waves,
// so it wins only by filling chunks (MI355X, 5120 x 17408 Q4_K: 544 units as 3 parts of 3 chunks, 94 % busy, 13.6 us;
// 4 parts, 71 % busy, 14.5 us; Q8_0 17408 x 5120 keeps S = 2: 17.3 us against 20.8 with S = 3). Returns the chunks
// the parts need, or -1.
template <int T, int M>
static int gv_parts(int64_t U, int* S, int* PU) {
    const int64_t gran = kquant(T) ? 8 : T == T_Q4_0 ? 1 : 2, cap = 64 * std::min(GV_ITEM_CHUNKS, gv_chmax<T>(M));
    auto pu_of = [&](int s) { return ((U + s - 1) / s + gran - 1) / gran * gran; };
    for (int s = 1; s <= GV_WAVES; s *= 2) {
        const int64_t pu = pu_of(s);
        if (pu <= cap) {
            const int64_t ch = (pu + 63) / 64, pu3 = pu_of(3), ch3 = (pu3 + 63) / 64;
            if (s > 3 && pu3 <= cap && 100 * U / (3 * 64 * ch3) >= 100 * U / (s * 64 * ch) + 20) {
                *S = 3;
                *PU = (int)pu3;
                return (int)ch3;
            }
            *S = s;
            *PU = (int)pu;
            return (int)ch;
        }
    }
    return -1;
}

template <int T, int M, int CH, int R = 1>
static int launch_gemv_ch(const Args& a, int S, int PU, hipStream_t s) {
    auto kern = gemv_kernel<T, M, CH, 2, R>;
    const int cus = cus_of_device();
    int P = resident_blocks(kern, 4096);
    if (P < 1) return set_error(MBQ_LAUNCH_FAIL, "GEMV occupancy query failed");
    const int bpc = gv_two_blocks(a.N, S, M, cus) ? 2 : 1;
    P = (int)std::min<int64_t>({(int64_t)P, (int64_t)cus * bpc, a.N});
    const int64_t rows_max = (a.N + P - 1) / P;
    const size_t lds = S > 1 ? (size_t)rows_max * S * M * 4 : 0;
    if (lds > 64 * 1024) return set_error(MBQ_BAD_ARG, "GEMV N = %lld needs too much LDS", (long long)a.N);
    GvArgs g{a.base, a.stride, a.layer_dev, a.nlayers, a.sc_off, a.hi_off, a.d_off, a.wbytes, a.srow, a.x, (int)a.N, (int)a.K, S, PU, a.y, a.out_bf16};
    kern<<<dim3((unsigned)P), GV_THREADS, lds, s>>>(g);
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return set_error(MBQ_LAUNCH_FAIL, "gemv: %s", hipGetErrorString(e));
    return 0;
}

// rows per item at one activation row: 4 when a row is 80 units (2560-value K-quant rows, 1280-value Q8_0 / int8 rows),
// whose second chunk would have 16 of 64 lanes busy: 4 rows are 5 full chunks. Measured on MI355X (151936-row heads):
// Q4_K 11 %, Q5_K 10 %, Q6_K 3 % faster; packing 2 rows of 96 or 160 units was slower (Q6_K K = 3072 by 8 %, Q8_0
// K = 2560 by 3 %), so other rows keep one row per item.
template <int T>
static int gv_pack(int64_t U) {
    return (U == 80 && 4 * U <= 64 * gv_chmax<T>(1)) ? 4 : 1;
}

// The GEMV's plan for a call: rows per item R (4 for 80-unit rows at one activation row, else 1), parts S, units per
// part PU and chunks per item CH; false when the GEMV does not run the shape (operands over the buffer range, a row
// too long for the activation rows' registers, or the parts' sums over the LDS of one block). mbq_matmul then runs the
// weight-stream kernel, which takes any K.
struct GvPlan { int R, S, PU, CH; };
template <int T, int M>
static bool gv_plan(const Args& a, GvPlan* p) {
    if (a.wbytes > BUF_MAX_BYTES || a.M * a.K * 2 > BUF_MAX_BYTES) return false;
    const int64_t U = a.K / gv_uw<T>();
    if (M == 1 && gv_pack<T>(U) > 1) {
        *p = GvPlan{gv_pack<T>(U), 1, (int)(gv_pack<T>(U) * U), 5};         // 4 rows of 80 units: 5 chunks
        return true;
    }
    int S = 1, PU = 0;
    const int ch = gv_parts<T, M>(U, &S, &PU);
    if (ch < 1) return false;
    // the parts' sums of a block's rows in LDS: at most ceil(N / min(CUs, N)) rows per block
    const int64_t blocks = std::min<int64_t>(cus_of_device(), a.N), rows_max = (a.N + blocks - 1) / blocks;
    if (S > 1 && rows_max * S * M * 4 > 64 * 1024) return false;
    *p = GvPlan{1, S, PU, ch};
    return true;
}

template <int T, int M>
static int launch_gemv_m(const Args& a, hipStream_t s) {
    GvPlan p;
    if (!gv_plan<T, M>(a, &p)) return set_error(MBQ_BAD_ARG, "GEMV has no plan for K = %lld at %d activation rows", (long long)a.K, M);
    if (p.R > 1) {
        if constexpr (M == 1) return launch_gemv_ch<T, 1, 5, 4>(a, 1, p.PU, s);
        return set_error(MBQ_BAD_ARG, "GEMV: packed rows at %d activation rows", M);
    }
    constexpr int C = gv_chmax<T>(M);
    switch (p.CH) {
        case 1: return launch_gemv_ch<T, M, 1>(a, p.S, p.PU, s);
        case 2: if constexpr (C >= 2) return launch_gemv_ch<T, M, 2>(a, p.S, p.PU, s); break;
        case 3: if constexpr (C >= 3) return launch_gemv_ch<T, M, 3>(a, p.S, p.PU, s); break;
        case 4: if constexpr (C >= 4) return launch_gemv_ch<T, M, 4>(a, p.S, p.PU, s); break;
        case 5: if constexpr (C >= 5) return launch_gemv_ch<T, M, 5>(a, p.S, p.PU, s); break;
        case 6: if constexpr (C >= 6) return launch_gemv_ch<T, M, 6>(a, p.S, p.PU, s); break;
    }
    return set_error(MBQ_BAD_ARG, "GEMV: no kernel for %d chunks", p.CH);
}

template <int T>
static int launch_gemv_t(const Args& a, hipStream_t s) {
    switch (a.M) {
        case 1: return launch_gemv_m<T, 1>(a, s);
        case 2: return launch_gemv_m<T, 2>(a, s);
        case 3: return launch_gemv_m<T, 3>(a, s);
        case 4: return launch_gemv_m<T, 4>(a, s);
    }
    return set_error(MBQ_BAD_ARG, "GEMV: M = %lld", (long long)a.M);
}

int launch_gemv(int t, const Args& a, hipStream_t s) {
    if (tiled_type(t)) return launch_tgemv(t, a, s);   // one row on 16-row tiles (mbq_tgemv.hip)
    switch (t) {
        case T_Q4_0: return launch_gemv_t<T_Q4_0>(a, s);
        case T_Q8_0: return launch_gemv_t<T_Q8_0>(a, s);
        case T_Q4_K: return launch_gemv_t<T_Q4_K>(a, s);
        case T_Q5_K: return launch_gemv_t<T_Q5_K>(a, s);
        case T_Q6_K: return launch_gemv_t<T_Q6_K>(a, s);
        case T_INT8: return launch_gemv_t<T_INT8>(a, s);
    }
    return set_error(MBQ_BAD_ARG, "no GEMV for type %d", t);
}

template <int T>
static bool gemv_runs_t(const Args& a) {
    GvPlan p;
    switch (a.M) {
        case 1: return gv_plan<T, 1>(a, &p);
        case 2: return gv_plan<T, 2>(a, &p);
        case 3: return gv_plan<T, 3>(a, &p);
        case 4: return gv_plan<T, 4>(a, &p);
    }
    return false;
}

bool gemv_runs(int t, const Args& a) {
    if (tiled_type(t)) return tgemv_runs(t, a);
    switch (t) {
        case T_Q4_0: return gemv_runs_t<T_Q4_0>(a);
        case T_Q8_0: return gemv_runs_t<T_Q8_0>(a);
        case T_Q4_K: return gemv_runs_t<T_Q4_K>(a);
        case T_Q5_K: return gemv_runs_t<T_Q5_K>(a);
        case T_Q6_K: return gemv_runs_t<T_Q6_K>(a);
        case T_INT8: return gemv_runs_t<T_INT8>(a);
    }
    return false;
}

}  // namespace mbq
