// gfx950 weight-direct GEMM of the quantized linear for large activation batches (chunked prefill): big output tiles,
// weights from HBM straight into MFMA operands, activations shared through LDS.
//
// y (M, N) = x (M, K) @ W.T with W dequantized on the fly: reference src/mashbox/ops/__init__.py:594-632 (qmatmul,
// float32 accumulation) on the weights of reference src/mashbox/ops/reference.py:66-70 (Q4_0), :101-103 (Q8_0),
// :132-149 (Q4_K), :150-159 (Q5_K) and :164-173 (Q6_K), and reference src/mashbox/models/qwen3_8_27b/model.py:72-82 (int8 per output channel: dot, then * s).
//
// Block = 4 waves, one per SIMD (one block per CU: the float32 accumulators of a 16 MT x 16 NT wave tile live in the
// accumulation registers). The block's tile is 16 MT activation rows x 64 NT weight rows; wave w owns weight rows
// 16 NT w .. 16 NT w + 16 NT - 1 of it and all 16 MT activation rows. Per iteration (mbq_wdirect.h: KI values of K)
//   - each wave loads its NT x 16 weight rows' bytes for the iteration straight from HBM into registers (no LDS) and
//     dequantizes them once into the B operands of v_mfma_f32_16x16x32_bf16, each B operand then feeding MT MFMAs;
//   - the block's x tile (16 MT rows x KI) arrives in LDS by DMA, read by all 4 waves as A operands, each A operand
//     feeding NT MFMAs.
// So per MFMA a wave spends about 26 / MT VALU instructions on dequantization and 1 KiB / NT of LDS reads: with
// MT = 16 and NT >= 3 neither the VALU nor the LDS keeps up with less than the matrix cores.
//
// Pipeline: a ring of D LDS stages of x (D - 1 iterations in flight; D = 2 for the 64 KiB stages of 256 rows of Q4_0 and the
// K-quants, else 4) and a ring of DW = 4 register buffers of weights (DW iterations in flight). Step l:
// wait for x stage l % D (an exact vmcnt: the loads issued after its DMA), one barrier (the stage has landed for every
// wave; stage (l - 1) % D is no longer read), DMA x of iteration l + D - 1 into stage (l - 1) % D, dequantize and
// multiply, then load the weights of iteration l + DW into the buffer just used. The weights of iteration l were loaded
// before the x of iteration l (DW >= D), so the same vmcnt covers them (loads complete in order).
//
// x stage layout: 16 MT rows of KI bfloat16 in 16-byte chunks, chunk c of row r at slot c ^ (r & (CH - 1)) (the A
// operand reads of 16 rows hit distinct banks; the DMA applies the swizzle through each lane's source address). M is at
// least the tile's 16 MT rows, and the last activation tile ends at row M - 1 (it overlaps the tile before, whose rows
// it computes again but does not store), so every x row a block reads exists: a DMA instruction's rows differ from the
// first instruction's by a scalar offset. Chunks past K read zero through the buffer range check; weight rows past N
// are clamped to row N - 1 (their outputs are never stored); loads past the last iteration are clamped to it (they fill
// buffers nobody reads). The loop runs whole rounds of 4 iterations; the iterations past the last one (K not a multiple
// of 4 KI) read x as zero and add nothing.
//
// Tiles are dealt to blocks XCD by XCD (block b runs on XCD b % 8, which takes a contiguous range of tiles, activation
// tiles fastest), so the blocks running at once on one XCD share weight panels and x panels in its L2.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <algorithm>
#include <type_traits>

#include "mbq_device.h"
#include "mbq_launch.h"
#include "mbq_layout.h"
#include "mbq_wdirect.h"

namespace mbq {

constexpr int PG_THREADS = 256;    // 4 waves
// x stages in LDS: 2 for the 64 KiB stages of 256 rows x 128 values (Q4_0, K-quants), else 4 (at most 128 KiB); Q6_K, with 4 weight
// loads per row tile, always 2 (the loads in flight stay within the 63 that vmcnt counts)
template <int T, int MT> constexpr int pg_stages() { return (T == T_Q6_K || (unit32(T) && MT > 8)) ? 2 : 4; }
// weight iterations in flight per wave
template <int T, int MT, int NT> constexpr int pg_wdepth() { return 4; }
template <int T, int MT> constexpr size_t pg_lds_bytes() { return (size_t)pg_stages<T, MT>() * 16 * MT * ws_ki<T>() * 2; }

struct PgArgs {
    const uint8_t* base;        // planes of the weight (host layer applied)
    int64_t stride;             // bytes between stacked weights (layer_dev)
    const int32_t* layer_dev;   // device layer index, or nullptr
    int nlayers;
    int64_t sc_off, wbytes;     // scale plane offset and bytes of one weight's planes (int8: N x K)
    int64_t hi_off, d_off;      // Q6_K high-bit and super-block scale planes
    const float* srow;          // int8: per-row scales
    const uint16_t* x;
    int M, N, K;
    void* y;
    int out_bf16;
    int mtiles, tiles;          // activation tiles, all tiles
};

template <int T, int MT, int NT, bool KFULL>
__global__ __launch_bounds__(PG_THREADS, 1) void pgemm_kernel(const PgArgs g) {
    extern __shared__ __attribute__((aligned(16))) uint16_t pg_x[];   // D stages of 16 MT x KI bfloat16
    constexpr int KI = ws_ki<T>(), KS = KI / 32, CH = KI / 8, D = pg_stages<T, MT>(), DW = pg_wdepth<T, MT, NT>();
    constexpr int ROWS = 16 * MT, STAGE = ROWS * KI;                // bfloat16 per stage
    constexpr int NDW = ROWS * CH / 256;                            // DMA instructions per wave per stage
    constexpr int RPI = 64 / CH;                                    // x rows per DMA instruction
    constexpr int NWL = NT * ws_wloads<T>();                        // weight loads per wave per iteration
    static_assert(ROWS * CH % 256 == 0 && DW >= D && 4 % DW == 0 && 4 % D == 0, "stage and buffer rings");
    const int M = g.M, N = g.N, K = g.K;

    const int b = blockIdx.x, xcd = b & 7, q = g.tiles >> 3, rem = g.tiles & 7;
    const int tile = xcd * q + min(xcd, rem) + (b >> 3);
    const int mt = tile % g.mtiles, nt = tile / g.mtiles;
    const int mfirst = mt * ROWS, m0 = min(mfirst, M - ROWS);       // rows m0 .. m0 + ROWS - 1 exist; store from mfirst
    const int lane = threadIdx.x & 63, lg = lane >> 4, r16 = lane & 15;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int n0 = nt * 64 * NT + wave * 16 * NT;                   // this wave's first weight row
    const int64_t lo = layer_offset(g.stride, g.layer_dev, g.nlayers);
    const bool ok = lo >= 0;
    const rsrc_t wr = make_rsrc(g.base + (ok ? lo : 0), (uint32_t)g.wbytes);
    const rsrc_t xr = make_rsrc(g.x + (int64_t)m0 * K, (uint32_t)((int64_t)ROWS * K * 2));

    const int KT = (K + KI - 1) / KI;
    const int n = ok ? KT : 0;
    auto k0 = [&](int l) { return min(l, n - 1) * KI; };            // K offset of iteration l (clamped)

    WsOff wo[NT];
#pragma unroll
    for (int j = 0; j < NT; ++j) wo[j] = ws_off<T>((uint32_t)min(n0 + 16 * j + r16, N - 1), K, lg, g.sc_off, g.hi_off, g.d_off);
    // x DMA: instruction i of wave w fills rows RPI (w + 4 i) ..; lane l writes slot l % CH of row l / CH, which holds
    // chunk (l % CH) ^ (row & (CH - 1)) (4 RPI is a multiple of CH, so the chunk is the same for every instruction)
    const int xr0 = RPI * wave + lane / CH, xc = (lane % CH) ^ (xr0 & (CH - 1));
    const uint32_t xv = (uint32_t)((xr0 * K + xc * 8) * 2);
    // x of iteration `it` into stage st; iterations past the last one read zero (the loop runs whole rounds of 4)
    auto dma_x = [&](int st, int it) {
        const int kk = k0(it);
        uint32_t v = it < n ? xv : OOB_VOFF;
        if constexpr (!KFULL) v = (kk + 8 * xc < K) ? v : OOB_VOFF;        // past K: out of range, reads zero
#pragma unroll
        for (int i = 0; i < NDW; ++i)
            ws_dma16(xr, pg_x + st * STAGE + RPI * (wave + 4 * i) * KI, v, (uint32_t)(kk * 2 + i * 4 * RPI * K * 2));
    };
    auto load_w = [&](WsRaw<T>* W, int kk) {
#pragma unroll
        for (int j = 0; j < NT; ++j) ws_load<T, KFULL>(W[j], wr, wo[j], kk, K, lg);
    };
    // A operand of K step s, row tile i: chunk lg KS + s (8 bfloat16) of x row 16 i + (lane & 15) of stage st, where
    // (16 i + r16) & (CH - 1) = r16 & (CH - 1)
    auto a_op = [&](int st, int s, int i) {
        return *reinterpret_cast<const bf16x8_t*>(pg_x + st * STAGE + (16 * i + r16) * KI + (((lg * KS + s) ^ (r16 & (CH - 1))) << 3));
    };

    f32x4_t acc[MT][NT];
#pragma unroll
    for (int i = 0; i < MT; ++i)
#pragma unroll
        for (int j = 0; j < NT; ++j) acc[i][j] = f32x4_t{0.f, 0.f, 0.f, 0.f};

    WsRaw<T> W[DW][NT];
    // the DMA of iteration l has landed once at most the loads issued after it are in flight: the weight loads of its
    // own step and both groups of the D - 2 steps after
    constexpr int XWAIT = NWL + (D - 2) * (NDW + NWL);

    // Schedule of a K step (fixed by scheduling fences): MT x NT MFMA slots; before the NT MFMAs of row tile i the A
    // operand PF reads ahead is read from LDS (a ring of AR registers); after every MFMA, a slice of VALU work: the B
    // dwords of the next K step of this iteration, or, in the last K step, the scales and the K step 0 B dwords of the
    // next iteration. So the VALU work runs while the matrix cores are busy, and the LDS latency is hidden behind PF
    // row tiles of MFMAs.
    constexpr int PF = 3, AR = 4, SLOTS = MT * NT, PAIRS = 4 * NT;
    static_assert(SLOTS - NT >= PAIRS, "a K step has a slot for every B dword of the next one");
    WsScale sc[NT];          // scales of the current iteration
    u32x4 Bc[NT];            // B dwords of the current K step
    bf16x8_t Ar[AR];
    auto fence = [] { __builtin_amdgcn_sched_barrier(0); };
    // slot (0 .. SLOTS-1) that computes B dword q (0 .. PAIRS-1), spread evenly over the first n slots after `first`
    auto pair_slot = [](int q, int first, int n) { return first + q * n / PAIRS; };

    auto step = [&](auto U_, int l) {
        constexpr int U = decltype(U_)::value;                       // l % 4
        constexpr int ST = U % D, WB = U % DW, WN = (U + 1) % DW;    // x stage, weight buffers of l and l + 1
        wait_vm<XWAIT>();
        barrier_nofence();
        fence();
        dma_x((ST + D - 1) % D, l + D - 1);
        fence();
#pragma unroll
        for (int p = 0; p < PF; ++p) Ar[p] = a_op(ST, 0, p);
        fence();
        const int j0n = ((k0(l + 1) >> 5) & 7) + lg;                 // Q4_K: sub-block of the lane group, next iteration
        WsScale scn[NT];
#pragma unroll
        for (int s = 0; s < KS; ++s) {
            u32x4 Bn[NT];
            const bool last = s + 1 == KS;
#pragma unroll
            for (int i = 0; i < MT; ++i) {
                const int na = s * MT + i + PF;                      // A read ahead (this iteration only)
                if (na < KS * MT) Ar[na % AR] = a_op(ST, na / MT, na % MT);
#pragma unroll
                for (int j = 0; j < NT; ++j) {
                    mfma_acc(acc[i][j], Ar[(s * MT + i) % AR], __builtin_bit_cast(bf16x8_t, Bc[j]));
                    const int k = i * NT + j;
                    if (!last) {
#pragma unroll
                        for (int q = 0; q < PAIRS; ++q)
                            if (pair_slot(q, 0, SLOTS) == k) Bn[q / 4][q % 4] = ws_bpair<T>(W[WB][q / 4], sc[q / 4], s + 1, q % 4);
                    } else {
                        if (k < NT) scn[k] = ws_scale<T>(W[WN][k], j0n);
#pragma unroll
                        for (int q = 0; q < PAIRS; ++q)
                            if (pair_slot(q, NT, SLOTS - NT) == k) Bn[q / 4][q % 4] = ws_bpair<T>(W[WN][q / 4], scn[q / 4], 0, q % 4);
                    }
                    fence();
                }
            }
#pragma unroll
            for (int j = 0; j < NT; ++j) Bc[j] = Bn[j];
        }
#pragma unroll
        for (int j = 0; j < NT; ++j) sc[j] = scn[j];
        load_w(W[WB], k0(l + DW));
        fence();
    };

    using I0 = std::integral_constant<int, 0>;
    using I1 = std::integral_constant<int, 1>;
    using I2 = std::integral_constant<int, 2>;
    using I3 = std::integral_constant<int, 3>;
    if (n > 0) {                                                      // block-uniform
        // prologue: x of iterations 0 .. D-2 into stages 0 .. D-2, weights of iterations 0 .. DW-1
#pragma unroll
        for (int p = 0; p < DW; ++p) {
            if (p < D - 1) dma_x(p, p);
            load_w(W[p], k0(p));
        }
        const int j00 = ((k0(0) >> 5) & 7) + lg;
#pragma unroll
        for (int j = 0; j < NT; ++j) {
            sc[j] = ws_scale<T>(W[0][j], j00);
            Bc[j] = __builtin_bit_cast(u32x4, ws_bop<T>(W[0][j], sc[j], 0));
        }
        // whole rounds of 4 iterations, the last padded with iterations whose x is zero: no conditional steps, whose
        // block boundaries would make the compiler move accumulators between registers right after the asm MFMAs
        for (int l = 0; l < n; l += 4) {
            step(I0{}, l);
            step(I1{}, l + 1);
            step(I2{}, l + 2);
            step(I3{}, l + 3);
            mfma_drain();                                             // before any accumulator copy at the back edge or exit
        }
        wait_vm<0>();                                                 // no DMA may land after the block ends
    }

    // epilogue: lane holds weight row n0 + 16 j + (lane & 15) and activation rows m0 + 16 i + 4 (lane >> 4) + r; the rows
    // before mfirst belong to the tile before
#pragma unroll
    for (int j = 0; j < NT; ++j) {
        const int nn = n0 + 16 * j + r16;
        if (nn >= N) continue;
        const float s = (T == T_INT8) ? g.srow[nn] : 1.f;
#pragma unroll
        for (int i = 0; i < MT; ++i)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int m = m0 + 16 * i + 4 * lg + r;
                if (m >= mfirst) store_y(g.y, (int64_t)m * N + nn, ok ? acc[i][j][r] * s : __builtin_nanf(""), g.out_bf16);
            }
    }
}

// ------------------------------------------------------------------------------------------------------ launchers
template <int T, int MT, int NT, bool KFULL>
static int pg_launch(const Args& a, hipStream_t s) {
    auto kern = pgemm_kernel<T, MT, NT, KFULL>;
    const size_t lds = pg_lds_bytes<T, MT>();
    static std::atomic<uint64_t> lds_set{0};
    if (set_lds_limit((const void*)kern, lds, lds_set) != hipSuccess)
        return set_error(MBQ_LAUNCH_FAIL, "weight-direct GEMM: %zu bytes of LDS refused", lds);
    const int64_t mtiles = (a.M + 16 * MT - 1) / (16 * MT), ntiles = (a.N + 64 * NT - 1) / (64 * NT);
    PgArgs g{a.base, a.stride, a.layer_dev, a.nlayers, a.sc_off, a.wbytes, a.hi_off, a.d_off, a.srow, a.x, (int)a.M, (int)a.N, (int)a.K,
             a.y, a.out_bf16, (int)mtiles, (int)(mtiles * ntiles)};
    kern<<<dim3((unsigned)(mtiles * ntiles)), PG_THREADS, lds, s>>>(g);
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return set_error(MBQ_LAUNCH_FAIL, "weight-direct GEMM launch: %s", hipGetErrorString(e));
    return 0;
}

template <int T, int MT, int NT>
static int pg_launch_k(const Args& a, hipStream_t s) {
    if constexpr (kquant(T)) return pg_launch<T, MT, NT, true>(a, s);   // rows of whole 256-value blocks
    else return a.K % ws_ki<T>() == 0 ? pg_launch<T, MT, NT, true>(a, s) : pg_launch<T, MT, NT, false>(a, s);
}

// tile shapes: activation row tiles MT x weight row tiles NT per wave
struct PgShape { int mt, nt; };
static constexpr PgShape PG_SHAPES[] = {{16, 4}, {16, 3}, {16, 2}, {8, 5}, {8, 4}, {8, 2}};
constexpr int PG_NSHAPES = (int)(sizeof PG_SHAPES / sizeof PG_SHAPES[0]);

template <int T>
static int pg_dispatch(const Args& a, int idx, hipStream_t s) {
    switch (idx) {
        case 0: if constexpr (T != T_Q5_K && T != T_Q6_K) return pg_launch_k<T, 16, 4>(a, s); break;
        case 1: return pg_launch_k<T, 16, 3>(a, s);
        case 2: return pg_launch_k<T, 16, 2>(a, s);
        case 3: if constexpr (T != T_Q5_K && T != T_Q6_K) return pg_launch_k<T, 8, 5>(a, s); break;
        case 4: return pg_launch_k<T, 8, 4>(a, s);
        case 5: return pg_launch_k<T, 8, 2>(a, s);
    }
    return set_error(MBQ_BAD_ARG, "weight-direct GEMM: no tile shape %d for ggml type %d", idx, T);
}

static int pg_cus() {
    static int cache[64] = {0};
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
    if (cache[dev] == 0) {
        int n = 0;
        if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) n = 256;
        cache[dev] = n;
    }
    return cache[dev];
}

// Modelled time of a tile shape: rounds of one block per CU, each tile 16 MT x 64 NT outputs over K, at a matrix rate
// that drops as the dequantization (per MFMA: ~ 1 / MT) and the LDS reads (~ 1 / NT) take a larger share of a wave's
// issue slots.
static double pg_model(int64_t M, int64_t N, int64_t K, int cus, const PgShape& sh) {
    const int64_t tiles = ((M + 16 * sh.mt - 1) / (16 * sh.mt)) * ((N + 64 * sh.nt - 1) / (64 * sh.nt));
    const int64_t rounds = (tiles + cus - 1) / cus;
    const double eff = 1.0 / (1.0 + 2.0 / sh.mt + 0.25 / sh.nt);
    return (double)rounds * sh.mt * sh.nt * (double)K / eff;
}

// the weight buffers of Q5_K and Q6_K (3 and 4 loads per row tile) leave no registers for the 16 x 4 and 8 x 5 tiles
static bool pg_type_has(int t, int i) { return (t != T_Q5_K && t != T_Q6_K) || (i != 0 && i != 3); }

static int pg_best(int t, int64_t M, int64_t N, int64_t K) {
    const int cus = pg_cus();
    int best = (t == T_Q5_K || t == T_Q6_K) ? 1 : 0;
    double bt = 1e300;
    for (int i = 0; i < PG_NSHAPES; ++i) {
        if (16 * PG_SHAPES[i].mt > M || !pg_type_has(t, i)) continue;
        const double t = pg_model(M, N, K, cus, PG_SHAPES[i]);
        if (t < bt) bt = t, best = i;
    }
    return best;
}

int pgemm_shape(int t, int64_t M, int64_t N, int64_t K, int* mt, int* nt) {
    const int i = pg_best(t, M, N, K);
    *mt = PG_SHAPES[i].mt;
    *nt = PG_SHAPES[i].nt;
    return 0;
}

static int pg_index(int mt, int nt) {
    for (int i = 0; i < PG_NSHAPES; ++i)
        if (PG_SHAPES[i].mt == mt && PG_SHAPES[i].nt == nt) return i;
    return -1;
}

bool pgemm_shape_known(int mt, int nt) { return pg_index(mt, nt) >= 0; }

int launch_pgemm(int t, const Args& a, int mt, int nt, hipStream_t s) {
    const int idx = pg_index(mt, nt);
    if (idx < 0) return set_error(MBQ_BAD_ARG, "weight-direct GEMM: no tile of %d x %d activation x weight row tiles", mt, nt);
    if (a.wbytes > BUF_MAX_BYTES || a.M * a.K * 2 > BUF_MAX_BYTES)
        return set_error(MBQ_BAD_ARG, "weight-direct GEMM operands over 2 GiB");
    if (a.M < 16 * mt) return set_error(MBQ_BAD_ARG, "weight-direct GEMM: %lld activation rows, fewer than a tile's %d", (long long)a.M, 16 * mt);
    switch (t) {
        case T_INT8: return pg_dispatch<T_INT8>(a, idx, s);
        case T_Q4_0: return pg_dispatch<T_Q4_0>(a, idx, s);
        case T_Q8_0: return pg_dispatch<T_Q8_0>(a, idx, s);
        case T_Q4_K: return pg_dispatch<T_Q4_K>(a, idx, s);
        case T_Q5_K: return pg_dispatch<T_Q5_K>(a, idx, s);
        case T_Q6_K: return pg_dispatch<T_Q6_K>(a, idx, s);
    }
    return set_error(MBQ_BAD_ARG, "weight-direct GEMM: no kernel for type %d", t);
}

}  // namespace mbq
