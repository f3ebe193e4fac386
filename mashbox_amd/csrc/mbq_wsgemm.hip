// gfx950 weight-stream GEMM of the quantized linear for small activation batches (M <= WS_MAX_M): the batched-decode
// regime, and decode batches whose rows are too long for the GEMV's registers.
//
// y (M, N) = x (M, K) @ W.T with W dequantized on the fly: reference src/mashbox/ops/__init__.py:594-632 (qmatmul,
// float32 accumulation) on the weights of reference src/mashbox/ops/reference.py:101-103 (Q8_0), :132-149 (Q4_K) and
// :164-173 (Q6_K),
// and reference src/mashbox/models/qwen3_8_27b/model.py:72-82 (int8 per output channel: dot, then * s).
//
// With at most 64 activation rows the weight stream bounds the time, so every weight byte goes from HBM (non-temporal
// loads) straight into the registers that feed v_mfma_f32_16x16x32_bf16 as its B operand, with no LDS round trip. The
// activations are shared: a block's 4 waves own different weight rows (16 NT each) and walk the same K iterations,
// and x for an iteration is copied once into LDS by DMA and read by all 4 waves as A operands.
//
// Latency. An iteration's work is short next to HBM latency, so each wave keeps the weights of D iterations in flight
// and the block keeps x of D - 1 iterations in flight, in a ring of D LDS stages. Step l: wait for stage l % D (an
// exact vmcnt: the loads issued after that DMA), one barrier (stage l % D has landed for every thread; stage
// (l - 1) % D is no longer read), DMA x of iteration l + D - 1 into stage (l - 1) % D, convert and multiply, then load
// the weights of iteration l + D into the buffer just used.
//
// Iterations, lane layout and the B operand of each type: mbq_wdirect.h.
// x stage layout: ROWS rows of KI bfloat16 in 16-byte chunks, chunk c of row r at slot c ^ (r & (CH - 1)), so that
// the A-operand reads (16 rows, one chunk each per lane group) hit distinct banks; the DMA applies the swizzle through
// each lane's source address. x rows past M and chunks past K read zero through the buffer range check. Weight rows
// past N are clamped to row N - 1 (their outputs are never stored); loads past the block's last iteration are clamped
// to it (they fill buffers nobody reads).
//
// K split (S > 1): the blocks of a tile each run a contiguous range of iterations and store their float32 partial
// tile; the block that arrives last, by an atomic counter per tile that it resets, reads the S partials and adds them
// in split order, so the result does not depend on which block finishes last. The partials live in uncached device
// memory (no XCD's L2 holds them, so no cache write-back or invalidation is needed), or, for mbq_matmul_noalloc, in
// the static scratch array, where the exchange releases and acquires at agent scope (split_release / split_acquire).
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <algorithm>
#include <type_traits>

#include "mbq_device.h"
#include "mbq_launch.h"
#include "mbq_layout.h"
#include "mbq_wdirect.h"

namespace mbq {

constexpr int WS_THREADS = 256;    // 4 waves

// iterations in flight (= LDS stages of x): x stages of 8 KB (int8, Q8_0) or 16 KB (Q4_0, K-quants) at 64 activation
// rows. 4 for every type: int8 and Q8_0 ran 1-8 % faster with 4 than with 8 on MI355X at 8-64 rows over 1024-17408-row
// weights (twice the blocks fit a CU's LDS), except 5120 x 17408 int8 at 8 rows (+4 %)
template <int T> constexpr int ws_depth() { return 4; }
// x rows staged: 16 MT, rounded so that every wave issues the same number of 1 KiB DMA instructions per stage
template <int T, int MT> constexpr int ws_rows() { return unit32(T) ? 16 * MT : (MT <= 2 ? 32 : 64); }

struct WsArgs {
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
    int S, kts;                 // K splits and iterations per split
    float* ws;                  // S > 1: partial tiles, one block's outputs per (tile, split)
    int* cnt;                   // S > 1: per-tile arrival counters (zero between launches)
    uint32_t ws_bytes;          // S > 1: bytes of ws
    int fenced;                 // S > 1: ws is cached memory: release / acquire around the exchange
};

template <int T, int MT, int NT, bool KFULL>
__global__ __launch_bounds__(WS_THREADS, 2) void wsgemm_kernel(const WsArgs g) {
    extern __shared__ __attribute__((aligned(16))) uint16_t ws_x[];   // D stages of ROWS x KI bfloat16
    __shared__ int ws_flag;
    constexpr int KI = ws_ki<T>(), KS = KI / 32, CH = KI / 8, D = ws_depth<T>();
    constexpr int ROWS = ws_rows<T, MT>(), STAGE = ROWS * KI;     // bfloat16 per stage
    constexpr int NDW = ROWS * CH / 64 / 4;                         // DMA instructions per wave per stage
    constexpr int RPI = 64 / CH;                                    // x rows per DMA instruction
    constexpr int NWL = NT * ws_wloads<T>();                        // weight loads per wave per iteration
    constexpr int E = MT * NT * 1024;                               // outputs of the block (4 waves), padded
    static_assert(NDW >= 1 && ROWS * CH % 256 == 0, "every wave issues whole DMA instructions");
    const int M = g.M, N = g.N, K = g.K;
    const int tile = blockIdx.x / g.S, kz = blockIdx.x - tile * g.S;
    const int lane = threadIdx.x & 63, lg = lane >> 4, r16 = lane & 15;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int n0 = tile * 64 * NT + wave * 16 * NT;                 // this wave's first weight row
    const int64_t lo = layer_offset(g.stride, g.layer_dev, g.nlayers);
    const bool ok = lo >= 0;
    const rsrc_t wr = make_rsrc(g.base + (ok ? lo : 0), (uint32_t)g.wbytes);
    const rsrc_t xr = make_rsrc(g.x, (uint32_t)((int64_t)M * K * 2));

    const int KT = (K + KI - 1) / KI;
    const int kb = kz * g.kts, n = ok ? min(KT, kb + g.kts) - kb : 0;    // iterations kb .. kb + n - 1
    auto k0 = [&](int l) { return (kb + min(l, n - 1)) * KI; };          // K offset of local iteration l (clamped)

    // weight offsets: row (clamped) x row bytes + the lane group's 16 bytes
    WsOff wo[NT];
#pragma unroll
    for (int j = 0; j < NT; ++j) wo[j] = ws_off<T>((uint32_t)min(n0 + 16 * j + r16, N - 1), K, lg, g.sc_off, g.hi_off, g.d_off);
    // x DMA: instruction i of wave w fills rows RPI (w + 4 i) ..; lane l writes slot l % CH of row l / CH, which holds
    // chunk (l % CH) ^ (row & (CH - 1)); rows past M are out of the buffer's range and read zero
    uint32_t xvo[NDW];
    int xk[NDW];
#pragma unroll
    for (int i = 0; i < NDW; ++i) {
        const int r = RPI * (wave + 4 * i) + lane / CH, c = (lane % CH) ^ (r & (CH - 1));
        xvo[i] = r < M ? (uint32_t)(((int64_t)r * K + c * 8) * 2) : OOB_VOFF;
        xk[i] = c * 8;
    }
    auto dma_x = [&](int st, int kk) {
#pragma unroll
        for (int i = 0; i < NDW; ++i) {
            uint32_t v = xvo[i];
            if constexpr (!KFULL) v = (kk + xk[i] < K) ? v : OOB_VOFF;      // past K: out of range, reads zero
            dma16(xr, ws_x + st * STAGE + RPI * (wave + 4 * i) * KI, v, (uint32_t)kk * 2u);
        }
    };
    auto load_w = [&](WsRaw<T>* W, int kk) {
#pragma unroll
        for (int j = 0; j < NT; ++j) ws_load<T, KFULL>(W[j], wr, wo[j], kk, K, lg);
    };
    // A operand: chunk c (8 bfloat16) of x row 16 i + (lane & 15) from stage st
    auto a_op = [&](int st, int i, int c) {
        const int r = 16 * i + r16;
        return *reinterpret_cast<const bf16x8_t*>(ws_x + st * STAGE + r * KI + ((c ^ (r & (CH - 1))) << 3));
    };

    f32x4_t acc[MT][NT];
#pragma unroll
    for (int i = 0; i < MT; ++i)
#pragma unroll
        for (int j = 0; j < NT; ++j) acc[i][j] = f32x4_t{0.f, 0.f, 0.f, 0.f};

    WsRaw<T> W[D][NT];
    // The DMA of iteration l has landed once at most the loads issued after it are in flight: the weight loads of
    // its own step and both groups of the D - 2 steps after. J < 0: a step of the unrolled loop. J >= 0: step J of the
    // last n % D, whose x and weights would be for iterations past n, so it issues no DMA and no loads (loads nobody
    // reads are dropped by the compiler, and the wait must count what is issued): only the loop steps before it count.
    auto step = [&](auto U_, auto J_, int l) {
        constexpr int U = decltype(U_)::value;                       // l % D
        constexpr int J = decltype(J_)::value;
        wait_vm<NWL + (D - 2 - (J < 0 ? 0 : J)) * (NDW + NWL)>();
        barrier_nofence();
        __builtin_amdgcn_sched_barrier(0);
        if constexpr (J < 0) dma_x((U + D - 1) % D, k0(l + D - 1));
        __builtin_amdgcn_sched_barrier(0);
        // the step's A operands are all read first, the weights converted while the reads are in flight, then the
        // MFMAs run: one LDS latency per step instead of one per MFMA
        bf16x8_t A[MT][KS], B[NT][KS];
#pragma unroll
        for (int i = 0; i < MT; ++i)
#pragma unroll
            for (int s = 0; s < KS; ++s) A[i][s] = a_op(U, i, lg * KS + s);
        __builtin_amdgcn_sched_barrier(0);
        const int j0 = ((k0(l) >> 5) & 7) + lg;                      // Q4_K: sub-block of the lane group
#pragma unroll
        for (int j = 0; j < NT; ++j) {
            const WsScale sc = ws_scale<T>(W[U][j], j0);
#pragma unroll
            for (int s = 0; s < KS; ++s) B[j][s] = ws_bop<T>(W[U][j], sc, s);
        }
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int s = 0; s < KS; ++s)
#pragma unroll
            for (int j = 0; j < NT; ++j)
#pragma unroll
                for (int i = 0; i < MT; ++i)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(A[i][s], B[j][s], acc[i][j], 0, 0, 0);
        __builtin_amdgcn_sched_barrier(0);
        if constexpr (J < 0) load_w(W[U], k0(l + D));
    };

    using I0 = std::integral_constant<int, 0>;
    using I1 = std::integral_constant<int, 1>;
    using I2 = std::integral_constant<int, 2>;
    using I3 = std::integral_constant<int, 3>;
    using I4 = std::integral_constant<int, 4>;
    using I5 = std::integral_constant<int, 5>;
    using I6 = std::integral_constant<int, 6>;
    using I7 = std::integral_constant<int, 7>;
    if (n > 0) {                                                      // block-uniform
        // prologue: x of iterations 0 .. D-2 into stages 0 .. D-2, weights of iterations 0 .. D-1. The empty asm keeps
        // the compiler from merging loads of two iterations at one address (a K-quant's scale block is shared by the
        // iterations of a 256-value superblock), which would leave fewer loads in flight than the waits count.
#pragma unroll
        for (int p = 0; p < D; ++p) {
            if (p < D - 1) dma_x(p, k0(p));
            load_w(W[p], k0(p));
            asm volatile("" ::: "memory");
        }
        using LOOP = std::integral_constant<int, -1>;
        int l = 0;
        for (; l + D <= n; l += D) {
            step(I0{}, LOOP{}, l);
            step(I1{}, LOOP{}, l + 1);
            step(I2{}, LOOP{}, l + 2);
            step(I3{}, LOOP{}, l + 3);
            if constexpr (D == 8) {
                step(I4{}, LOOP{}, l + 4);
                step(I5{}, LOOP{}, l + 5);
                step(I6{}, LOOP{}, l + 6);
                step(I7{}, LOOP{}, l + 7);
            }
        }
        if (l < n) step(I0{}, I0{}, l);
        if (l + 1 < n) step(I1{}, I1{}, l + 1);
        if (l + 2 < n) step(I2{}, I2{}, l + 2);
        if constexpr (D == 8) {
            if (l + 3 < n) step(I3{}, I3{}, l + 3);
            if (l + 4 < n) step(I4{}, I4{}, l + 4);
            if (l + 5 < n) step(I5{}, I5{}, l + 5);
            if (l + 6 < n) step(I6{}, I6{}, l + 6);
        }
        wait_vm<0>();                                                 // no DMA may land after the block ends
    }

    // epilogue: lane holds weight row n0 + 16 j + (lane & 15) and activation rows 16 i + 4 (lane >> 4) + r
    if (g.S > 1) {
        // 16-byte element ((w MT + i) NT + j) 64 + lane of the block's partial tile, in the lanes' own layout, stored and
        // read with sc1 (device-coherent) buffer accesses, which the compiler batches
        const rsrc_t pr = make_rsrc(g.ws, g.ws_bytes);
        const uint32_t mine = (uint32_t)((tile * g.S + kz) * E) * 4u, part = (uint32_t)E * 4u;
        const uint32_t lofs = (uint32_t)((wave * MT * NT) * 64 + lane) * 16u;
#pragma unroll
        for (int i = 0; i < MT; ++i)
#pragma unroll
            for (int j = 0; j < NT; ++j)
                __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, acc[i][j]), pr, lofs + (uint32_t)((i * NT + j) * 64) * 16u, mine, 16);
        if (g.fenced) split_release();                                // the partial is visible at agent scope
        else wait_vm<0>();
        __syncthreads();
        if (threadIdx.x == 0) {
            const int old = __hip_atomic_fetch_add(g.cnt + tile, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            ws_flag = old == g.S - 1;
            if (old == g.S - 1) __hip_atomic_store(g.cnt + tile, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
        __syncthreads();
        if (!ws_flag) return;
        if (g.fenced) split_acquire();                                              // the other blocks' partials, not stale lines
        const uint32_t first = (uint32_t)(tile * g.S * E) * 4u;
        for (int z = 0; z < g.S; ++z) {                               // split order: the same sum whoever is last
            f32x4_t v[MT][NT];
#pragma unroll
            for (int i = 0; i < MT; ++i)
#pragma unroll
                for (int j = 0; j < NT; ++j)
                    v[i][j] = __builtin_bit_cast(f32x4_t, __builtin_amdgcn_raw_buffer_load_b128(
                                  pr, lofs + (uint32_t)((i * NT + j) * 64) * 16u, first + (uint32_t)z * part, 16));
#pragma unroll
            for (int i = 0; i < MT; ++i)
#pragma unroll
                for (int j = 0; j < NT; ++j) acc[i][j] = z == 0 ? v[i][j] : acc[i][j] + v[i][j];
        }
    }
    // every scale is loaded before the first store: a scale load between stores would make each store wait for the ones
    // before it (vmcnt counts stores)
    float sc[NT];
#pragma unroll
    for (int j = 0; j < NT; ++j) {
        const int nn = n0 + 16 * j + r16;
        sc[j] = nn < N ? row_scale<T>(g.srow, g.base + (ok ? lo : 0), g.sc_off, nn) : 0.f;
    }
#pragma unroll
    for (int j = 0; j < NT; ++j) {
        const int nn = n0 + 16 * j + r16;
        if (nn >= N) continue;
        const float s = sc[j];
#pragma unroll
        for (int i = 0; i < MT; ++i)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int m = 16 * i + 4 * lg + r;
                if (m < M) store_y(g.y, (int64_t)m * N + nn, ok ? acc[i][j][r] * s : __builtin_nanf(""), g.out_bf16);
            }
    }
}

// ------------------------------------------------------------------------------------------------------ launchers
template <int T, int MT>
static size_t ws_lds_bytes() { return (size_t)ws_depth<T>() * ws_rows<T, MT>() * ws_ki<T>() * sizeof(uint16_t); }

template <int T, int MT, int NT, bool KFULL>
static int ws_launch(const Args& a, int S, int kts, const Workspace& w, hipStream_t s) {
    auto kern = wsgemm_kernel<T, MT, NT, KFULL>;
    const size_t lds = ws_lds_bytes<T, MT>();
    static std::atomic<uint64_t> lds_set{0};
    if (set_lds_limit((const void*)kern, lds, lds_set) != hipSuccess)
        return set_error(MBQ_LAUNCH_FAIL, "weight-stream GEMM: %zu bytes of LDS refused", lds);
    WsArgs g{a.base, a.stride, a.layer_dev, a.nlayers, a.sc_off, a.wbytes, a.hi_off, a.d_off, a.srow, a.x, (int)a.M, (int)a.N, (int)a.K,
             a.y, a.out_bf16, S, kts, w.ws, w.cnt, (uint32_t)w.bytes, w.fenced};
    const int64_t tiles = (a.N + 64 * NT - 1) / (64 * NT);
    kern<<<dim3((unsigned)(tiles * S)), WS_THREADS, lds, s>>>(g);
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return set_error(MBQ_LAUNCH_FAIL, "weight-stream GEMM launch: %s", hipGetErrorString(e));
    return 0;
}

template <int T, int NT>
static int ws_launch_m(const Args& a, int S, int kts, const Workspace& w, hipStream_t s) {
    const bool kfull = a.K % ws_ki<T>() == 0;
    if constexpr (kquant(T)) {                       // rows of whole 256-value blocks
        switch ((a.M + 15) / 16) {
            case 1: return ws_launch<T, 1, NT, true>(a, S, kts, w, s);
            case 2: return ws_launch<T, 2, NT, true>(a, S, kts, w, s);
            case 3: return ws_launch<T, 3, NT, true>(a, S, kts, w, s);
            default: return ws_launch<T, 4, NT, true>(a, S, kts, w, s);
        }
    } else {
        switch ((a.M + 15) / 16) {
            case 1: return kfull ? ws_launch<T, 1, NT, true>(a, S, kts, w, s) : ws_launch<T, 1, NT, false>(a, S, kts, w, s);
            case 2: return kfull ? ws_launch<T, 2, NT, true>(a, S, kts, w, s) : ws_launch<T, 2, NT, false>(a, S, kts, w, s);
            case 3: return kfull ? ws_launch<T, 3, NT, true>(a, S, kts, w, s) : ws_launch<T, 3, NT, false>(a, S, kts, w, s);
            default: return kfull ? ws_launch<T, 4, NT, true>(a, S, kts, w, s) : ws_launch<T, 4, NT, false>(a, S, kts, w, s);
        }
    }
}


// float32 bytes of one block's partial tile
static size_t ws_partial_bytes(int64_t M, int nr) { return (size_t)((M + 15) / 16) * (nr / 64) * 1024 * 4; }

// Rows per block (64 or 128) and K splits, from timings on MI355X at 64 activation rows: when the 64-row tiles alone
// fill the CUs, 128-row blocks (each x stage feeds twice the weights) and no split; else 64-row blocks and as many K
// splits as fit the CUs in one round (3 for 80 tiles: 5120 x 17408 in 38 us instead of 50 with 2; 2 for 96, 8 for
// 16), at most 8 ranges of at least 512 K values (4 iterations of 128, 8 of 64), the partial tiles within the
// workspace.
static void ws_choose(int t, int64_t M, int64_t N, int64_t K, int cus, int* nr, int* S) {
    const int64_t KT = (K + ws_ki_of(t) - 1) / ws_ki_of(t);
    const int depth = unit32(t) ? 4 : 8;                          // iterations of 512 K values
    const int64_t tiles64 = (N + 63) / 64;
    if (tiles64 >= cus) {
        *nr = 128;
        *S = 1;
        return;
    }
    int64_t s = std::max<int64_t>(1, cus / tiles64);
    s = std::min<int64_t>({s, 8, std::max<int64_t>(1, KT / depth)});
    while (s > 1 && (tiles64 > WS_TILES || (size_t)tiles64 * s * ws_partial_bytes(M, 64) > WS_BYTES)) --s;
    *nr = 64;
    *S = (int)s;
}

int wsgemm_plan(int t, const Args& a, int* rows_per_block, int* splits) {
    ws_choose(t, a.M, a.N, a.K, cus_of_device(), rows_per_block, splits);
    return 0;
}

void wsgemm_effective(int t, const Args& a, int* nr, int* S) {
    (void)nr;
    const int64_t KT = (a.K + ws_ki_of(t) - 1) / ws_ki_of(t);
    const int64_t kts = (KT + std::max(1, *S) - 1) / std::max(1, *S);
    *S = (int)((KT + kts - 1) / kts);                              // no empty split
}

int launch_wsgemm(int t, const Args& a, int nr, int S, hipStream_t s) {
    if (a.M < 1 || a.M > WS_MAX_M) return set_error(MBQ_BAD_ARG, "weight-stream GEMM: M = %lld", (long long)a.M);
    if (nr != 64 && nr != 128) return set_error(MBQ_BAD_ARG, "weight-stream GEMM: %d rows per block (64 or 128)", nr);
    wsgemm_effective(t, a, &nr, &S);
    if (a.wbytes > BUF_MAX_BYTES || a.M * a.K * 2 > BUF_MAX_BYTES)
        return set_error(MBQ_BAD_ARG, "weight-stream GEMM operands over 2 GiB");
    const int64_t KT = (a.K + ws_ki_of(t) - 1) / ws_ki_of(t);
    const int64_t kts = (KT + S - 1) / S;
    const int64_t tiles = (a.N + nr - 1) / nr;
    Workspace w;
    if (S > 1)
        if (int rc = split_workspace(a, tiles, (size_t)tiles * S * ws_partial_bytes(a.M, nr), s, &w)) return rc;
    switch (t) {
        case T_INT8: return nr == 64 ? ws_launch_m<T_INT8, 1>(a, S, (int)kts, w, s) : ws_launch_m<T_INT8, 2>(a, S, (int)kts, w, s);
        case T_I8T: return nr == 64 ? ws_launch_m<T_I8T, 1>(a, S, (int)kts, w, s) : ws_launch_m<T_I8T, 2>(a, S, (int)kts, w, s);
        case T_Q4_0: return nr == 64 ? ws_launch_m<T_Q4_0, 1>(a, S, (int)kts, w, s) : ws_launch_m<T_Q4_0, 2>(a, S, (int)kts, w, s);
        case T_Q8_0: return nr == 64 ? ws_launch_m<T_Q8_0, 1>(a, S, (int)kts, w, s) : ws_launch_m<T_Q8_0, 2>(a, S, (int)kts, w, s);
        case T_Q4_K: return nr == 64 ? ws_launch_m<T_Q4_K, 1>(a, S, (int)kts, w, s) : ws_launch_m<T_Q4_K, 2>(a, S, (int)kts, w, s);
        case T_Q5_K: return nr == 64 ? ws_launch_m<T_Q5_K, 1>(a, S, (int)kts, w, s) : ws_launch_m<T_Q5_K, 2>(a, S, (int)kts, w, s);
        case T_Q6_K: return nr == 64 ? ws_launch_m<T_Q6_K, 1>(a, S, (int)kts, w, s) : ws_launch_m<T_Q6_K, 2>(a, S, (int)kts, w, s);
    }
    return set_error(MBQ_BAD_ARG, "weight-stream GEMM: no kernel for type %d", t);
}

}  // namespace mbq
