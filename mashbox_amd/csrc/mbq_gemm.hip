// gfx950 MFMA GEMM of the quantized linear for the prefill / batched-decode regime (many activation rows).
//
// y (M, N) = x (M, K) @ W.T with W dequantized on the fly: reference src/mashbox/ops/__init__.py:594-632 (qmatmul,
// float32 accumulation) on the weights of reference src/mashbox/ops/reference.py:101-103 (Q8_0) and :132-149 (Q4_K),
// and reference src/mashbox/models/qwen3_8_27b/model.py:72-82 (int8 per output channel: dot, then * s).
//
// Block tile BM x 256 (activation rows x weight rows), K step 64, 512 threads = 8 waves in a 2 x 4 grid; each wave owns a
// (BM/2) x 64 piece of the tile as (BM/32) x 4 tiles of v_mfma_f32_16x16x32_bf16 with float32 accumulators.
// Per K step every thread
//   - copies ACH 16-byte chunks of the x tile (bfloat16) into LDS,
//   - dequantizes one 32-value weight unit into LDS as bfloat16 (Q4_K: a sub-block, 16 bytes of nibbles + the
//     super-block's scales; Q8_0 / int8: 32 bytes of quants); each value is the float32 dequantization (d*sc)*q - dmin*m
//     resp. q*d rounded to nearest even (int8 values are exact),
//   - runs 2 K-substeps of MFMAs on the tiles of the step before, from the other LDS stage.
// Pipeline: the raw bytes of step k+2 are loaded into registers at the top of step k, the raw bytes of step k+1 (loaded
// one step earlier) are dequantized into LDS stage (k+1)&1 in slices placed between the MFMAs of step k, so global
// latency hides behind a whole step and the VALU dequant behind the matrix work; one barrier per step. The main loop is
// branch free: loads past the last row or step are clamped to valid addresses (they only feed outputs that are never
// stored, or an LDS stage nobody reads); only a K that is not a multiple of 64 (Q8_0, int8) zeroes the x chunks past K.
// LDS rows are 64 bfloat16 (8 chunks of 16 bytes) with chunk c stored at c ^ (row & 7), so the 16-byte MFMA operand
// reads of 8 consecutive rows hit distinct banks. Tiles are mapped to blocks XCD by XCD (blocks are dealt to the 8 XCDs
// round robin), so the blocks that share an x row-panel run on one XCD at once and share its L2.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "mbq_device.h"
#include "mbq_launch.h"
#include "mbq_layout.h"

namespace mbq {

constexpr int GK = 64, GT = 512;

// element offset of chunk c (8 bfloat16) of row r in an LDS tile of 64-value rows
__device__ __forceinline__ int lds_off(int r, int c) { return r * GK + ((c ^ (r & 7)) << 3); }

// buffer resources: loads carry a 32-bit per-lane offset and a scalar offset, and read zero past num_records
typedef __amdgpu_buffer_rsrc_t rsrc_t;
__device__ __forceinline__ rsrc_t make_rsrc(const void* p, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p), (short)0, (int)bytes, 0x00020000);
}
__device__ __forceinline__ u32x4 bload16(rsrc_t r, uint32_t voff, uint32_t soff) {
    return __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(r, voff, soff, 0));
}
__device__ __forceinline__ uint32_t bload2(rsrc_t r, uint32_t voff, uint32_t soff) {
    return (uint32_t)__builtin_amdgcn_raw_buffer_load_b16(r, voff, soff, 0);
}
// 16 bytes per lane from global memory straight into LDS: lane l writes lds_wave + 16 l (lds_wave wave-uniform)
__device__ __forceinline__ void dma16(rsrc_t r, uint16_t* lds_wave, uint32_t voff, uint32_t soff) {
    __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (__attribute__((address_space(3))) void*)lds_wave, 16, voff, soff, 0, 0);
}

// the raw bytes of one weight unit (32 values of one row), as loaded from the planes
template <int T> struct BUnit;
template <> struct BUnit<T_Q4_K> { u32x4 q, meta; };
template <> struct BUnit<T_Q8_0> { u32x4 q0, q1; uint32_t d; };
template <> struct BUnit<T_INT8> { u32x4 q0, q1; };
template <int T> constexpr int b_loads() { return T == T_Q8_0 ? 3 : 2; }   // buffer loads per unit

// per-thread byte offsets of a weight unit's planes (the K step's part goes in the scalar offset)
struct BOff { uint32_t q, s; };

template <int T>
__device__ __forceinline__ BOff b_off(int64_t sc_off, int64_t bn, int K, int u) {
    if constexpr (T == T_Q4_K) return BOff{(uint32_t)(bn * (K >> 1) + 16 * u), (uint32_t)(sc_off + bn * (K >> 8) * 16)};
    else return BOff{(uint32_t)(bn * K + 32 * u), (uint32_t)(sc_off + bn * (K >> 5) * 2 + 2 * u)};
}

// loads unit u of the K step at k0; with KFULL false, a Q8_0 unit past K gets scale 0 (its quants may be any bytes;
// the x they meet is zero)
template <int T, bool KFULL>
__device__ __forceinline__ void b_load(BUnit<T>& b, rsrc_t r, const BOff& o, int K, int k0, int u) {
    if constexpr (T == T_Q4_K) {
        b.q = bload16(r, o.q, (uint32_t)k0 >> 1);
        b.meta = bload16(r, o.s, ((uint32_t)k0 >> 8) * 16);
    } else {
        b.q0 = bload16(r, o.q, (uint32_t)k0);
        b.q1 = bload16(r, o.q + 16, (uint32_t)k0);
        if constexpr (T == T_Q8_0) {
            b.d = bload2(r, o.s, ((uint32_t)k0 >> 5) * 2);
            if constexpr (!KFULL) b.d = (k0 + 32 * u < K) ? b.d : 0u;
        }
    }
}

// 4 int8 quants (one dword) -> 2 bfloat16 pairs of q * d (exact in float32: q * d has at most 19 significant bits)
template <bool SCALED>
__device__ __forceinline__ void i8x4(uint32_t w, float d, float d128, uint32_t* o) {
    const uint32_t x = opaque(w ^ 0x80808080u);     // bytes q + 128
    const float u0 = (float)(x & 0xFFu), u1 = (float)((x >> 8) & 0xFFu);
    const float u2 = (float)((x >> 16) & 0xFFu), u3 = (float)(x >> 24);
    if constexpr (SCALED) {   // (q + 128) * d - 128 * d = q * d, one exact FMA
        o[0] = pack_bf16(__builtin_fmaf(u0, d, -d128), __builtin_fmaf(u1, d, -d128));
        o[1] = pack_bf16(__builtin_fmaf(u2, d, -d128), __builtin_fmaf(u3, d, -d128));
    } else {
        o[0] = pack_bf16(u0 - 128.f, u1 - 128.f);
        o[1] = pack_bf16(u2 - 128.f, u3 - 128.f);
    }
}

// per-unit dequant constants
struct BScale { float a, b, c; };   // Q4_K: d*sc, dmin*m, d*sc/16; Q8_0: d, 128 d

template <int T>
__device__ __forceinline__ BScale b_scale(const BUnit<T>& b, int j) {
    BScale s{1.f, 128.f, 0.f};
    if constexpr (T == T_Q4_K) {
        uint32_t sc, mn;
        q4k_scale_min_sel(b.meta[1], b.meta[2], b.meta[3], q4k_sel(j), &sc, &mn);
        s.a = f16f(b.meta[0]) * (float)sc;                   // exact
        s.b = f16f(b.meta[0] >> 16) * (float)mn;             // exact
        s.c = s.a * 0.0625f;                                 // exact: a power-of-two scale
    } else if constexpr (T == T_Q8_0) {
        s.a = f16f(b.d);
        s.b = 128.f * s.a;
    }
    return s;
}

// chunk t (0..3: values 8t .. 8t+7) of a unit, as 8 bfloat16
template <int T>
__device__ __forceinline__ u32x4 b_chunk(const BUnit<T>& b, const BScale& s, int t) {
    u32x4 o;
    if constexpr (T == T_Q4_K) {
        // dword t: quant 8t+2p in bits 4p..4p+3, quant 8t+2p+1 in bits 16+4p.. (mbq_layout.h)
        const uint32_t w = b.q[t];
        const uint32_t m0 = opaque(w & 0x000F000Fu), m1 = opaque(w & 0x00F000F0u);
        const uint32_t m2 = opaque(w & 0x0F000F00u), m3 = opaque(w & 0xF000F000u);
        o[0] = pack_bf16(__builtin_fmaf((float)(m0 & 0xFFu), s.a, -s.b), __builtin_fmaf((float)((m0 >> 16) & 0xFFu), s.a, -s.b));
        o[1] = pack_bf16(__builtin_fmaf((float)(m1 & 0xFFu), s.c, -s.b), __builtin_fmaf((float)((m1 >> 16) & 0xFFu), s.c, -s.b));
        o[2] = pack_bf16(__builtin_fmaf((float)((m2 >> 8) & 0xFFu), s.a, -s.b), __builtin_fmaf((float)(m2 >> 24), s.a, -s.b));
        o[3] = pack_bf16(__builtin_fmaf((float)((m3 >> 8) & 0xFFu), s.c, -s.b), __builtin_fmaf((float)(m3 >> 24), s.c, -s.b));
    } else {
        const u32x4 q = t < 2 ? b.q0 : b.q1;
        const int h = (t & 1) * 2;
        uint32_t r[4];
        i8x4<T == T_Q8_0>(q[h], s.a, s.b, &r[0]);
        i8x4<T == T_Q8_0>(q[h + 1], s.a, s.b, &r[2]);
        o = u32x4{r[0], r[1], r[2], r[3]};
    }
    return o;
}

template <int T, int BM, int BN, bool KFULL>
__global__ __launch_bounds__(GT, 1) void gemm_kernel(const uint8_t* __restrict__ base, int64_t stride,
                                                     const int32_t* __restrict__ layer_dev, int nlayers, int64_t sc_off,
                                                     int64_t wbytes, const float* __restrict__ srow,
                                                     const uint16_t* __restrict__ x, int M, int N, int K,
                                                     void* __restrict__ y, int out_bf16) {
    extern __shared__ __attribute__((aligned(16))) uint16_t gemm_lds[];   // [A stage 0][A stage 1][B stage 0][B stage 1]
    uint16_t* const B0 = gemm_lds + 2 * BM * GK;
    constexpr int TI = BM / 32, TJ = BN / 64;           // MFMA tiles per wave
    constexpr int XD = BM / 64;                         // x DMA instructions per wave per step (8 rows each)
    constexpr int NB = b_loads<T>();

    // XCD-aware tile order: block b runs on XCD b % 8; XCD x takes a contiguous range of tiles, N fastest, so the
    // blocks running at once on one XCD share one x row-panel (BM x K) in that XCD's L2
    const int MT = (M + BM - 1) / BM, NT = (N + BN - 1) / BN, T_ = MT * NT;
    const int b = blockIdx.x, xcd = b & 7, q = T_ >> 3, rem = T_ & 7;
    const int tile = xcd * q + min(xcd, rem) + (b >> 3);
    const int m0 = (tile / NT) * BM, n0 = (tile % NT) * BN;

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wm = wave >> 2, wn = wave & 3;
    const int64_t lo = layer_offset(stride, layer_dev, nlayers);
    const bool ok = lo >= 0;
    base += ok ? lo : 0;
    const rsrc_t wr = make_rsrc(base, (uint32_t)wbytes);
    const rsrc_t xr = make_rsrc(x, (uint32_t)((int64_t)M * K * 2));

    // x tile by DMA: instruction i of wave w fills tile rows 8 (w + 8 i) .. +7; lane l writes LDS slot l & 7 of row
    // l >> 3, which holds chunk (l & 7) ^ (l >> 3) of that row (the swizzle of lds_off). Rows past M read zero.
    uint32_t xvo[XD];
    int xk[XD];
#pragma unroll
    for (int i = 0; i < XD; ++i) {
        const int r = 8 * (wave + 8 * i) + (lane >> 3), c = (lane & 7) ^ (lane >> 3);
        xvo[i] = (uint32_t)(((int64_t)(m0 + r) * K + c * 8) * 2);
        xk[i] = c * 8;
    }
    auto dma_x = [&](int s, int k0) {
#pragma unroll
        for (int i = 0; i < XD; ++i) {
            uint32_t v = xvo[i];
            if constexpr (!KFULL) v = (k0 + xk[i] < K) ? v : 0x7FFFFFF0u;     // past K: out of range, reads zero
            dma16(xr, gemm_lds + s * BM * GK + 8 * (wave + 8 * i) * GK, v, (uint32_t)k0 * 2);
        }
    };

    // this thread's weight unit: row br (clamped to N-1: rows past N only feed outputs that are never stored), unit bu;
    // the tile has 2 BN units, so with BN < 256 the threads from 2 BN on dequantize nothing
    constexpr bool ALL_OWN = 2 * BN >= GT;
    const int br = ALL_OWN ? tid >> 1 : min(tid >> 1, BN - 1), bu = tid & 1;
    const bool bown = ALL_OWN || tid < 2 * BN;
    const BOff bo = b_off<T>(sc_off, min(n0 + br, N - 1), K, bu);

    f32x4_t acc[TI][TJ];
#pragma unroll
    for (int i = 0; i < TI; ++i)
#pragma unroll
        for (int j = 0; j < TJ; ++j) acc[i][j] = f32x4_t{0.f, 0.f, 0.f, 0.f};

    const int KT = ok ? (K + GK - 1) / GK : 0;

    // one pipeline step: MFMAs on stage kt & 1; meanwhile x of step kt + 1 streams into the other stage by DMA, the
    // weight unit of step kt + 1 (`dq`, loaded a step ago) is dequantized into it in slices between the MFMAs, and the
    // weight unit of step kt + 2 is loaded into `nl`
    auto step = [&](int kt, BUnit<T>& nl, const BUnit<T>& dq) {
        const int cur = kt & 1, nxt = cur ^ 1, kn = (kt + 1) * GK;
        dma_x(nxt, min(kt + 1, KT - 1) * GK);
        __builtin_amdgcn_sched_barrier(0);             // the DMA stays ahead of the weight loads (vmcnt order below)
        b_load<T, KFULL>(nl, wr, bo, K, min(kt + 2, KT - 1) * GK, bu);
        const uint16_t* Ac = gemm_lds + cur * BM * GK;
        const uint16_t* Bc = B0 + cur * BN * GK;
        uint16_t* Bn = B0 + nxt * BN * GK + br * GK;
        const BScale sc = b_scale<T>(dq, ((kn >> 5) + bu) & 7);
#pragma unroll
        for (int ks = 0; ks < 2; ++ks) {
            const int c = ks * 4 + (lane >> 4);
            bf16x8_t bb[TJ];
#pragma unroll
            for (int j = 0; j < TJ; ++j)
                bb[j] = *reinterpret_cast<const bf16x8_t*>(Bc + lds_off(wn * (BN / 4) + j * 16 + (lane & 15), c));
#pragma unroll
            for (int i = 0; i < TI; ++i) {
                const bf16x8_t a = *reinterpret_cast<const bf16x8_t*>(Ac + lds_off(wm * (BM / 2) + i * 16 + (lane & 15), c));
#pragma unroll
                for (int j = 0; j < TJ; ++j) acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, bb[j], acc[i][j], 0, 0, 0);
                // one 16-byte chunk of the next stage's weight tile after every few activation-row tiles
                constexpr int EVERY = TI / 2;
                if (i % EVERY == EVERY - 1) {
                    const int t = ks * 2 + i / EVERY;
                    if (bown) st16(Bn + (((4 * bu + t) ^ (br & 7)) << 3), b_chunk<T>(dq, sc, t));
                }
            }
        }
        // the x DMA of step kt + 1 has landed once at most the NB weight loads issued after it are in flight
        __builtin_amdgcn_s_waitcnt(0x0F70 | NB);
        __syncthreads();
    };

    BUnit<T> r0, r1;
    if (KT > 0) {
        dma_x(0, 0);
        b_load<T, KFULL>(r0, wr, bo, K, 0, bu);
        b_load<T, KFULL>(r1, wr, bo, K, min(1, KT - 1) * GK, bu);
        const BScale sc = b_scale<T>(r0, bu);
        if (bown)
#pragma unroll
            for (int t = 0; t < 4; ++t) st16(B0 + br * GK + (((4 * bu + t) ^ (br & 7)) << 3), b_chunk<T>(r0, sc, t));
        __builtin_amdgcn_s_waitcnt(0x0F70);              // vmcnt(0): the first x tile has landed
    }
    __syncthreads();
    // both steps of a pair unconditional, so that no load is sunk into a conditional block (its latency must overlap
    // the step before its use); an odd step count ends with one more step
    int kt = 0;
    for (; kt + 1 < KT; kt += 2) {
        step(kt, r0, r1);
        step(kt + 1, r1, r0);
    }
    if (kt < KT) step(kt, r0, r1);

    // epilogue: lane holds column n = lane & 15 and rows 4 * (lane >> 4) + r of each 16 x 16 tile
#pragma unroll
    for (int j = 0; j < TJ; ++j) {
        const int n = n0 + wn * (BN / 4) + j * 16 + (lane & 15);
        if (n >= N) continue;
        const float s = (T == T_INT8) ? srow[n] : 1.f;
#pragma unroll
        for (int i = 0; i < TI; ++i)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int m = m0 + wm * (BM / 2) + i * 16 + (lane >> 4) * 4 + r;
                if (m < M) store_y(y, (int64_t)m * N + n, ok ? acc[i][j][r] * s : __builtin_nanf(""), out_bf16);
            }
    }
}

template <int T, int BM, int BN, bool KFULL>
static int launch_tile(const Args& a, hipStream_t s) {
    auto kern = gemm_kernel<T, BM, BN, KFULL>;
    const size_t lds = (size_t)(2 * BM * GK + 2 * BN * GK) * sizeof(uint16_t);
    static bool attr_set = false;
    if (!attr_set) {
        if (hipFuncSetAttribute((const void*)kern, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds) != hipSuccess)
            return set_error(MBQ_LAUNCH_FAIL, "GEMM: %zu bytes of LDS refused", lds);
        attr_set = true;
    }
    const int64_t tiles = ((a.M + BM - 1) / BM) * ((a.N + BN - 1) / BN);
    kern<<<dim3((unsigned)tiles), GT, lds, s>>>(a.base, a.stride, a.layer_dev, a.nlayers, a.sc_off, a.wbytes, a.srow, a.x,
                                                (int)a.M, (int)a.N, (int)a.K, a.y, a.out_bf16);
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return set_error(MBQ_LAUNCH_FAIL, "GEMM launch: %s", hipGetErrorString(e));
    return 0;
}

template <int T, int BM, int BN>
static int launch_k(const Args& a, hipStream_t s) {
    return (a.K % GK == 0) ? launch_tile<T, BM, BN, true>(a, s) : launch_tile<T, BM, BN, false>(a, s);
}

// compute units of the current device (cached per device)
static int cu_count() {
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

// Tile shape for an (M, N) problem: the one with the least modelled time, where time = rounds of tiles over the CUs
// (one block per CU: the LDS stages take most of a CU's 160 KB) x the tile's work x a per-tile overhead that shrinks
// with the tile's size (operand traffic per flop ~ 1/BM + 1/BN).
template <int T>
static int launch_gemm_t(const Args& a, hipStream_t s) {
    // buffer resources address one weight's planes and the whole x with 32-bit offsets
    if (a.wbytes >= ((int64_t)1 << 31) || a.M * a.K * 2 >= ((int64_t)1 << 31))
        return set_error(MBQ_BAD_ARG, "GEMM operands over 2 GiB (weight %lld bytes, x %lld x %lld)", (long long)a.wbytes,
                         (long long)a.M, (long long)a.K);
    const int cus = cu_count();
    static const int shapes[][2] = {{256, 256}, {256, 192}, {256, 128}, {128, 256}, {128, 192}, {128, 128}, {128, 64}, {64, 256}, {64, 128}, {64, 64}};
    int best = 0;
    double best_t = 1e300;
    for (int i = 0; i < (int)(sizeof shapes / sizeof shapes[0]); ++i) {
        const int bm = shapes[i][0], bn = shapes[i][1];
        if (bm > 64 && a.M <= bm / 2) continue;            // more than half the tile's rows would be padding
        const int64_t tiles = ((a.M + bm - 1) / bm) * ((a.N + bn - 1) / bn);
        const int64_t rounds = (tiles + cus - 1) / cus;
        const double t = (double)rounds * bm * bn * (1.0 + 64.0 / bm + 64.0 / bn);
        if (t < best_t) best_t = t, best = i;
    }
    switch (best) {
        case 0: return launch_k<T, 256, 256>(a, s);
        case 1: return launch_k<T, 256, 192>(a, s);
        case 2: return launch_k<T, 256, 128>(a, s);
        case 3: return launch_k<T, 128, 256>(a, s);
        case 4: return launch_k<T, 128, 192>(a, s);
        case 5: return launch_k<T, 128, 128>(a, s);
        case 6: return launch_k<T, 128, 64>(a, s);
        case 7: return launch_k<T, 64, 256>(a, s);
        case 8: return launch_k<T, 64, 128>(a, s);
        default: return launch_k<T, 64, 64>(a, s);
    }
}

int launch_gemm(int t, const Args& a, hipStream_t s) {
    switch (t) {
        case T_Q8_0: return launch_gemm_t<T_Q8_0>(a, s);
        case T_Q4_K: return launch_gemm_t<T_Q4_K>(a, s);
        case T_INT8: return launch_gemm_t<T_INT8>(a, s);
    }
    return set_error(MBQ_BAD_ARG, "no GEMM for type %d", t);
}

}  // namespace mbq
