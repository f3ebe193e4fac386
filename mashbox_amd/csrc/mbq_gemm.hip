// gfx950 MFMA GEMM of the quantized linear for the prefill / batched-decode regime (many activation rows).
//
// y (M, N) = x (M, K) @ W.T with W dequantized on the fly: reference src/mashbox/ops/__init__.py:594-632 (qmatmul,
// float32 accumulation) on the weights of reference src/mashbox/ops/reference.py:66-70 (Q4_0), :101-103 (Q8_0),
// :132-149 (Q4_K), :150-159 (Q5_K) and :164-173 (Q6_K),
// and reference src/mashbox/models/qwen3_8_27b/model.py:72-82 (int8 per output channel: dot, then * s).
//
// Block tile BM x 256 (activation rows x weight rows), K step 64, 512 threads = 8 waves in a 2 x 4 grid; each wave owns a
// (BM/2) x 64 piece of the tile as (BM/32) x 4 tiles of v_mfma_f32_16x16x32_bf16 with float32 accumulators.
// Per K step every thread
//   - copies ACH 16-byte chunks of the x tile (bfloat16) into LDS,
//   - dequantizes one 32-value weight unit into LDS as bfloat16 (Q4_K: a sub-block, 16 bytes of nibbles + the
//     super-block's scales; Q4_0: a block, 16 bytes of nibbles and its scale; Q6_K: 16 bytes of low nibbles, 8 of high
//     bits, 2 sub-block scales and the super-block scale; Q8_0 / int8: 32 bytes of quants); each value is the float32
//     dequantization (d*sc)*q - dmin*m, d*(q - 8), (d*sc)*(q - 32) resp. q*d rounded to nearest even (int8 values are
//     exact),
//   - runs 2 K-substeps of MFMAs on the tiles of the step before, from the other LDS stage.
// Pipeline: the raw bytes of step k+2 are loaded into registers at the top of step k, the raw bytes of step k+1 (loaded
// one step earlier) are dequantized into LDS stage (k+1)&1 in slices placed between the MFMAs of step k, so global
// latency hides behind a whole step and the VALU dequant behind the matrix work; one barrier per step. The main loop is
// branch free: loads past the last row or step are clamped to valid addresses (they only feed outputs that are never
// stored, or an LDS stage nobody reads); only a K that is not a multiple of 64 (Q4_0, Q8_0, int8) zeroes the x chunks
// past K.
// LDS rows are 64 bfloat16 (8 chunks of 16 bytes) with chunk c stored at c ^ (row & 7), so the 16-byte MFMA operand
// reads of 8 consecutive rows hit distinct banks. Tiles are mapped to blocks XCD by XCD (blocks are dealt to the 8 XCDs
// round robin), so the blocks that share an x row-panel run on one XCD at once and share its L2.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <algorithm>
#include <atomic>
#include <mutex>
#include <type_traits>

#include "mbq_device.h"
#include "mbq_launch.h"
#include "mbq_layout.h"

namespace mbq {

constexpr int GK = 64, GT = 512;

// element offset of chunk c (8 bfloat16) of row r in an LDS tile of 64-value rows
__device__ __forceinline__ int lds_off(int r, int c) { return r * GK + ((c ^ (r & 7)) << 3); }

// the raw bytes of one weight unit (32 values of one row), as loaded from the planes
template <int T> struct BUnit;
template <> struct BUnit<T_Q4_K> { u32x4 q, meta; };
template <> struct BUnit<T_Q4KT> { u32x4 q, meta; };
template <> struct BUnit<T_Q4_0> { u32x4 q; uint32_t d; };
template <> struct BUnit<T_Q40T> { u32x4 q; uint32_t d; };
template <> struct BUnit<T_Q8_0> { u32x4 q0, q1; uint32_t d; };
template <> struct BUnit<T_Q8T> { u32x4 q0, q1; uint32_t d; };
template <> struct BUnit<T_INT8> { u32x4 q0, q1; };
template <> struct BUnit<T_I8T> { u32x4 q0, q1; };
template <> struct BUnit<T_Q6_K> { u32x4 q; u32x2 h; uint32_t s, d; };
template <> struct BUnit<T_Q6KT> { u32x4 q; u32x2 h; uint32_t s, d; };
template <> struct BUnit<T_Q5_K> { u32x4 q, meta; uint32_t h; };
template <> struct BUnit<T_Q5KT> { u32x4 q, meta; uint32_t h; };
template <int T> constexpr int b_loads() { return T == T_Q8T ? 5 : q6k_like(T) ? 4 : (T == T_Q8_0 || q5k_like(T)) ? 3 : 2; }   // buffer loads per unit

// per-thread byte offsets of a weight unit's planes (the K step's part goes in the scalar offset); h: Q5_K, Q6_K; d: Q6_K
struct BOff { uint32_t q, s, h, d; };

template <int T>
__device__ __forceinline__ BOff b_off(int64_t sc_off, int64_t hi_off, int64_t d_off, int64_t bn, int K, int u) {
    if constexpr (T == T_Q6_K)
        return BOff{(uint32_t)(bn * (K >> 1) + 16 * u), (uint32_t)(sc_off + bn * (K >> 4) + 2 * u),
                    (uint32_t)(hi_off + bn * (K >> 2) + 8 * u), (uint32_t)(d_off + bn * (K >> 7))};
    else if constexpr (T == T_Q6KT)
        return BOff{(uint32_t)(q4kt_off(bn, K) + 16 * u), (uint32_t)(sc_off + q6kt_s_off(bn, K) + 2 * u),
                    (uint32_t)(hi_off + q6kt_h_off(bn, K) + 8 * u), (uint32_t)(d_off + q6kt_d_off(bn, K))};
    else if constexpr (T == T_Q5KT)
        return BOff{(uint32_t)(q4kt_off(bn, K) + 16 * u), (uint32_t)(sc_off + q4kt_meta_off(bn, K)), (uint32_t)(hi_off + q5kt_h_off(bn, K) + 4 * u), 0};
    else if constexpr (T == T_Q5_K)
        return BOff{(uint32_t)(bn * (K >> 1) + 16 * u), (uint32_t)(sc_off + bn * (K >> 8) * 16), (uint32_t)(hi_off + bn * (K >> 3) + 4 * u), 0};
    else if constexpr (T == T_Q4_K) return BOff{(uint32_t)(bn * (K >> 1) + 16 * u), (uint32_t)(sc_off + bn * (K >> 8) * 16), 0, 0};
    else if constexpr (T == T_Q4KT) return BOff{(uint32_t)(q4kt_off(bn, K) + 16 * u), (uint32_t)(sc_off + q4kt_meta_off(bn, K)), 0, 0};
    else if constexpr (T == T_Q40T) return BOff{(uint32_t)(q40t_off(bn, K) + 16 * u), (uint32_t)(sc_off + q40t_d_off(bn, K) + 2 * u), 0, 0};
    else if constexpr (T == T_Q4_0) return BOff{(uint32_t)(bn * (K >> 1) + 16 * u), (uint32_t)(sc_off + bn * (K >> 5) * 2 + 2 * u), 0, 0};
    else if constexpr (T == T_I8T) return BOff{(uint32_t)(i8t_off(bn, K, 0) + 32 * u), 0, 0, 0};   // 16-row tiles
    else if constexpr (T == T_Q8T) return BOff{(uint32_t)(i8t_off(bn, K, 0) + 8 * u), (uint32_t)(sc_off + q8t_d_off(bn, K) + 2 * u), 0, 0};
    else return BOff{(uint32_t)(bn * K + 32 * u), (uint32_t)(sc_off + bn * (K >> 5) * 2 + 2 * u), 0, 0};
}

// loads unit u of the K step at k0; with KFULL false, a Q4_0 / Q8_0 unit past K gets scale 0 (its quants may be any
// bytes; the x they meet is zero)
template <int T, bool KFULL>
__device__ __forceinline__ void b_load(BUnit<T>& b, rsrc_t r, const BOff& o, int K, int k0, int u) {
    if constexpr (T == T_Q6_K) {
        b.q = bload16(r, o.q, (uint32_t)k0 >> 1);
        b.h = __builtin_bit_cast(u32x2, __builtin_amdgcn_raw_buffer_load_b64(r, o.h, (uint32_t)k0 >> 2, 0));
        b.s = bload2(r, o.s, (uint32_t)k0 >> 4);
        b.d = bload2(r, o.d, ((uint32_t)k0 >> 8) * 2);
    } else if constexpr (T == T_Q6KT) {
        // the step's half of the chunk (values 128 (k0 / 128) + 64 ((k0 / 64) % 2) ..) in each tiled plane
        b.q = bload16(r, o.q, ((uint32_t)k0 >> 7) * 1024u + (((uint32_t)k0 >> 1) & 63u));
        b.h = __builtin_bit_cast(u32x2, __builtin_amdgcn_raw_buffer_load_b64(r, o.h, ((uint32_t)k0 >> 7) * 512u + (((uint32_t)k0 >> 2) & 31u), 0));
        b.s = bload2(r, o.s, ((uint32_t)k0 >> 7) * 128u + (((uint32_t)k0 >> 4) & 7u));
        b.d = bload2(r, o.d, ((uint32_t)k0 >> 8) * 32u);
    } else if constexpr (T == T_Q4KT || T == T_Q5KT) {
        // the step's 32 bytes of the row sit in the tile block of values 128 (k0 / 128) .., at byte (k0 / 2) % 64
        b.q = bload16(r, o.q, ((uint32_t)k0 >> 7) * 1024u + (((uint32_t)k0 >> 1) & 63u));
        b.meta = bload16(r, o.s, ((uint32_t)k0 >> 8) * 256);
        if constexpr (T == T_Q5KT)
            b.h = (uint32_t)__builtin_amdgcn_raw_buffer_load_b32(r, o.h, ((uint32_t)k0 >> 7) * 256u + (((uint32_t)k0 >> 3) & 15u), 0);
    } else if constexpr (T == T_Q4_K || T == T_Q5_K) {
        b.q = bload16(r, o.q, (uint32_t)k0 >> 1);
        b.meta = bload16(r, o.s, ((uint32_t)k0 >> 8) * 16);
        if constexpr (T == T_Q5_K) b.h = (uint32_t)__builtin_amdgcn_raw_buffer_load_b32(r, o.h, (uint32_t)k0 >> 3, 0);
    } else if constexpr (q40_like(T)) {
        // T_Q40T: the step's two units in the tile block of values 128 (k0 / 128) .., and their scales beside
        b.q = bload16(r, o.q, T == T_Q40T ? ((uint32_t)k0 >> 7) * 1024u + (((uint32_t)k0 >> 1) & 63u) : (uint32_t)k0 >> 1);
        b.d = bload2(r, o.s, T == T_Q40T ? ((uint32_t)k0 >> 7) * 128u + (((uint32_t)k0 >> 5) & 3u) * 2u : ((uint32_t)k0 >> 5) * 2);
        if constexpr (!KFULL) b.d = (k0 + 32 * u < K) ? b.d : 0u;
    } else {
        const uint32_t qk = (T == T_I8T || T == T_Q8T) ? (uint32_t)k0 * 16u : (uint32_t)k0;   // tiles: a KiB per 64 values
        if constexpr (T == T_Q8T) {
            // the block's quants 8g .. 8g + 7 sit 16 g bytes apart (its other 8 bytes of each group: the other block)
            u32x2 p[4];
#pragma unroll
            for (int g = 0; g < 4; ++g)
                p[g] = __builtin_bit_cast(u32x2, __builtin_amdgcn_raw_buffer_load_b64(r, o.q + 16u * g, qk, 0));
            b.q0 = u32x4{p[0][0], p[0][1], p[1][0], p[1][1]};
            b.q1 = u32x4{p[2][0], p[2][1], p[3][0], p[3][1]};
        } else {
            b.q0 = bload16(r, o.q, qk);
            b.q1 = bload16(r, o.q + 16, qk);
        }
        if constexpr (q8_like(T)) {
            b.d = bload2(r, o.s, T == T_Q8T ? ((uint32_t)k0 >> 6) * 64u : ((uint32_t)k0 >> 5) * 2);
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
// Q4_K, Q5_K: d*sc, dmin*m, d*sc/16; Q4_0: d, 8 d, d/16; Q8_0: d, 128 d; Q6_K: d*sc0, 32 d*sc0, d*sc1, 32 d*sc1
struct BScale { float a, b, c, e; };

template <int T>
__device__ __forceinline__ BScale b_scale(const BUnit<T>& b, int j) {
    BScale s{1.f, 128.f, 0.f, 0.f};
    if constexpr (q6k_like(T)) {
        const float d = f16f(b.d);
        s.a = d * (float)(int8_t)(b.s & 0xFFu);           // exact
        s.b = 32.f * s.a;
        s.c = d * (float)(int8_t)((b.s >> 8) & 0xFFu);
        s.e = 32.f * s.c;
    } else if constexpr (q4k_like(T) || q5k_like(T)) {
        uint32_t sc, mn;
        q4k_scale_min_sel(b.meta[1], b.meta[2], b.meta[3], q4k_sel(j), &sc, &mn);
        s.a = f16f(b.meta[0]) * (float)sc;                   // exact
        s.b = f16f(b.meta[0] >> 16) * (float)mn;             // exact
        s.c = s.a * 0.0625f;                                 // exact: a power-of-two scale
    } else if constexpr (q40_like(T)) {
        s.a = f16f(b.d);
        s.b = 8.f * s.a;                                     // q d - 8 d = (q - 8) d, exact in float32
        s.c = s.a * 0.0625f;
    } else if constexpr (q8_like(T)) {
        s.a = f16f(b.d);
        s.b = 128.f * s.a;
    }
    return s;
}

// element i (0..3) of a vector, by selects (an index that varies across lanes must not send the vector to scratch)
__device__ __forceinline__ uint32_t sel4(const u32x4& v, int i) {
    const uint32_t lo = (i & 1) ? v[1] : v[0], hi = (i & 1) ? v[3] : v[2];
    return (i & 2) ? hi : lo;
}

// chunk t (0..3: values 8t .. 8t+7) of a unit, as 8 bfloat16
template <int T>
__device__ __forceinline__ u32x4 b_chunk(const BUnit<T>& b, const BScale& s, int t) {
    u32x4 o;
    if constexpr (q6k_like(T)) {
        // the quants of values 8t .. 8t+3 and 8t+4 .. 8t+7 as bytes; (q - 32) * (d sc) is one exact FMA
        uint32_t lo, hi;
        q6k_bytes(sel4(b.q, t), (t & 2) ? b.h[1] : b.h[0], t, &lo, &hi);
        const float ds = (t & 2) ? s.c : s.a, m = (t & 2) ? s.e : s.b;
        o[0] = pack_bf16(__builtin_fmaf((float)(lo & 0xFFu), ds, -m), __builtin_fmaf((float)((lo >> 8) & 0xFFu), ds, -m));
        o[1] = pack_bf16(__builtin_fmaf((float)((lo >> 16) & 0xFFu), ds, -m), __builtin_fmaf((float)(lo >> 24), ds, -m));
        o[2] = pack_bf16(__builtin_fmaf((float)(hi & 0xFFu), ds, -m), __builtin_fmaf((float)((hi >> 8) & 0xFFu), ds, -m));
        o[3] = pack_bf16(__builtin_fmaf((float)((hi >> 16) & 0xFFu), ds, -m), __builtin_fmaf((float)(hi >> 24), ds, -m));
    } else if constexpr (q5k_like(T)) {
        // the quants of values 8t .. 8t+3 and 8t+4 .. 8t+7 as bytes; (d sc) q - dmin m is one FMA with one rounding
        uint32_t lo, hi;
        q5k_bytes(sel4(b.q, t), b.h, t, &lo, &hi);
        o[0] = pack_bf16(__builtin_fmaf((float)(lo & 0xFFu), s.a, -s.b), __builtin_fmaf((float)((lo >> 8) & 0xFFu), s.a, -s.b));
        o[1] = pack_bf16(__builtin_fmaf((float)((lo >> 16) & 0xFFu), s.a, -s.b), __builtin_fmaf((float)(lo >> 24), s.a, -s.b));
        o[2] = pack_bf16(__builtin_fmaf((float)(hi & 0xFFu), s.a, -s.b), __builtin_fmaf((float)((hi >> 8) & 0xFFu), s.a, -s.b));
        o[3] = pack_bf16(__builtin_fmaf((float)((hi >> 16) & 0xFFu), s.a, -s.b), __builtin_fmaf((float)(hi >> 24), s.a, -s.b));
    } else if constexpr (nib4(T)) {
        // dword t: quant 8t+2p in bits 4p..4p+3, quant 8t+2p+1 in bits 16+4p.. (mbq_layout.h); two masks leave bytes
        // (q0, q4, q1, q5) and (16 q2, 16 q6, 16 q3, 16 q7), the latter taking the scale / 16
        const uint32_t w = sel4(b.q, t);
        const uint32_t lo = opaque(w & 0x0F0F0F0Fu), hi = opaque(w & 0xF0F0F0F0u);
        auto f = [](uint32_t v, int by) { return (float)((v >> (8 * by)) & 0xFFu); };
        o[0] = pack_bf16(__builtin_fmaf(f(lo, 0), s.a, -s.b), __builtin_fmaf(f(lo, 2), s.a, -s.b));
        o[1] = pack_bf16(__builtin_fmaf(f(hi, 0), s.c, -s.b), __builtin_fmaf(f(hi, 2), s.c, -s.b));
        o[2] = pack_bf16(__builtin_fmaf(f(lo, 1), s.a, -s.b), __builtin_fmaf(f(lo, 3), s.a, -s.b));
        o[3] = pack_bf16(__builtin_fmaf(f(hi, 1), s.c, -s.b), __builtin_fmaf(f(hi, 3), s.c, -s.b));
    } else {
        // dwords 2t, 2t+1 of the unit's 8 (q0: 0..3, q1: 4..7)
        const uint32_t w0 = (t & 2) ? ((t & 1) ? b.q1[2] : b.q1[0]) : ((t & 1) ? b.q0[2] : b.q0[0]);
        const uint32_t w1 = (t & 2) ? ((t & 1) ? b.q1[3] : b.q1[1]) : ((t & 1) ? b.q0[3] : b.q0[1]);
        uint32_t r[4];
        i8x4<q8_like(T)>(w0, s.a, s.b, &r[0]);
        i8x4<q8_like(T)>(w1, s.a, s.b, &r[2]);
        o = u32x4{r[0], r[1], r[2], r[3]};
    }
    return o;
}

// rows of one LDS weight stage: the tile's rows, plus 16 private rows of a 192-row tile's spare threads
constexpr int b_rows(int bn) { return (GT % (2 * bn) == 0) ? bn : bn + 16; }

// kernel arguments
struct GemmArgs {
    const uint8_t* base;        // planes of the weight (host layer applied)
    int64_t stride;             // bytes between stacked weights (layer_dev)
    const int32_t* layer_dev;   // device layer index, or nullptr
    int nlayers;
    int64_t sc_off, wbytes;     // scale plane offset and bytes of one weight's planes
    int64_t hi_off, d_off;      // Q6_K high-bit and super-block scale planes
    const float* srow;          // int8: per-row scales
    const uint16_t* x;
    int M, N, K;
    void* y;
    int out_bf16;
    int S, kts;                 // K splits and K steps per split
    float* ws;                  // S > 1: partial tiles, BM x BN floats per (tile, split)
    int* cnt;                   // S > 1: per-tile arrival counters (zero between launches)
    uint32_t ws_bytes;          // S > 1: bytes of ws
    int fenced;                 // S > 1: ws is cached memory: release / acquire around the exchange
};

// Pipeline of depth P (1 or 3): x is DMA'd P steps ahead into P + 1 LDS stages, weight units are loaded into P + 1
// register buffers P + 1 steps ahead, and the unit of step l + 1 is dequantized into one of 2 LDS weight stages during
// step l. With split-K (S > 1) the blocks of one tile each run a contiguous range of K steps; each writes its float32
// partial tile to the workspace, and the block that arrives last (an atomic counter per tile, reset by that block)
// adds the S partials in split order, so the result does not depend on which block finishes last. The workspace is
// uncached device memory (no fence needed), or the static scratch of mbq_matmul_noalloc, where the exchange releases
// and acquires at agent scope.
template <int T, int BM, int BN, int P, bool KFULL>
__global__ __launch_bounds__(GT, (BM == 64 && BN <= 192) ? 4 : 2) void gemm_kernel(const GemmArgs g) {
    extern __shared__ __attribute__((aligned(16))) uint16_t gemm_lds[];   // [A stage 0 .. P][B stage 0][B stage 1]
    constexpr int NA = P + 1;
    constexpr int BROWS = b_rows(BN);                   // weight stage rows (a 192-row tile adds 16 private rows)
    uint16_t* const B0 = gemm_lds + NA * BM * GK;
    constexpr int TI = BM / 32, TJ = BN / 64;           // MFMA tiles per wave
    constexpr int XD = BM / 64;                         // x DMA instructions per wave per step (8 rows each)
    constexpr int NB = b_loads<T>();
    static_assert(P == 1 || P == 3, "the weight stage of a step must follow from its register buffer");
    const int M = g.M, N = g.N, K = g.K;

    // XCD-aware order: block b runs on XCD b % 8; XCD x takes a contiguous range of (tile, split) items, splits
    // fastest, then tiles N fastest, so the blocks running at once on one XCD share one x row-panel in its L2
    const int MT = (M + BM - 1) / BM, NT = (N + BN - 1) / BN, TB = MT * NT * g.S;
    const int b = blockIdx.x, xcd = b & 7, q = TB >> 3, rem = TB & 7;
    const int item = xcd * q + min(xcd, rem) + (b >> 3);
    const int tile = item / g.S, kz = item - tile * g.S;
    const int m0 = (tile / NT) * BM, n0 = (tile % NT) * BN;

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wm = wave >> 2, wn = wave & 3;
    const int64_t lo = layer_offset(g.stride, g.layer_dev, g.nlayers);
    const bool ok = lo >= 0;
    const uint8_t* base = g.base + (ok ? lo : 0);
    const rsrc_t wr = make_rsrc(base, (uint32_t)g.wbytes);
    const rsrc_t xr = make_rsrc(g.x, (uint32_t)((int64_t)M * K * 2));

    // this block's K steps [ks0, ks0 + n)
    const int KT = (K + GK - 1) / GK;
    const int ks0 = kz * g.kts, n = ok ? min(KT - ks0, g.kts) : 0;
    auto k0 = [&](int l) { return (ks0 + min(l, n - 1)) * GK; };      // K offset of local step l (clamped)

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
    auto dma_x = [&](int s, int kk) {
#pragma unroll
        for (int i = 0; i < XD; ++i) {
            uint32_t v = xvo[i];
            if constexpr (!KFULL) v = (kk + xk[i] < K) ? v : OOB_VOFF;     // past K: out of range, reads zero
            dma16(xr, gemm_lds + s * BM * GK + 8 * (wave + 8 * i) * GK, v, (uint32_t)kk * 2);
        }
    };

    // Dequant work: the tile's 2 BN weight units (row br, unit bu; rows clamped to N - 1, since rows past N only feed
    // outputs that are never stored), LPU threads per unit, each dequantizing CPT of its 4 chunks. A tile of 192 rows
    // has 384 units for 512 threads: the last 128 threads repeat a unit and store it to private rows past the tile, so
    // every step stays free of branches and no two lanes store to one LDS address.
    constexpr int LPU = (GT % (2 * BN) == 0) ? GT / (2 * BN) : 1, CPT = 4 / LPU, OWN = 2 * BN * LPU;
    const int unit = min(tid / LPU, 2 * BN - 1), br = unit >> 1, bu = unit & 1, t0 = (tid % LPU) * CPT;
    const BOff bo = b_off<T>(g.sc_off, g.hi_off, g.d_off, min(n0 + br, N - 1), K, bu);
    int boff[CPT];                                       // LDS element offset of each of this thread's chunks
#pragma unroll
    for (int c = 0; c < CPT; ++c) {
        const int d = tid - OWN;
        boff[c] = (OWN >= GT || d < 0) ? br * GK + (((4 * bu + t0 + c) ^ (br & 7)) << 3) : (BN + d / 8) * GK + ((d % 8) << 3);
    }
    auto put_chunk = [&](uint16_t* Bst, const BUnit<T>& u, const BScale& sc, int c) {
        st16(Bst + boff[c], b_chunk<T>(u, sc, t0 + c));
    };

    f32x4_t acc[TI][TJ];
#pragma unroll
    for (int i = 0; i < TI; ++i)
#pragma unroll
        for (int j = 0; j < TJ; ++j) acc[i][j] = f32x4_t{0.f, 0.f, 0.f, 0.f};

    BUnit<T> R[NA];

    // local step l (l % NA == U): MFMAs on A stage U and B stage U & 1; x of step l + P streams into A stage
    // (U + P) % NA, the unit of step l + 1 (register buffer U + 1) is dequantized into B stage (U + 1) & 1 between the
    // MFMAs, and buffer U (dequantized a step ago) is refilled with the unit of step l + P + 1. J < 0: a step of the
    // unrolled loop. J >= 0: step J of the last n % NA, whose x and weights would be for steps past n, so it issues no
    // DMA and no loads (loads nobody reads are dropped by the compiler, and the wait must count what is issued).
    auto step = [&](auto U_, auto J_, int l) {
        constexpr int U = decltype(U_)::value;
        constexpr int J = decltype(J_)::value;
        if constexpr (J < 0) {
            dma_x((U + P) % NA, k0(l + P));
            __builtin_amdgcn_sched_barrier(0);         // the DMA stays ahead of the weight loads (vmcnt order below)
            b_load<T, KFULL>(R[U], wr, bo, K, k0(l + P + 1), bu);
        }
        const BUnit<T>& dq = R[(U + 1) % NA];
        const uint16_t* Ac = gemm_lds + U * BM * GK;
        const uint16_t* Bc = B0 + (U & 1) * BROWS * GK;
        uint16_t* Bn = B0 + ((U + 1) & 1) * BROWS * GK;
        const BScale sc = b_scale<T>(dq, ((k0(l + 1) >> 5) + bu) & 7);
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
                if (i % EVERY == EVERY - 1 && ks * 2 + i / EVERY < CPT) put_chunk(Bn, dq, sc, ks * 2 + i / EVERY);
            }
        }
        // the x DMA of step l + 1 (issued P steps ago) has landed once at most the loads issued after it are in flight:
        // its own step's NB weight loads and P - 1 later steps' XD + NB. In tail step J those later steps are the
        // P - 2 - J loop steps before the tail (the tail issues nothing); in the last one no later step reads x.
        constexpr int VM = J < 0 ? NB + (P - 1) * (XD + NB) : J <= P - 2 ? NB + (P - 2 - J) * (XD + NB) : 0;
        wait_vm<VM>();
        __syncthreads();
    };

    if (n > 0) {
#pragma unroll
        for (int p = 0; p < P; ++p) dma_x(p, k0(p));
#pragma unroll
        for (int r = 0; r < NA; ++r) b_load<T, KFULL>(R[r], wr, bo, K, k0(r), bu);
        const BScale sc = b_scale<T>(R[0], ((k0(0) >> 5) + bu) & 7);
#pragma unroll
        for (int c = 0; c < CPT; ++c) put_chunk(B0, R[0], sc, c);
        __builtin_amdgcn_s_waitcnt(0x0F70);              // vmcnt(0): the first x tiles have landed
    }
    __syncthreads();
    // the NA steps of a round are unconditional, so that no load is sunk into a conditional block (its latency must
    // overlap the steps before its use); the last n % NA steps run one by one
    using I0 = std::integral_constant<int, 0>;
    using I1 = std::integral_constant<int, 1>;
    using I2 = std::integral_constant<int, 2>;
    using I3 = std::integral_constant<int, 3>;
    using LOOP = std::integral_constant<int, -1>;
    int l = 0;
    for (; l + NA <= n; l += NA) {
        step(I0{}, LOOP{}, l);
        step(I1{}, LOOP{}, l + 1);
        if constexpr (NA == 4) {
            step(I2{}, LOOP{}, l + 2);
            step(I3{}, LOOP{}, l + 3);
        }
    }
    if (l < n) step(I0{}, I0{}, l);
    if constexpr (NA == 4) {
        if (l + 1 < n) step(I1{}, I1{}, l + 1);
        if (l + 2 < n) step(I2{}, I2{}, l + 2);
    }

    // epilogue: lane holds column n = lane & 15 and rows 4 * (lane >> 4) + r of each 16 x 16 tile
    if (g.S > 1) {
        // this split's partial tile, in the lanes' own layout, stored and read with sc1 (device-coherent) buffer
        // accesses: written through the XCD's L2, so the block that arrives last reads every split's partial without an
        // L2-wide fence (__threadfence writes back and invalidates the whole L2 on gfx950)
        const rsrc_t pr = make_rsrc(g.ws, g.ws_bytes);
        constexpr uint32_t E = (uint32_t)BM * BN * 4u;                  // bytes of one partial tile
        const uint32_t lofs = (uint32_t)((wave * TI * TJ) * 64 + lane) * 16u;
#pragma unroll
        for (int i = 0; i < TI; ++i)
#pragma unroll
            for (int j = 0; j < TJ; ++j)
                __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, acc[i][j]), pr, lofs + (uint32_t)((i * TJ + j) * 64) * 16u,
                                                       (uint32_t)(tile * g.S + kz) * E, 16);
        if (g.fenced) split_release();                                // the partial is visible at agent scope
        else wait_vm<0>();
        __syncthreads();
        int* flag = reinterpret_cast<int*>(gemm_lds);
        if (tid == 0) {
            const int old = __hip_atomic_fetch_add(g.cnt + tile, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            *flag = old == g.S - 1;
            if (old == g.S - 1) __hip_atomic_store(g.cnt + tile, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);   // ready for the next launch
        }
        __syncthreads();
        if (!*flag) return;
        if (g.fenced) split_acquire();                                // the other blocks' partials, not stale lines
        const uint32_t first = (uint32_t)(tile * g.S) * E;
        for (int z = 0; z < g.S; ++z) {                               // split order: the same sum whoever is last
#pragma unroll
            for (int i = 0; i < TI; ++i)
#pragma unroll
                for (int j = 0; j < TJ; ++j) {
                    const f32x4_t v = __builtin_bit_cast(f32x4_t, __builtin_amdgcn_raw_buffer_load_b128(
                                          pr, lofs + (uint32_t)((i * TJ + j) * 64) * 16u, first + (uint32_t)z * E, 16));
                    acc[i][j] = z == 0 ? v : acc[i][j] + v;
                }
        }
    }
    // every scale is loaded before the first store: a scale load between stores would make each store wait for the ones
    // before it (vmcnt counts stores)
    float sc[TJ];
#pragma unroll
    for (int j = 0; j < TJ; ++j) {
        const int nn = n0 + wn * (BN / 4) + j * 16 + (lane & 15);
        sc[j] = nn < N ? row_scale<T>(g.srow, base, g.sc_off, nn) : 0.f;
    }
#pragma unroll
    for (int j = 0; j < TJ; ++j) {
        const int nn = n0 + wn * (BN / 4) + j * 16 + (lane & 15);
        if (nn >= N) continue;
        const float s = sc[j];
#pragma unroll
        for (int i = 0; i < TI; ++i)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int m = m0 + wm * (BM / 2) + i * 16 + (lane >> 4) * 4 + r;
                if (m < M) store_y(g.y, (int64_t)m * N + nn, ok ? acc[i][j][r] * s : __builtin_nanf(""), g.out_bf16);
            }
    }
}

// ----------------------------------------------------------------------------------------- specialized waves
// Block tile 256 x 192 with specialized waves. On gfx950 a wave's VALU instructions do not overlap its own MFMAs, but
// another wave's VALU instructions issue while the matrix core runs. So waves 0-3 (one per SIMD) only multiply: each
// owns a 128 x 96 quarter of the tile as 4 x 3 tiles of v_mfma_f32_32x32x16_bf16 (accumulators pinned by mfma32_acc /
// mfma32_accv: 128 accumulation registers and 64 vector registers, the even split of 256 at two waves per SIMD; the
// 32 x 32 shape needs half the operand registers of 16 x 16 per K, so a whole K substep is read ahead) and reads its
// A and B operands from LDS. Waves 4-7 (the other wave of each SIMD) only produce: x tiles by DMA into a ring of 3 LDS stages (issued
// two steps ahead), weight units from HBM into a ring of 3 register sets (three steps ahead), dequantized into a ring of
// 2 bf16 LDS stages one step ahead. One barrier per step: the step-l barrier says stage l is complete, and that the
// stages of step l - 1 are no longer read.
//
// Step l, producers (after barrier l): DMA x(l + 2) into A stage (l + 2) % 3 (spread between the next item's chunks),
// load weights (l + 3), dequantize weights (l + 1) into B stage (l + 1) % 2, wait for x(l + 1), barrier l + 1. Consumers: barrier l, then the 48 MFMAs of step l
// from A stage l % 3 and B stage l % 2, each K substep's operands read during the one before. Both roles pass n
// barriers in the same order, and one more before bfloat16 outputs leave through LDS (the consumers' epilogue).
constexpr int SG_BM = 256, SG_BN = 192;
// element offset of chunk c of row r in the specialized kernel's LDS tiles: rows of 64 bfloat16 (128 bytes, half of the
// 64 four-byte banks), chunk c at c ^ ((r >> 1) & 7). A 32-lane pass of its operand reads (32 rows, one chunk) and of
// its dequantized-weight writes (16 rows, two chunks each) then covers every bank twice, the least 512 bytes can; under
// c ^ (r & 7) rows r and r + 8 shared banks (SQ_LDS_BANK_CONFLICT measured 3.3 cycles per LDS instruction).
__device__ __forceinline__ int sg_off(int r, int c) { return r * GK + ((c ^ ((r >> 1) & 7)) << 3); }
constexpr size_t SG_LDS = (size_t)(3 * SG_BM + 2 * SG_BN) * GK * sizeof(uint16_t);   // 144 KiB
// row stride (elements) of a consumer wave's output quarter in LDS: 96 values and 8 of padding, so that the two rows a
// two-byte write covers (4 apart) fall on different banks; 4 quarters of 128 rows take 104 KiB
constexpr int SG_QS = 104;
static_assert((size_t)4 * 128 * SG_QS * sizeof(uint16_t) <= SG_LDS && SG_QS % 8 == 0, "output quarters fit the LDS");

template <int T, bool KFULL>
__global__ __launch_bounds__(GT, 1) void sgemm_kernel(const GemmArgs g) {
    extern __shared__ __attribute__((aligned(16))) uint16_t sg_lds[];   // A[3][256][64], B[2][192][64] bfloat16
    uint16_t* const A0 = sg_lds;
    uint16_t* const B0 = sg_lds + 3 * SG_BM * GK;
    const int M = g.M, N = g.N, K = g.K;

    // XCD-aware order, as gemm_kernel
    const int MT = (M + SG_BM - 1) / SG_BM, NT = (N + SG_BN - 1) / SG_BN, TB = MT * NT;
    const int b = blockIdx.x, xcd = b & 7, q = TB >> 3, rem = TB & 7;
    const int tile = xcd * q + min(xcd, rem) + (b >> 3);
    const int m0 = (tile / NT) * SG_BM, n0 = (tile % NT) * SG_BN;
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int64_t lo = layer_offset(g.stride, g.layer_dev, g.nlayers);
    const bool ok = lo >= 0;
    const int KT = (K + GK - 1) / GK, n = ok ? KT : 0;
    auto k0 = [&](int l) { return min(l, n - 1) * GK; };
    auto fence = [] { __builtin_amdgcn_sched_barrier(0); };
    // bfloat16 output rows whose 8-value chunks are 16-byte aligned leave through LDS (the consumers' epilogue)
    const bool vec = g.out_bf16 && (N & 7) == 0 && (reinterpret_cast<uintptr_t>(g.y) & 15) == 0;

    if (wave < 4) {
        // ---------------------------------------------------------------------------------------------- consumer
        // 4 x 3 tiles of v_mfma_f32_32x32x16_bf16; a K step is 4 substeps of 16 values, and the 7 operands of substep
        // s + 1 (4 A row tiles, 3 B column tiles) are read while the 12 MFMAs of substep s run
        const int cm = wave >> 1, cn = wave & 1;
        f32x16_t acc[4][3];
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int j = 0; j < 3; ++j) acc[i][j] = f32x16_t{};
        const int ar = cm * 128 + (lane & 31), br = cn * 96 + (lane & 31), lh = lane >> 5;
        for (int l = 0; l < n; ++l) {
            barrier_nofence();                                     // stage l is complete
            fence();
            const uint16_t* As = A0 + (l % 3) * SG_BM * GK;
            const uint16_t* Bs = B0 + (l & 1) * SG_BN * GK;
            // operand o of substep s: o < 4 A row tile o, else B column tile o - 4; chunk 2 s + (lane >> 5)
            auto rd = [&](int s, int o) {
                const uint16_t* base = o < 4 ? As + sg_off(ar + 32 * o, 2 * s + lh) : Bs + sg_off(br + 32 * (o - 4), 2 * s + lh);
                return *reinterpret_cast<const bf16x8_t*>(base);
            };
            bf16x8_t op[2][7];
#pragma unroll
            for (int o = 0; o < 7; ++o) op[0][o] = rd(0, o);
            fence();
#pragma unroll
            for (int s = 0; s < 4; ++s) {
#pragma unroll
                for (int i = 0; i < 4; ++i)
#pragma unroll
                    for (int j = 0; j < 3; ++j) {
                        const int k = 3 * i + j;
                        if (s + 1 < 4 && k < 7) op[(s + 1) & 1][k] = rd(s + 1, k);
                        // 128 of the 192 accumulator registers fit the accumulation registers at two waves per SIMD
                        if (j < 2) mfma32_acc(acc[i][j], op[s & 1][i], op[s & 1][4 + j]);
                        else mfma32_accv(acc[i][j], op[s & 1][i], op[s & 1][4 + j]);
                        fence();
                    }
            }
            // the compiler may copy accumulators at the loop's back edge or exit (the join with the path that skips the
            // loop): no such copy may follow an MFMA that is still writing
            mfma_drain();
        }
        // lane holds weight row n0 + 96 cn + 32 j + (lane & 31) and activation rows m0 + 128 cm + 32 i + 8 e + 4 (lane >> 5) + r
        float scs[3];
#pragma unroll
        for (int j = 0; j < 3; ++j) {
            const int nn = n0 + br + 32 * j;
            scs[j] = nn < N ? row_scale<T>(g.srow, g.base + (ok ? lo : 0), g.sc_off, nn) : 0.f;
        }
        if (vec) {
            // The wave's 128 x 96 quarter goes to a region of LDS of its own as bfloat16 rows, and from there to y in
            // 16-byte chunks: 24 coalesced stores per lane instead of 192 two-byte ones (measured on MI355X: the
            // two-byte stores kept a tile's waves busy for about a sixth of its time). The barrier pairs with the
            // producers' last one: no stage is read any more and every DMA has landed.
            barrier_nofence();
            uint16_t* const stg = sg_lds + wave * (128 * SG_QS);
#pragma unroll
            for (int j = 0; j < 3; ++j)
#pragma unroll
                for (int i = 0; i < 4; ++i)
#pragma unroll
                    for (int e = 0; e < 4; ++e)
#pragma unroll
                        for (int r = 0; r < 4; ++r)
                            stg[(32 * i + 8 * e + 4 * lh + r) * SG_QS + 32 * j + (lane & 31)] =
                                (uint16_t)bf16_bits(ok ? acc[i][j][4 * e + r] * scs[j] : __builtin_nanf(""));
            asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");         // the wave reads back what its lanes wrote
            uint16_t* const y = reinterpret_cast<uint16_t*>(g.y);
#pragma unroll
            for (int t = 0; t < 128 * 12 / 64; ++t) {                  // chunk q: row q / 12, 8 values from 8 (q % 12)
                const int qd = 64 * t + lane, row = qd / 12, c = qd - 12 * row;
                const int m = m0 + cm * 128 + row, nn = n0 + cn * 96 + 8 * c;
                const u32x4 v = *reinterpret_cast<const u32x4*>(stg + row * SG_QS + 8 * c);
                if (m < M && nn < N) *reinterpret_cast<u32x4*>(y + (int64_t)m * N + nn) = v;   // N % 8 == 0: whole chunks
            }
            return;
        }
#pragma unroll
        for (int j = 0; j < 3; ++j) {
            const int nn = n0 + br + 32 * j;
            if (nn >= N) continue;
            const float sc = scs[j];
#pragma unroll
            for (int i = 0; i < 4; ++i)
#pragma unroll
                for (int e = 0; e < 4; ++e)
#pragma unroll
                    for (int r = 0; r < 4; ++r) {
                        const int m = m0 + cm * 128 + 32 * i + 8 * e + 4 * lh + r;
                        if (m < M) store_y(g.y, (int64_t)m * N + nn, ok ? acc[i][j][4 * e + r] * sc : __builtin_nanf(""), g.out_bf16);
                    }
        }
        return;
    }

    // -------------------------------------------------------------------------------------------------- producer
    const int pt = tid - 4 * 64, pw = wave - 4;                     // producer thread 0..255, producer wave 0..3
    const uint8_t* base = g.base + (ok ? lo : 0);
    const rsrc_t wr = make_rsrc(base, (uint32_t)g.wbytes);
    const rsrc_t xr = make_rsrc(g.x, (uint32_t)((int64_t)M * K * 2));
    // x DMA: instruction i of producer wave w fills tile rows 8 (w + 4 i) .. +7 (8 instructions x 4 waves x 8 rows);
    // lane l writes LDS slot l & 7 of row l >> 3, holding chunk (l & 7) ^ ((row >> 1) & 7) (the swizzle of sg_off)
    constexpr int XD = SG_BM * GK * 2 / (4 * 64 * 16);              // 8
    static_assert(XD == 8, "the producer step spreads its 8 DMA instructions among its 6 or 8 dequantized chunks");
    uint32_t xvo[XD];
    int xk[XD];
#pragma unroll
    for (int i = 0; i < XD; ++i) {
        const int r = 8 * (pw + 4 * i) + (lane >> 3), c = (lane & 7) ^ ((r >> 1) & 7);
        xvo[i] = m0 + r < M ? (uint32_t)(((int64_t)(m0 + r) * K + c * 8) * 2) : OOB_VOFF;     // rows past M: zero
        xk[i] = c * 8;
    }
    auto dma_x = [&](int l) {                                        // x of step l into A stage l % 3
        const int kk = k0(l);
        uint16_t* st = A0 + (l % 3) * SG_BM * GK;
#pragma unroll
        for (int i = 0; i < XD; ++i) {
            uint32_t v = xvo[i];
            if constexpr (!KFULL) v = (kk + xk[i] < K) ? v : OOB_VOFF;      // past K: zero
            dma16(xr, st + 8 * (pw + 4 * i) * GK, v, (uint32_t)kk * 2);
        }
    };
    // Weight units of a step: 2 per row (32 values each) = 384 (row u >> 1, unit u & 1 of the step), 3 per pair of
    // producer threads. Thread 2p dequantizes unit 3p whole and chunks 0-1 of unit 3p + 2, thread 2p + 1 unit 3p + 1
    // whole and chunks 2-3 of unit 3p + 2: 6 chunks of 8 values per thread, so the four producer waves share the work
    // evenly (with units 0-255 whole and 128 second units on two of the waves, those two set the step: measured on
    // MI355X, the other two waited ≈ 700 of ≈ 2,300 cycles per step at the barrier). Both threads of a pair load the
    // shared unit whole (the same bytes). Q6_K units take 8 registers each and the even split spills there, so Q6_K
    // keeps that uneven one: thread t takes unit t whole and, for t < 128, unit t + 256. Rows past N are clamped
    // (their outputs are never stored).
    constexpr bool EVEN = !q6k_like(T);
    constexpr int UPT = 2;                                          // the thread's whole unit, then the shared (second) one
    constexpr int NCH = EVEN ? 6 : 8;                               // chunks of 8 values per thread and step
    const int ph = pt & 1;                                          // EVEN: which half of the shared unit
    const bool two = EVEN || pt < 2 * SG_BN - 256;                  // uneven: the threads with a second unit
    BOff bo[UPT];
    int bu[UPT], brow[UPT];
#pragma unroll
    for (int v = 0; v < UPT; ++v) {
        const int u = EVEN ? 3 * (pt >> 1) + (v == 0 ? ph : 2) : pt + 256 * v;
        brow[v] = u >> 1;
        bu[v] = u & 1;
        bo[v] = b_off<T>(g.sc_off, g.hi_off, g.d_off, min(n0 + brow[v], N - 1), K, bu[v]);
    }
    if (!two) bo[1] = BOff{OOB_VOFF, OOB_VOFF, OOB_VOFF, OOB_VOFF};   // no second unit: its loads read zero, no traffic
    // chunk i of the thread: chunks 0-3 of its whole unit, then (EVEN) chunks 2 ph and 2 ph + 1 of the shared one or
    // (uneven) chunks 0-3 of the second unit, which only threads with `two` have (wave-uniform)
    auto chunk_v = [](int i) { return i < 4 ? 0 : 1; };
    auto chunk_c = [&](int i) { return i < 4 ? i : EVEN ? 2 * ph + (i - 4) : i - 4; };
    BUnit<T> R[3][UPT];
    auto load_w = [&](BUnit<T>* Rr, int l) {
#pragma unroll
        for (int v = 0; v < UPT; ++v) b_load<T, KFULL>(Rr[v], wr, bo[v], K, k0(l), bu[v]);
    };
    auto dequant = [&](const BUnit<T>* Rr, int l) {                   // weights of step l into B stage l % 2
        uint16_t* st = B0 + (l & 1) * SG_BN * GK;
        BScale sc[UPT];
#pragma unroll
        for (int v = 0; v < UPT; ++v) sc[v] = b_scale<T>(Rr[v], ((k0(l) >> 5) + bu[v]) & 7);
#pragma unroll
        for (int i = 0; i < NCH; ++i) {
            const int v = chunk_v(i), c = chunk_c(i);
            if (v == 0 || two) st16(st + sg_off(brow[v], 4 * bu[v] + c), b_chunk<T>(Rr[v], sc[v], c));
        }
    };
    constexpr int NDW = XD, NWL = UPT * b_loads<T>();
    if (n > 0) {
        dma_x(0);
        dma_x(1);
        load_w(R[0], 0);
        load_w(R[1], 1);
        load_w(R[2], 2);
        dequant(R[0], 0);
        // x(0) has landed: only x(1)'s DMA is certain to follow it, since the three weight sets may share loads the
        // compiler merges (a K-quant's scale block is the same for the steps of one 256-value superblock)
        wait_vm<NDW>();
        wait_lgkm0();                                                 // and the dequantized weights of step 0
        barrier_nofence();                                            // barrier 0
        // step l (l = 0 .. n - 2): x(l + 2), weights (l + 3), dequantize (l + 1), wait x(l + 1), barrier l + 1. The x
        // DMA's 8 instructions are spread between the dequantized chunks (a burst of them slows the consumers' reads).
        // The wait counts the vector-memory instructions the step itself issues, so it must match them exactly: the
        // last one or two steps (after the unrolled loop) load no weights, because no later step dequantizes them. They
        // say so (W false) rather than leave the loads for the compiler to drop, which would leave the wait 4 too high
        // and let the consumers read the tail of x(l + 1) before its DMA landed.
        auto pstep = [&](auto U_, auto W_, int l) {
            constexpr int U = decltype(U_)::value;                    // l % 3
            constexpr bool W = decltype(W_)::value;                   // the step loads the weights of step l + 3
            const int kk = k0(l + 2);
            uint16_t* ast = A0 + ((l + 2) % 3) * SG_BM * GK;
            auto dma_i = [&](int i) {
                uint32_t v = xvo[i];
                if constexpr (!KFULL) v = (kk + xk[i] < K) ? v : OOB_VOFF;
                dma16(xr, ast + 8 * (pw + 4 * i) * GK, v, (uint32_t)kk * 2);
            };
            const BUnit<T>* Rr = R[(U + 1) % 3];                      // weights of step l + 1
            uint16_t* bst = B0 + ((l + 1) & 1) * SG_BN * GK;
            BScale sc[UPT];
#pragma unroll
            for (int v = 0; v < UPT; ++v) sc[v] = b_scale<T>(Rr[v], ((k0(l + 1) >> 5) + bu[v]) & 7);
            dma_i(0);
            if constexpr (W) load_w(R[U], l + 3);                     // the set of step l, dequantized a step ago
#pragma unroll
            for (int i = 0; i < XD; ++i) {
                if (i > 0) dma_i(i);
                if (i < NCH) {
                    const int v = chunk_v(i), c = chunk_c(i);
                    if (v == 0 || two) st16(bst + sg_off(brow[v], 4 * bu[v] + c), b_chunk<T>(Rr[v], sc[v], c));
                }
            }
            wait_vm<NDW + (W ? NWL : 0)>();                           // x(l + 1) has landed (loads complete in order)
            wait_lgkm0();                                             // and the dequantized weights of step l + 1
            barrier_nofence();
        };
        using I0 = std::integral_constant<int, 0>;
        using I1 = std::integral_constant<int, 1>;
        using I2 = std::integral_constant<int, 2>;
        using LOAD = std::true_type;
        using TAIL = std::false_type;
        int l = 0;
        for (; l + 3 <= n - 1; l += 3) {
            pstep(I0{}, LOAD{}, l);
            pstep(I1{}, LOAD{}, l + 1);
            pstep(I2{}, LOAD{}, l + 2);
        }
        if (l < n - 1) pstep(I0{}, TAIL{}, l);                        // steps l + 2 and l + 3 do not exist
        if (l + 1 < n - 1) pstep(I1{}, TAIL{}, l + 1);
        wait_vm<0>();                                                 // no DMA may land after the block ends
    }
    if (vec) barrier_nofence();                                       // the consumers may now write the output tile into LDS
}

// ------------------------------------------------------------------------------------------------- workspace
// Split-K partials and arrival counters: one set per (device, stream), so that split-K calls overlapping in time on two
// streams of a device (a server's prefill and decode streams) never share partials or counters. A stream's set is
// allocated (its counters cleared) by the first split-K call made on it eagerly, and kept until the process ends.
//
// An allocation cannot be recorded into a HIP graph, so each eager split-K call also makes sure the device holds one
// spare set: the first split-K call recorded on a stream that has no set of its own (torch.cuda.graph records on a side
// stream) takes the spare, which is then that stream's for good. A call under capture that finds neither (no eager
// split-K call yet on the device, or the spare taken by another capturing stream since the last eager call) is refused
// with an error and launches nothing. Graphs recorded on one stream share its set: replays of two such graphs must not
// overlap in time. A destroyed stream's set is kept (a later stream at the same handle reuses it).
constexpr int WS_MAX_STREAMS = 32;            // sets per device (each WS_BYTES + WS_TILES counters), spare included

static int ws_alloc(Workspace* w, int dev) {
    // Uncached device memory: no L2 holds its lines, so a partial one XCD stores is what another XCD loads after the
    // arrival count, with no cache write-back or invalidation between (the exchange of every split-K kernel). Never
    // freed, also on a failed set-up.
    void *p = nullptr, *c = nullptr;
    if (hipExtMallocWithFlags(&p, WS_BYTES, hipDeviceMallocUncached) != hipSuccess)
        return set_error(MBQ_LAUNCH_FAIL, "GEMM: split-K workspace allocation on device %d failed", dev);
    // the counters are zeroed on the null stream and waited for here, once: the first kernel that uses them may run on
    // a non-blocking stream, which does not wait for the null stream
    if (hipExtMallocWithFlags(&c, WS_TILES * sizeof(int), hipDeviceMallocUncached) != hipSuccess ||
        hipMemset(c, 0, WS_TILES * sizeof(int)) != hipSuccess || hipStreamSynchronize(nullptr) != hipSuccess)
        return set_error(MBQ_LAUNCH_FAIL, "GEMM: split-K counter allocation on device %d failed", dev);
    w->ws = static_cast<float*>(p);
    w->cnt = static_cast<int*>(c);
    w->bytes = WS_BYTES;
    w->tiles = WS_TILES;
    w->fenced = 0;
    return 0;
}

int workspace(Workspace* out, hipStream_t s) {
    struct Dev { hipStream_t stream[WS_MAX_STREAMS]; Workspace set[WS_MAX_STREAMS]; int n = 0; Workspace spare; };
    static Dev per_dev[64];
    static std::mutex mu;
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return set_error(MBQ_LAUNCH_FAIL, "GEMM: no device");
    std::lock_guard<std::mutex> lk(mu);
    Dev& d = per_dev[dev];
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    const bool capturing = hipStreamIsCapturing(s, &cs) == hipSuccess && cs != hipStreamCaptureStatusNone;
    // sets held: d.n streams' and the spare, at most WS_MAX_STREAMS; the spare is refilled by eager calls (best effort:
    // a failed refill only means that a later first capture on a new stream is refused)
    auto refill = [&] { if (!capturing && !d.spare.ws && d.n < WS_MAX_STREAMS) ws_alloc(&d.spare, dev); };
    for (int i = 0; i < d.n; ++i)
        if (d.stream[i] == s) {
            *out = d.set[i];
            refill();
            return 0;
        }
    if (!capturing && d.n + (d.spare.ws ? 1 : 0) >= WS_MAX_STREAMS)
        return set_error(MBQ_BAD_ARG, "GEMM: split-K calls on more than %d streams of device %d (one workspace each)",
                         WS_MAX_STREAMS - 1, dev);
    Workspace w;
    if (capturing) {
        if (!d.spare.ws)
            return set_error(MBQ_BAD_ARG, "GEMM: the first split-K call on this stream of device %d needs a workspace, "
                                          "which a stream being captured into a graph cannot allocate: make one eager "
                                          "call first", dev);
        w = d.spare;
        d.spare = Workspace{};
    } else {
        if (int rc = ws_alloc(&w, dev)) return rc;
    }
    d.stream[d.n] = s;
    d.set[d.n] = w;
    ++d.n;
    refill();
    *out = w;
    return 0;
}

// --------------------------------------------------------------------------------------------------- scratch
// The split-K partials and arrival counters of mbq_matmul_noalloc, for callers that cannot allocate (code under HIP
// graph capture, serving loops, harnesses that forbid hipMalloc): one static device array, which every GPU the library
// runs on holds at its own address until the process ends. Its SCRATCH_BYTES of partial tiles (the allocated
// workspace's size) cover every automatic split plan: the planners keep each plan's partials within it, so both entry
// points run the same plan and give the same bits; a forced plan that needs more is refused. In host code the name
// `scratch` is not a device address: the address is taken once per device with hipGetSymbolAddress and used from then
// on.
static __device__ __align__(256) uint8_t scratch[SCRATCH_BYTES + SCRATCH_TILES * sizeof(int)];

// the scratch's device address on the current device, set up once per device: the address from hipGetSymbolAddress
// (the current device's copy of the array), and the arrival counters cleared by a fill kernel on the caller's stream
// (they must start at zero; each split-K launch leaves the counters it used at zero)
static int scratch_workspace(hipStream_t s, Workspace* out) {
    static void* addr[64] = {};
    static std::mutex mu;
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return set_error(MBQ_LAUNCH_FAIL, "GEMM: no device");
    std::lock_guard<std::mutex> lk(mu);
    if (!addr[dev]) {
        void* p = nullptr;
        const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess || p == nullptr)
            return set_error(MBQ_LAUNCH_FAIL, "GEMM: the scratch array's address on device %d: %s", dev, hipGetErrorString(e));
        if (int rc = launch_zero(static_cast<uint8_t*>(p) + SCRATCH_BYTES, (int64_t)SCRATCH_TILES * sizeof(int), s)) return rc;
        addr[dev] = p;
    }
    out->ws = static_cast<float*>(addr[dev]);
    out->cnt = reinterpret_cast<int*>(static_cast<uint8_t*>(addr[dev]) + SCRATCH_BYTES);
    out->bytes = SCRATCH_BYTES;
    out->tiles = SCRATCH_TILES;
    out->fenced = 1;
    return 0;
}

int split_workspace(const Args& a, int64_t tiles, size_t bytes, hipStream_t s, Workspace* out) {
    const size_t cap = a.noalloc ? SCRATCH_BYTES : WS_BYTES;
    const int ntiles = a.noalloc ? SCRATCH_TILES : WS_TILES;
    if (tiles > ntiles || bytes > cap)                                // checked before any set-up: nothing launches
        return set_error(MBQ_BAD_ARG, "GEMM: a split-K plan of %lld tiles and %zu partial bytes exceeds the %s (%d tiles, %zu bytes)",
                         (long long)tiles, bytes, a.noalloc ? "scratch of mbq_matmul_noalloc" : "workspace", ntiles, cap);
    return a.noalloc ? scratch_workspace(s, out) : workspace(out, s);
}

// ------------------------------------------------------------------------------------------------- launchers
template <int T, int BM, int BN, int P>
static size_t lds_bytes() { return (size_t)((P + 1) * BM * GK + 2 * b_rows(BN) * GK) * sizeof(uint16_t); }

template <int T, int BM, int BN, int P, bool KFULL>
static int launch_tile(const Args& a, int S, int kts, const Workspace& w, hipStream_t s) {
    auto kern = gemm_kernel<T, BM, BN, P, KFULL>;
    const size_t lds = lds_bytes<T, BM, BN, P>();
    static std::atomic<uint64_t> lds_set{0};
    if (set_lds_limit((const void*)kern, lds, lds_set) != hipSuccess)
        return set_error(MBQ_LAUNCH_FAIL, "GEMM: %zu bytes of LDS refused", lds);
    GemmArgs g{a.base, a.stride, a.layer_dev, a.nlayers, a.sc_off, a.wbytes, a.hi_off, a.d_off, a.srow, a.x, (int)a.M,
               (int)a.N, (int)a.K, a.y, a.out_bf16, S, kts, w.ws, w.cnt, (uint32_t)w.bytes, w.fenced};
    const int64_t tiles = ((a.M + BM - 1) / BM) * ((a.N + BN - 1) / BN);
    kern<<<dim3((unsigned)(tiles * S)), GT, lds, s>>>(g);
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return set_error(MBQ_LAUNCH_FAIL, "GEMM launch: %s", hipGetErrorString(e));
    return 0;
}

template <int T, bool KFULL>
static int launch_sg(const Args& a, hipStream_t s) {
    auto kern = sgemm_kernel<T, KFULL>;
    static std::atomic<uint64_t> lds_set{0};
    if (set_lds_limit((const void*)kern, SG_LDS, lds_set) != hipSuccess)
        return set_error(MBQ_LAUNCH_FAIL, "GEMM: %zu bytes of LDS refused", SG_LDS);
    GemmArgs g{a.base, a.stride, a.layer_dev, a.nlayers, a.sc_off, a.wbytes, a.hi_off, a.d_off, a.srow, a.x, (int)a.M,
               (int)a.N, (int)a.K, a.y, a.out_bf16, 1, (int)((a.K + GK - 1) / GK), nullptr, nullptr, 0u};
    const int64_t tiles = ((a.M + SG_BM - 1) / SG_BM) * ((a.N + SG_BN - 1) / SG_BN);
    kern<<<dim3((unsigned)tiles), GT, SG_LDS, s>>>(g);
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return set_error(MBQ_LAUNCH_FAIL, "GEMM launch: %s", hipGetErrorString(e));
    return 0;
}

// the 256 x 192 tile without a K split runs the specialized-wave kernel; K-quant rows (multiples of 256 values) always
// fill whole K steps
template <int T, int BM, int BN, int P>
static int launch_k(const Args& a, int S, int kts, const Workspace& w, hipStream_t s) {
    if constexpr (kquant(T)) {
        if (BM == SG_BM && BN == SG_BN && S == 1) return launch_sg<T, true>(a, s);
        return launch_tile<T, BM, BN, P, true>(a, S, kts, w, s);
    } else {
        if (BM == SG_BM && BN == SG_BN && S == 1) return (a.K % GK == 0) ? launch_sg<T, true>(a, s) : launch_sg<T, false>(a, s);
        return (a.K % GK == 0) ? launch_tile<T, BM, BN, P, true>(a, S, kts, w, s) : launch_tile<T, BM, BN, P, false>(a, S, kts, w, s);
    }
}

struct Plan { int idx, S, kts; };


// blocks of one tile shape resident per CU (LDS and registers), queried once per process
template <int T, int BM, int BN, int P>
static int occupancy() {
    static int v = 0;
    if (v == 0) {
        auto kern = gemm_kernel<T, BM, BN, P, true>;
        int n = 0;
        if (hipFuncSetAttribute((const void*)kern, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds_bytes<T, BM, BN, P>()) != hipSuccess ||
            hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, kern, GT, lds_bytes<T, BM, BN, P>()) != hipSuccess || n < 1)
            n = 1;
        v = n;
    }
    return v;
}

template <int T>
struct Cand {
    int bm, bn;
    int (*occ)();
    int (*launch)(const Args&, int, int, const Workspace&, hipStream_t);
};

template <int T, int BM, int BN, int P>
static constexpr Cand<T> cand() { return Cand<T>{BM, BN, occupancy<T, BM, BN, P>, launch_k<T, BM, BN, P>}; }

template <int T>
static const Cand<T> CANDS[] = {cand<T, 256, 256, 1>(), cand<T, 256, 192, 1>(), cand<T, 256, 128, 1>(),
                                cand<T, 128, 256, 1>(), cand<T, 128, 192, 1>(), cand<T, 128, 128, 3>(),
                                cand<T, 128, 64, 3>(),  cand<T, 64, 256, 3>(),  cand<T, 64, 192, 3>(),
                                cand<T, 64, 128, 3>(),  cand<T, 64, 64, 3>()};

// K-step time (us) of one block of each candidate when it runs alone on its CU (the order of CANDS; 256 x 192 without a
// split is the specialized-wave kernel)
static constexpr double T1_US[] = {1.56, 1.20, 1.14, 1.10, 1.04, 0.83, 0.57, 0.84, 0.80, 0.58, 0.43};
// Batches of more than 64 rows: the busiest CU's time. It runs ceil(blocks / CUs) blocks, `occ` at a time, each K step
// taking T1_US when a block has its CU alone and PG_G2 / PG_G3 times that when 2 / 3 blocks share it; 256 x 192 tiles
// with a split K run the plain LDS-tile kernel, PG_SGX times slower per step than the specialized one; a split adds
// PG_SA us and PG_SB us per MB of one block's partials (S bm bn float32 tiles: its own store and the last arriver's
// loads). The constants are a least-squares fit (of log time) to 1,320 timings of every candidate at 1, 2 and 4 splits
// on MI355X: Q4_K and int8 tiles, 128-2048 rows, the 17408 x 5120, 5120 x 17408, 6144 x 5120 and 1024 x 5120 weights of a
// 27B-class layer. Its choices run within 5 % of the fastest candidate on 38 of those 40 shapes (all 40 together 0.3 %
// over the fastest), where the model below (fitted to loaded CUs of one tile shape) lost 15 % (512 rows: 1.6-1.9x).
constexpr double PG_G2 = 1.44, PG_G3 = 2.11, PG_SGX = 1.18, PG_SA = 8.4, PG_SB = 22.5;

template <int T>
static Plan plan_wide(int64_t M, int64_t N, int64_t K, int cus) {
    const int64_t KT = (K + GK - 1) / GK;
    Plan best{(int)(sizeof CANDS<T> / sizeof CANDS<T>[0]) - 1, 1, (int)KT};
    double best_t = 1e300;
    for (int i = 0; i < (int)(sizeof CANDS<T> / sizeof CANDS<T>[0]); ++i) {
        const int bm = CANDS<T>[i].bm, bn = CANDS<T>[i].bn;
        if (bm > 64 && M <= bm / 2) continue;                // more than half the tile's rows would be padding
        const int64_t tiles = ((M + bm - 1) / bm) * ((N + bn - 1) / bn);
        const int occ = std::max(1, std::min(3, CANDS<T>[i].occ()));
        for (int64_t S0 : {1, 2, 3, 4}) {
            const int64_t kts = (KT + S0 - 1) / S0, S = (KT + kts - 1) / kts;     // no empty split
            if (S != S0 || (S > 1 && kts < 4)) continue;
            if (S > 1 && (tiles > std::min<int64_t>(WS_TILES, SCRATCH_TILES) ||
                          (size_t)tiles * S * bm * bn * 4 > std::min(WS_BYTES, SCRATCH_BYTES))) continue;
            const int64_t nb = (tiles * S + cus - 1) / cus;
            const double g = occ == 1 ? 1.0 : occ == 2 ? PG_G2 : PG_G3;
            const int64_t part = nb % occ;
            const double steps = (double)(nb / occ) * g + (part == 0 ? 0.0 : part == 1 ? 1.0 : PG_G2);
            double t = (double)kts * T1_US[i] * (bm == SG_BM && bn == SG_BN && S > 1 ? PG_SGX : 1.0) * steps;
            if (S > 1) t += PG_SA + PG_SB * (double)(S * bm * bn * 4) / 1e6;
            if (t < best_t) best_t = t, best = Plan{i, (int)S, (int)kts};
        }
    }
    return best;
}

// Tile shape and K split for an (M, N, K) problem: the candidate with the least modelled time. More than 64 rows:
// plan_wide. Up to 64 rows (row-major planes the weight stream does not take): a block's K step costs about 0.1 us +
// 3.5e-5 us per output of its tile (fitted to MI355X timings of these kernels at 64 activation rows); blocks run in
// rounds over the CUs x the blocks of that shape a CU holds (LDS, registers); K is split into at most 4 ranges of at
// least 4 steps, until the tiles x splits reach 128 blocks (the weight stream, not the matrix work, bounds the time).
template <int T>
static Plan plan_gemm(int64_t M, int64_t N, int64_t K, int cus) {
    if (M > 64) return plan_wide<T>(M, N, K, cus);
    const int64_t KT = (K + GK - 1) / GK;
    Plan best{(int)(sizeof CANDS<T> / sizeof CANDS<T>[0]) - 1, 1, (int)KT};
    double best_t = 1e300;
    for (int i = 0; i < (int)(sizeof CANDS<T> / sizeof CANDS<T>[0]); ++i) {
        const int bm = CANDS<T>[i].bm, bn = CANDS<T>[i].bn;
        if (bm > 64 && M <= bm / 2) continue;                // more than half the tile's rows would be padding
        if (bn != 128) continue;
        const int64_t tiles = ((M + bm - 1) / bm) * ((N + bn - 1) / bn);
        const int occ = CANDS<T>[i].occ();
        int64_t S = 1;
        if (tiles < 128 && tiles <= WS_TILES) {
            S = std::min<int64_t>({(128 + tiles - 1) / tiles, 4, std::max<int64_t>(1, KT / 4)});
            S = std::max<int64_t>(1, std::min<int64_t>(S, (int64_t)(WS_BYTES / ((size_t)tiles * bm * bn * 4))));
        }
        const int64_t kts = (KT + S - 1) / S;
        S = (KT + kts - 1) / kts;                            // no empty split
        const int64_t rounds = (tiles * S + (int64_t)cus * occ - 1) / ((int64_t)cus * occ);
        const double t = (double)rounds * occ * (0.1 + 3.46e-5 * bm * bn) * kts;
        if (t < best_t) best_t = t, best = Plan{i, (int)S, (int)kts};
    }
    // Small tiles (at most 8192 outputs) that leave CUs idle split K until about two blocks run per CU, at most 4
    // ranges of at least 4 steps (MI355X, Q4_K: 64 x 17408 x 5120 64 x 128 tiles 51 -> 38 us with 3 ranges).
    {
        const int bm = CANDS<T>[best.idx].bm, bn = CANDS<T>[best.idx].bn;
        const int64_t tiles = ((M + bm - 1) / bm) * ((N + bn - 1) / bn);
        if (bm * bn <= 8192 && tiles <= cus && tiles <= WS_TILES) {
            int64_t S = std::min<int64_t>({4, 2 * (int64_t)cus / tiles, KT / 4});
            S = std::min<int64_t>(S, (int64_t)(WS_BYTES / ((size_t)tiles * bm * bn * 4)));
            if (S >= 2) {
                const int64_t kts = (KT + S - 1) / S;
                best = Plan{best.idx, (int)((KT + kts - 1) / kts), (int)kts};
            } else {
                best = Plan{best.idx, 1, (int)KT};
            }
        }
    }
    return best;
}

// forced plan (tests, tuning): kernel, tile rows, tile columns, splits; kernel 0 = automatic
static std::atomic<int> g_force_kind{0}, g_force_bm{0}, g_force_bn{0}, g_force_s{0};
int forced_gemm_kernel() { return g_force_kind.load(); }

template <int T>
static int find_cand(int bm, int bn) {
    for (int i = 0; i < (int)(sizeof CANDS<T> / sizeof CANDS<T>[0]); ++i)
        if (CANDS<T>[i].bm == bm && CANDS<T>[i].bn == bn) return i;
    return -1;
}

template <int T>
static int pick(const Args& a, Plan* p) {
    *p = plan_gemm<T>(a.M, a.N, a.K, cus_of_device());
    if (g_force_kind.load() == K_TILES && g_force_bm.load() > 0) {
        const int fbm = g_force_bm.load(), fbn = g_force_bn.load(), fs = g_force_s.load();
        const int i = find_cand<T>(fbm, fbn);
        if (i < 0) return set_error(MBQ_BAD_ARG, "no GEMM tile %d x %d", fbm, fbn);
        const int64_t KT = (a.K + GK - 1) / GK, tiles = ((a.M + fbm - 1) / fbm) * ((a.N + fbn - 1) / fbn);
        int64_t S = std::max(1, fs), kts = (KT + S - 1) / S;
        S = (KT + kts - 1) / kts;
        if (S > 1 && (tiles > WS_TILES || (size_t)tiles * S * fbm * fbn * 4 > WS_BYTES))
            return set_error(MBQ_BAD_ARG, "forced split of %lld tiles x %lld does not fit the workspace", (long long)tiles, (long long)S);
        *p = Plan{i, (int)S, (int)kts};
    }
    return 0;
}

// The kernel of a batch the GEMV does not run: the weight-stream kernel (mbq_wsgemm.hip) up to WS_MAX_M rows, else the
// LDS-tile kernel; a forced plan overrides it.
struct Choice { int kind, bm, bn, S; };   // K_STREAM: bn weight rows per block; K_KGROUP: bn rows per block

static int choose(int t, const Args& a, Choice* c) {
    const int fk = g_force_kind.load();
    // tiled planes up to 64 rows: the K-group kernel (mbq_kgemm.hip), unless another kernel is forced
    if (tiled_type(t) && a.M <= WS_MAX_M && (fk == K_AUTO || fk == K_KGROUP)) {
        int R = 0, S = 0;
        if (int rc = kgemm_plan(t, a, fk == K_KGROUP ? g_force_s.load() : 0, &R, &S)) return rc;
        *c = Choice{K_KGROUP, 16, R, S};
        return 0;
    }
    if (fk == K_KGROUP && a.M <= WS_MAX_M)
        return set_error(MBQ_BAD_ARG, "the K-group kernel runs tiled planes (MBQ_I8T and the tiled GGUF types) only");
    if (fk == K_STREAM) {
        if (tiled_type(t) && t != T_I8T) return set_error(MBQ_BAD_ARG, "the weight-stream GEMM does not read tiled GGUF planes");
        if (a.M > WS_MAX_M)
            return set_error(MBQ_BAD_ARG, "a forced weight-stream plan needs M <= %lld", (long long)WS_MAX_M);
        *c = Choice{K_STREAM, 16, g_force_bn.load(), std::max(1, g_force_s.load())};
        return 0;
    }
    if (fk == K_TILES) {
        *c = Choice{K_TILES, g_force_bm.load(), g_force_bn.load(), std::max(1, g_force_s.load())};
        return 0;
    }
    // 16 < M <= 64 over a weight whose 64-row tiles alone fill the CUs (the weight-stream kernel would run 128-row
    // blocks): the LDS-tile kernel's 64 x 128 tiles are faster (MI355X, N = 17408, K = 5120, M = 64: int8 45 vs 52 us,
    // Q8_0 59 vs 73, Q4_K 51 vs 57, Q6_K 54 vs 79; M = 16 keeps the weight stream, 41 vs 43 us int8)
    // M <= GEMV_MAX_M arrives here only when the GEMV has no plan for the shape (launch_t): the weight stream takes it
    if (a.M <= WS_MAX_M && !(a.M > 16 && (a.N + 63) / 64 >= cus_of_device())) {
        int nr = 0, S = 1;
        wsgemm_plan(t, a, &nr, &S);
        *c = Choice{K_STREAM, 16, nr, S};
    } else {
        *c = Choice{K_TILES, 0, 0, 0};
    }
    return 0;
}

template <int T>
static int launch_gemm_t(const Args& a, hipStream_t s) {
    // buffer resources address one weight's planes and the whole x with 32-bit offsets
    if (a.wbytes > BUF_MAX_BYTES || a.M * a.K * 2 > BUF_MAX_BYTES)
        return set_error(MBQ_BAD_ARG, "GEMM operands over 2 GiB (weight %lld bytes, x %lld x %lld)", (long long)a.wbytes,
                         (long long)a.M, (long long)a.K);
    Choice c;
    if (int rc = choose(T, a, &c)) return rc;
    if (c.kind == K_STREAM) return launch_wsgemm(T, a, c.bn, c.S, s);
    if (c.kind == K_KGROUP) return launch_kgemm(T, a, c.S, s);
    Plan p;
    if (int rc = pick<T>(a, &p)) return rc;
    Workspace w;
    if (p.S > 1) {
        const int64_t tiles = ((a.M + CANDS<T>[p.idx].bm - 1) / CANDS<T>[p.idx].bm) * ((a.N + CANDS<T>[p.idx].bn - 1) / CANDS<T>[p.idx].bn);
        if (int rc = split_workspace(a, tiles, (size_t)tiles * p.S * CANDS<T>[p.idx].bm * CANDS<T>[p.idx].bn * 4, s, &w)) return rc;
    }
    return CANDS<T>[p.idx].launch(a, p.S, p.kts, w, s);
}

int gemm_plan(int t, const Args& a, int* kernel, int* bm, int* bn, int* splits) {
    Choice c;
    if (int rc = choose(t, a, &c)) return rc;
    *kernel = c.kind;
    if (c.kind == K_KGROUP) {
        *bm = 16;
        *bn = c.bn;
        *splits = c.S;
        return 0;
    }
    if (c.kind == K_STREAM) {
        int nr = c.bn, S = c.S;
        wsgemm_effective(t, a, &nr, &S);
        *bm = 16;
        *bn = nr;
        *splits = S;
        return 0;
    }
    Plan p;
    int rc;
    switch (t) {
        case T_Q4_0: rc = pick<T_Q4_0>(a, &p); if (!rc) *bm = CANDS<T_Q4_0>[p.idx].bm, *bn = CANDS<T_Q4_0>[p.idx].bn; break;
        case T_Q8_0: rc = pick<T_Q8_0>(a, &p); if (!rc) *bm = CANDS<T_Q8_0>[p.idx].bm, *bn = CANDS<T_Q8_0>[p.idx].bn; break;
        case T_Q4_K: rc = pick<T_Q4_K>(a, &p); if (!rc) *bm = CANDS<T_Q4_K>[p.idx].bm, *bn = CANDS<T_Q4_K>[p.idx].bn; break;
        case T_Q5_K: rc = pick<T_Q5_K>(a, &p); if (!rc) *bm = CANDS<T_Q5_K>[p.idx].bm, *bn = CANDS<T_Q5_K>[p.idx].bn; break;
        case T_Q6_K: rc = pick<T_Q6_K>(a, &p); if (!rc) *bm = CANDS<T_Q6_K>[p.idx].bm, *bn = CANDS<T_Q6_K>[p.idx].bn; break;
        case T_INT8: rc = pick<T_INT8>(a, &p); if (!rc) *bm = CANDS<T_INT8>[p.idx].bm, *bn = CANDS<T_INT8>[p.idx].bn; break;
        case T_I8T: rc = pick<T_I8T>(a, &p); if (!rc) *bm = CANDS<T_I8T>[p.idx].bm, *bn = CANDS<T_I8T>[p.idx].bn; break;
        case T_Q4KT: rc = pick<T_Q4KT>(a, &p); if (!rc) *bm = CANDS<T_Q4KT>[p.idx].bm, *bn = CANDS<T_Q4KT>[p.idx].bn; break;
        case T_Q8T: rc = pick<T_Q8T>(a, &p); if (!rc) *bm = CANDS<T_Q8T>[p.idx].bm, *bn = CANDS<T_Q8T>[p.idx].bn; break;
        case T_Q6KT: rc = pick<T_Q6KT>(a, &p); if (!rc) *bm = CANDS<T_Q6KT>[p.idx].bm, *bn = CANDS<T_Q6KT>[p.idx].bn; break;
        case T_Q5KT: rc = pick<T_Q5KT>(a, &p); if (!rc) *bm = CANDS<T_Q5KT>[p.idx].bm, *bn = CANDS<T_Q5KT>[p.idx].bn; break;
        case T_Q40T: rc = pick<T_Q40T>(a, &p); if (!rc) *bm = CANDS<T_Q40T>[p.idx].bm, *bn = CANDS<T_Q40T>[p.idx].bn; break;
        default: return set_error(MBQ_BAD_ARG, "no GEMM for type %d", t);
    }
    if (rc) return rc;
    *splits = p.S;
    return 0;
}

int force_gemm_plan(int kernel, int bm, int bn, int splits) {
    if (splits < 0) return set_error(MBQ_BAD_ARG, "splits %d", splits);
    switch (kernel) {
        case K_AUTO: break;
        case K_STREAM:
            if (bm != 16 || (bn != 64 && bn != 128)) return set_error(MBQ_BAD_ARG, "the weight-stream GEMM runs 16 x 64 or 16 x 128, not %d x %d", bm, bn);
            break;
        case K_TILES:
            if ((bm || bn) && find_cand<T_Q4_K>(bm, bn) < 0) return set_error(MBQ_BAD_ARG, "no LDS GEMM tile %d x %d", bm, bn);
            break;
        case K_KGROUP:
            if (bm || bn) return set_error(MBQ_BAD_ARG, "the K-group kernel chooses its own rows per block (bm = bn = 0)");
            break;
        default: return set_error(MBQ_BAD_ARG, "no GEMM kernel %d", kernel);
    }
    g_force_kind = kernel;
    g_force_bm = kernel ? bm : 0;
    g_force_bn = kernel ? bn : 0;
    g_force_s = kernel ? splits : 0;
    return 0;
}

int launch_gemm(int t, const Args& a, hipStream_t s) {
    switch (t) {
        case T_Q4_0: return launch_gemm_t<T_Q4_0>(a, s);
        case T_Q8_0: return launch_gemm_t<T_Q8_0>(a, s);
        case T_Q4_K: return launch_gemm_t<T_Q4_K>(a, s);
        case T_Q5_K: return launch_gemm_t<T_Q5_K>(a, s);
        case T_Q6_K: return launch_gemm_t<T_Q6_K>(a, s);
        case T_INT8: return launch_gemm_t<T_INT8>(a, s);
        case T_I8T: return launch_gemm_t<T_I8T>(a, s);
        case T_Q4KT: return launch_gemm_t<T_Q4KT>(a, s);
        case T_Q8T: return launch_gemm_t<T_Q8T>(a, s);
        case T_Q6KT: return launch_gemm_t<T_Q6KT>(a, s);
        case T_Q5KT: return launch_gemm_t<T_Q5KT>(a, s);
        case T_Q40T: return launch_gemm_t<T_Q40T>(a, s);
    }
    return set_error(MBQ_BAD_ARG, "no GEMM for type %d", t);
}

}  // namespace mbq
