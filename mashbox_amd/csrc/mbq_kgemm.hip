// gfx950 K-group GEMM of the int8 per-channel linear on tiled planes (T_I8T) for decode batches of 5..64 activation
// rows: y (M, N) = (x (M, K) @ bf16(q).T, float32 accumulation) * s, reference
// src/mashbox/models/qwen3_8_27b/model.py:72-82, with the weights repacked once at load into 16-row tiles
// (mbq_layout.h) from reference src/mashbox/models/qwen3_8_27b/weights.py:55-74.
//
// What bounds this regime on MI355X is the vector-memory throughput of a CU, not the MFMAs: a CU streams its share of
// the weights from HBM (about 25 GB/s at the chip's ~6.5 TB/s) and must also bring in the x its weights meet, 128
// bytes per K value at 64 rows, from L2. A CU moves about 50 GB/s with 4 waves and 70 GB/s with 8 (b128 loads,
// measured), so the x bytes per weight byte are what the design minimises:
//   * one block of 8 waves per CU: RG row groups x KG K groups (RG KG = 8). The waves of a K group walk the chunks
//     (64 K values) c = kg, kg + KG, ... of the block's K range; x of a chunk is copied once into that K group's LDS
//     ring by DMA (contiguous 8-row x 128-byte loads) and read by its RG waves as MFMA A operands, so every x byte
//     enters the CU once per block;
//   * a block owns any row range [r0, r1) of the weight, not a multiple of 16: N is cut into as many equal ranges as
//     fill the CUs (17408 rows = 256 ranges of 68), and a wave loads only its rows of the 16-row tiles it touches
//     (the rest of a tile reads zero through the buffer range check: no traffic); the MFMAs of those rows are wasted;
//   * K splits S (blocks per row range) cut the x bytes per block by S at the cost of float32 partials: each split
//     stores its partial tile, and the split that arrives last (an atomic counter per range, which it resets) adds the
//     S partials in split order, so the sum does not depend on arrival order. The partials sit in uncached device
//     memory, or (mbq_matmul_noalloc) in the static scratch with an agent-scope release / acquire around the exchange.
// Weights go from HBM (non-temporal loads) straight into B-operand registers, D chunks in flight per wave. After the
// K loop a reduce-scatter through LDS leaves each wave the sums of a share of the block's tiles (K groups added in a
// fixed order), so the split exchange and the stores run on all 8 waves; the row scales are loaded at the start.
//
// Lane layout (the weight-stream kernel's, mbq_wdirect.h): in K step s (32 values) of a chunk, lane l holds K values
// 16 (l >> 4) + 8 s + e (e = 0..7) of x row 16 i + (l & 15) and of weight row (l & 15) of a tile; the MFMA sums over
// K, so this K order is as good as any. x stage layout: 16 MT rows of 128 bytes, the 16-byte piece p of row r at slot
// p ^ ((r >> 1) & 7); the DMA applies the swizzle through each lane's source address. SQ_LDS_BANK_CONFLICT reads
// 2.7-3.0 cycles per LDS instruction with this swizzle and with p ^ (r & 7) alike, and the kernel's time is the same
// with either (MI355X): the A reads' bank cycles are not what bounds this kernel.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <algorithm>
#include <atomic>
#include <cmath>
#include <type_traits>
#include <utility>

#include "mbq_device.h"
#include "mbq_launch.h"
#include "mbq_layout.h"
#include "mbq_wdirect.h"

namespace mbq {

constexpr int KGM_THREADS = 512;   // 8 waves: 2 per SIMD

struct KgmArgs {
    const uint8_t* base;           // planes (host layer applied)
    int64_t stride;                // bytes between stacked weights (layer_dev)
    const int32_t* layer_dev;
    int nlayers;
    int64_t sc_off, wbytes;
    int64_t hi_off, d_off;         // Q6_K tiles: the high-bit and super-block scale planes
    const uint16_t* x;
    int M, N, K;
    void* y;
    int out_bf16;
    int R;                         // rows per block
    int S, kcs;                    // K splits per row range and chunks per split
    float* ws;                     // S > 1: partial tiles, (range, split) -> E floats
    int* cnt;                      // S > 1: arrival counter per row range (zero between launches)
    uint32_t ws_bytes;
    int fenced;                    // S > 1: ws is cached memory: release / acquire around the exchange
};

// K values per chunk: one KiB of a 16-row weight tile (int8, Q8_0: 64 values; the K-quants and Q4_0: 128, four 32-value
// units per row of nibbles)
constexpr int kgm_cw(int t) { return (t == T_Q4KT || t == T_Q5KT || t == T_Q6KT || t == T_Q40T) ? 128 : 64; }
// bytes of one x stage: 16 MT rows of one chunk of bfloat16 values
constexpr size_t kgm_stage(int t, int mt) { return (size_t)16 * mt * 2 * kgm_cw(t); }
// most dynamic LDS a block may take (160 KiB per CU, less a little for the static variables)
constexpr size_t KGM_LDS_MAX = 160 * 1024 - 256;
// K groups and LDS stages per K group (3 with two row groups, when the rings fit)
template <int RG> constexpr int kgm_kg() { return 8 / RG; }
constexpr int kgm_depth(int t, int mt, int rg) { return rg == 1 ? 2 : ((size_t)(8 / rg) * 3 * kgm_stage(t, mt) <= KGM_LDS_MAX ? 3 : 2); }
// bytes of the x rings of a block
constexpr size_t kgm_ring(int t, int mt, int rg) { return (size_t)(8 / rg) * kgm_depth(t, mt, rg) * kgm_stage(t, mt); }
// tiles per round of the K groups' reduce-scatter: 8 waves x TR tiles of 1 KiB in LDS at once (at most 80 KiB)
template <int MT, int NTW> constexpr int kgm_round() { return MT * NTW < 10 ? MT * NTW : 10; }
// dynamic LDS: the x rings, or the reduce-scatter's buffer if larger
template <int T, int MT, int RG, int NTW>
constexpr size_t kgm_lds() {
    const size_t ring = kgm_ring(T, MT, RG);
    const size_t red = (size_t)8 * kgm_round<MT, NTW>() * 1024;
    return ring > red ? ring : red;
}
// floats of one block's partial tile: RG row groups x MT x NTW 16x16 tiles
template <int MT, int RG, int NTW> constexpr int kgm_elems() { return RG * MT * NTW * 256; }

// a Q6_K tile unit as the weight-direct helpers take it: low nibbles, then (high bits, sub-block scales, super-block
// scale) as loaded into one 4-dword register set
__device__ __forceinline__ WsRaw<T_Q6_K> q6raw(const u32x4& q, const u32x4& h) { return WsRaw<T_Q6_K>{q, u32x2{h[0], h[1]}, h[2], h[3]}; }

// x stage swizzle: piece p of row r sits in slot p ^ kgm_swz(r). 128-byte rows (8 pieces): (r >> 1) & 7; 256-byte rows
// (16 pieces, Q4_K chunks): r & 15, so the 16 rows an A-operand read of one lane group takes (one piece each) fall on
// 16 different slots, every bank once
template <int PCS> __device__ __forceinline__ int kgm_swz(int r) { return PCS == 8 ? (r >> 1) & 7 : r & 15; }

// f(integral_constant<int, P>) for each P of the sequence, in order
template <class F, int... P>
__device__ __forceinline__ void kgm_each(F&& f, std::integer_sequence<int, P...>) {
    (f(std::integral_constant<int, P>{}), ...);
}

// ---------------------------------------------------------------------------------- factored sub-block products
// Nibble tiles (Q4_K, Q5_K, Q4_0) at up to 32 activation rows take the scales out of the MFMA operands. A lane's 16
// bytes of a chunk are one 32-value unit (sub-block) of its row, so in the loaded order the four lane groups hold four
// different sub-blocks. Two v_permlane32_swap and two v_permlane16_swap transpose the four units' dwords across the
// lane groups (kgm_lg_transpose), after which dword u of lane group g is dword g of unit u: K step u of the chunk is then
// sub-block u alone, and its B operand is the exact bfloat16 pairs 128 + q, one AND-OR (Q4_K, Q4_0) or one byte permute
// (Q5_K) per pair. With x's sum X over the sub-block,
//     sum_k x_k ((d sc) q_k - dmin m) = (d sc) * sum_k x_k (128 + q_k) - (128 d sc + dmin m) * X,
// so each K step's MFMA product is scaled by its sub-block's d sc (4 FMAs per x row tile), and the offsets of the
// chunk's four sub-blocks are one v_mfma_f32_16x16x4_f32 of the x sums (16 x rows x 4 sub-blocks, from MFMAs of the x
// operand against ones) and the offsets (4 sub-blocks x 16 weight rows: each lane's own sub-block). Q4_0 is the case
// d sc = d, offset 136 d. The dequantization's ~3.2 VALU per weight value become ~1.1; from 33 rows on the per-value
// form shares its dequantization over 3-4 x row tiles and needs fewer instructions, so it stays there.
// chunks per wave the register-x path holds (its plans keep every wave's chunk count within this)
constexpr int kgm_rx_chunks() { return 5; }
// register-x path: chunks of weights in flight per wave (two: three or four were slower on MI355X, e.g. a 17408 x 5120
// Q4_K gate at one row 15.4 -> 17.1 us, the 5120 x 17408 down 17.0 -> 18.6 us)
constexpr int kgm_rx_depth(int) { return 2; }

template <int T, int MT> constexpr bool kgm_factored() { return (T == T_Q4KT || T == T_Q5KT || T == T_Q40T) && MT >= 1 && MT <= 2; }

// in: lane group g holds dwords 0..3 of unit g (of its row); out: lane group g holds dword g of units 0..3
__device__ __forceinline__ u32x4 kgm_lg_transpose(const u32x4& w) {
    const u32x2 a = __builtin_bit_cast(u32x2, __builtin_amdgcn_permlane32_swap(w[0], w[2], false, false));
    const u32x2 b = __builtin_bit_cast(u32x2, __builtin_amdgcn_permlane32_swap(w[1], w[3], false, false));
    const u32x2 c = __builtin_bit_cast(u32x2, __builtin_amdgcn_permlane16_swap(a[0], b[0], false, false));
    const u32x2 d = __builtin_bit_cast(u32x2, __builtin_amdgcn_permlane16_swap(a[1], b[1], false, false));
    return u32x4{c[0], c[1], d[0], d[1]};
}

// the sum over the four lane groups (rows of 16 lanes) of v, in every lane: one v_permlane32_swap and one
// v_permlane16_swap, each with an add
__device__ __forceinline__ float kgm_lg_sum(float v) {
    const u32x2 a = __builtin_bit_cast(u32x2, __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false));
    const float h = __uint_as_float(a[0]) + __uint_as_float(a[1]);                  // groups 0 + 2, 1 + 3
    const u32x2 b = __builtin_bit_cast(u32x2, __builtin_amdgcn_permlane16_swap(__float_as_uint(h), __float_as_uint(h), false, false));
    return __uint_as_float(b[0]) + __uint_as_float(b[1]);
}

// a row's 16-byte Q4_K / Q5_K header in every lane of the row, from lane group g's dword g of it (a transpose of four
// copies: dword u of the result comes from lane group u)
__device__ __forceinline__ u32x4 kgm_hdr(uint32_t v) { return kgm_lg_transpose(u32x4{v, v, v, v}); }

// Q4_K / Q5_K: d sc of sub-blocks 4 h + u (u = 0..3) of the lane's row, from its super-block header meta (d and dmin,
// then the 12 scale bytes s0 s1 s2 as dwords 1-3; reference src/mashbox/ops/reference.py:132-139), all four 6-bit
// scales (and mins) unpacked at once, one per byte; *on = -(128 d sc + dmin m) of the lane's own sub-block 4 h + lg.
// Without branches: sub-blocks 0-3 (h = 0) take the low 6 bits of s0 (scales) and s1 (mins); sub-blocks 4-7 the low
// (high) nibbles of s2 with bits 6-7 of s0 (s1) as their bits 4-5. km = h ? 0x0F0F0F0F : 0x3F3F3F3F and
// hm = h ? 0x30303030 : 0 are the wave's masks.
__device__ __forceinline__ void kgm_kq_scales(const u32x4& meta, bool h, uint32_t km, uint32_t hm, int lg, float s[4],
                                              float* on) {
    const float d = f16f(meta[0]), dm = f16f(meta[0] >> 16);
    const uint32_t scv = ((h ? meta[3] : meta[1]) & km) | ((meta[1] >> 2) & hm);
    const uint32_t mnv = ((h ? meta[3] >> 4 : meta[2]) & km) | ((meta[2] >> 2) & hm);
#pragma unroll
    for (int u = 0; u < 4; ++u) s[u] = d * (float)((scv >> (8 * u)) & 0xFFu);         // exact
    const float sg = d * (float)__builtin_amdgcn_ubfe(scv, 8u * (uint32_t)lg, 8u);
    const float mg = dm * (float)__builtin_amdgcn_ubfe(mnv, 8u * (uint32_t)lg, 8u);
    *on = -__builtin_fmaf(128.f, sg, mg);
}

// Q4_0: the four blocks' scales d (fp16 pairs dd[0] = blocks 0, 1 and dd[1] = blocks 2, 3 of the chunk) and
// *on = -136 d of the lane's own block (d (q - 8) = d (128 + q) - 136 d; 136 d is exact)
__device__ __forceinline__ void kgm_q40_scales(uint32_t d01, uint32_t d23, int lg, float s[4], float* on) {
    s[0] = f16f(d01);
    s[1] = f16f(d01 >> 16);
    s[2] = f16f(d23);
    s[3] = f16f(d23 >> 16);
    *on = -136.f * f16f(__builtin_amdgcn_ubfe(lg < 2 ? d01 : d23, 16u * (uint32_t)(lg & 1), 16u));
}

template <int T, int MT, int RG, int NTW, bool KFULL>
__global__ __launch_bounds__(KGM_THREADS, 1) void kgemm_kernel(const KgmArgs g) {
    extern __shared__ __attribute__((aligned(16))) uint8_t kgm_lds_buf[];
    constexpr bool DIAG = MT < 0;                        // sub-block-diagonal x tiles (M <= 4 |MT|, see kgm_mt)
    constexpr int MX = DIAG ? -MT : MT;                  // 16-row x tiles of a stage (and accumulator tiles per tile)
    constexpr bool RX = MT == -1;                        // x in registers, no LDS stages (kgm_rx_chunks)
    constexpr int CHX = kgm_rx_chunks();                 // RX: most chunks per wave
    __shared__ int kgm_last;
    constexpr bool Q6 = T == T_Q6KT;                     // Q6_K tiles (the Q4_K tiles' chunks and lane units)
    constexpr bool Q5 = T == T_Q5KT;                     // Q5_K tiles (Q4_K's, plus a high-bit word per unit)
    constexpr bool Q40 = T == T_Q40T;                    // Q4_0 tiles (Q4_K's units, one fp16 scale per unit)
    constexpr bool QK = T == T_Q4KT || Q5 || Q6 || Q40;  // nibble-unit tiles
    constexpr bool Q8 = T == T_Q8T;                      // Q8_0 tiles (else int8 tiles)
    constexpr bool FACT = kgm_factored<T, MT>();         // factored sub-block products (above)
    constexpr int CW = kgm_cw(T);                        // K values per chunk
    constexpr int XB = 2 * CW;                           // bytes of one x row of a chunk
    constexpr int PCS = XB / 16;                         // its 16-byte pieces
    constexpr int RPI = 64 / PCS;                        // x rows per DMA instruction
    constexpr int NS = CW / 32;                          // MFMA K steps per chunk
    constexpr int KG = kgm_kg<RG>(), D = RX ? kgm_rx_depth(NTW) : kgm_depth(T, MX, RG);
    constexpr int STAGE = (int)kgm_stage(T, MX);         // bytes of one x stage (16 MX rows x CW values)
    constexpr int NX = STAGE / 1024 / RG;                // x DMA instructions per wave per chunk (1 KiB each)
    static_assert(NX * RG * 1024 == STAGE, "the RG waves of a K group issue whole DMA instructions");
    static_assert(kgm_ring(T, MX, RG) <= KGM_LDS_MAX, "the x rings fit the LDS");
    constexpr int NWL = Q6 ? 4 * NTW : Q5 ? 3 * NTW : QK || Q8 ? 2 * NTW : NTW;   // weight loads per chunk (Q4_K:
                                                         // quants, headers; Q5_K: and high bits; Q6_K: the four
                                                         // planes; Q8_0: quants, scales)
    constexpr int VMT = (D - 1) * NWL + (D - 2) * NX;    // loads issued after a chunk's last load (see the loop)
    static_assert(VMT < 64, "vmcnt range");
    const int M = g.M, N = g.N, K = g.K;
    const int lane = threadIdx.x & 63, lg = lane >> 4, r16 = lane & 15;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int kg = wave % KG, q = wave / KG;             // K group, row group
    const int rr = blockIdx.x / g.S, z = blockIdx.x - rr * g.S;

    // rows of this wave's row group: [rq0, rq1); its tiles start at tile rq0 / 16
    const int r0 = rr * g.R, r1 = min(N, r0 + g.R);
    const int RQ = (g.R + RG - 1) / RG;
    const int rq0 = min(r1, r0 + q * RQ), rq1 = min(r1, rq0 + RQ);
    const int t0 = rq0 >> 4;

    const int64_t lo = layer_offset(g.stride, g.layer_dev, g.nlayers);
    const bool ok = lo >= 0;
    const uint8_t* wb = g.base + (ok ? lo : 0);
    const rsrc_t wr = make_rsrc(wb, (uint32_t)g.wbytes);
    const rsrc_t xr = make_rsrc(g.x, (uint32_t)((int64_t)M * K * 2));

    // chunks of this split: [c0, c1); K group kg takes c0 + kg + KG l for l < its count; every group walks `steps`
    // steps (the block's barrier keeps them together), a step past its count loads zero through the range check
    const int KC = (K + CW - 1) / CW;
    const int c0 = z * g.kcs, c1 = min(KC, c0 + g.kcs);
    const int nch = ok ? max(0, c1 - c0) : 0;
    const int steps = (nch + KG - 1) / KG;
    const int mine = (nch - kg + KG - 1) / KG;           // chunks of this K group

    // weight offsets: tile t0 + j, row r16, the lane group's 16 bytes (of the chunk's KiB); Q4_K: also the row's
    // super-block headers; rows outside [rq0, rq1) read zero
    uint32_t wo[NTW], mo[NTW], ho[NTW], dq[NTW];
#pragma unroll
    for (int j = 0; j < NTW; ++j) {
        const int row = 16 * (t0 + j) + r16;
        const bool in = row >= rq0 && row < rq1;
        wo[j] = in ? (uint32_t)(Q40 ? q40t_off(row, K) : QK ? q4kt_off(row, K) : i8t_off(row, K, 0)) + 16u * (uint32_t)lg : OOB_VOFF;
        // factored Q4_0 / Q5_K: every lane loads its row's four block scales / high-bit words of the chunk
        mo[j] = in && (QK || Q8) ? (uint32_t)(g.sc_off + (Q6 ? q6kt_s_off(row, K) + 2 * lg
                                                         : Q40 ? q40t_d_off(row, K) + (FACT ? 0 : 2 * lg)
                                                         : QK ? q4kt_meta_off(row, K) : q8t_d_off(row, K)))
                                 : OOB_VOFF;
        ho[j] = in && (Q5 || Q6) ? (uint32_t)(g.hi_off + (Q6 ? q6kt_h_off(row, K) + 8 * lg : q5kt_h_off(row, K) + (FACT ? 0 : 4 * lg)))
                                 : OOB_VOFF;
        dq[j] = in && Q6 ? (uint32_t)(g.d_off + q6kt_d_off(row, K)) : OOB_VOFF;
    }
    // int8: the row scales of the tiles this wave finishes (see the reduce-scatter below), loaded first so that their
    // latency hides behind the K loop; the first step's vmcnt wait covers them (they are the oldest loads). Q4_K and
    // Q8_0 apply their block scales in the loop: 1.
    float sc[(MX * NTW + kgm_kg<RG>() - 1) / kgm_kg<RG>()];
#pragma unroll
    for (int u = 0; u < (MX * NTW + kgm_kg<RG>() - 1) / kgm_kg<RG>(); ++u) {
        const int tt = kg + kgm_kg<RG>() * u, j = tt % NTW, n = 16 * (t0 + j) + r16;
        const bool live = ok && tt < MX * NTW && n >= rq0 && n < rq1;
        if constexpr (QK || Q8)
            sc[u] = 1.f;
        else
            sc[u] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(wr, live ? (uint32_t)(g.sc_off + 4 * (int64_t)n) : OOB_VOFF, 0, 0));
    }
    // x DMA: instruction i of this wave fills rows RPI (q + RG i) .. + RPI - 1 of the stage; lane l writes slot l % PCS
    // of row l / PCS, which holds piece (l % PCS) ^ kgm_swz(row); rows past M read zero
    uint32_t xvo[NX];
    int xk[NX];
#pragma unroll
    for (int i = 0; i < NX; ++i) {
        const int r = RPI * (q + RG * i) + lane / PCS, p = (lane % PCS) ^ kgm_swz<PCS>(r);
        if constexpr (DIAG) {
            // stage row r = 16 t + 4 u + e holds x row 4 t + e in the pieces of sub-block u (4 u .. 4 u + 3) and zeros
            // in the others
            const int xr = 4 * (r >> 4) + (r & 3);
            xvo[i] = xr < M && (p >> 2) == ((r >> 2) & 3) ? (uint32_t)(((int64_t)xr * K + 8 * p) * 2) : OOB_VOFF;
        } else {
            xvo[i] = r < M ? (uint32_t)(((int64_t)r * K + 8 * p) * 2) : OOB_VOFF;
        }
        xk[i] = 8 * p;
    }
    uint8_t* ring = kgm_lds_buf + (size_t)kg * D * STAGE;
    auto chunk_of = [&](int l) __attribute__((always_inline)) { return c0 + kg + KG * l; };            // valid while l < mine
    auto dma_x = [&](int st, int l) __attribute__((always_inline)) {
        const int c = chunk_of(l);
        const bool live = l < mine;
#pragma unroll
        for (int i = 0; i < NX; ++i) {
            uint32_t v = live ? xvo[i] : OOB_VOFF;
            if constexpr (!KFULL) v = (CW * c + xk[i] < K) ? v : OOB_VOFF;
            dma16(xr, reinterpret_cast<uint16_t*>(ring + st * STAGE + RPI * (q + RG * i) * XB), v,
                     live ? (uint32_t)c * (uint32_t)XB : 0u);
        }
    };
    // the chunk's weights: a KiB per tile (non-temporal), and for Q4_K the 16-byte header of the super-block (chunk / 2).
    // Q8_0: the lane's 16 bytes are its 8 quants of each of the chunk's two blocks (K step s = block s: values
    // 32 s + 8 lg ..), then the row's two block scales
    auto load_w = [&](u32x4* W, u32x4* H, u32x4* Hb, int l) __attribute__((always_inline)) {
        const int c = chunk_of(l);
        const bool live = l < mine;
#pragma unroll
        for (int j = 0; j < NTW; ++j) {
            W[j] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(wr, live ? wo[j] : OOB_VOFF,
                                                                                  live ? (uint32_t)c * 1024u : 0u, 2));
            if constexpr (Q8)
                H[j][0] = (uint32_t)__builtin_amdgcn_raw_buffer_load_b32(wr, live ? mo[j] : OOB_VOFF, live ? (uint32_t)c * 64u : 0u, 0);
            if constexpr (Q6) {
                // the unit's 8 bytes of high bits, its two sub-block scales, the super-block scale
                const u32x2 h = __builtin_bit_cast(u32x2, __builtin_amdgcn_raw_buffer_load_b64(
                                    wr, live ? ho[j] : OOB_VOFF, live ? (uint32_t)c * 512u : 0u, 2));
                H[j] = u32x4{h[0], h[1], bload2(wr, live ? mo[j] : OOB_VOFF, live ? (uint32_t)c * 128u : 0u),
                             bload2(wr, live ? dq[j] : OOB_VOFF, live ? (uint32_t)(c >> 1) * 32u : 0u)};
            } else if constexpr (Q40 && FACT) {                   // the four blocks' scales
                const u32x2 d = __builtin_bit_cast(u32x2, __builtin_amdgcn_raw_buffer_load_b64(
                                    wr, live ? mo[j] : OOB_VOFF, live ? (uint32_t)c * 128u : 0u, 0));
                H[j][0] = d[0];
                H[j][1] = d[1];
            } else if constexpr (Q40) {
                H[j][0] = bload2(wr, live ? mo[j] : OOB_VOFF, live ? (uint32_t)c * 128u : 0u);   // the unit's block scale
            } else if constexpr (QK) {
                // Q4_K / Q5_K: dword lg of the row's 16-byte super-block header (the four lane groups of a row load its
                // four dwords, 256 B per wave instead of a KiB; kgm_hdr gives every lane all four)
                H[j][0] = (uint32_t)__builtin_amdgcn_raw_buffer_load_b32(wr, live ? mo[j] + 4u * (uint32_t)lg : OOB_VOFF,
                                                                         live ? (uint32_t)(c >> 1) * 256u : 0u, 0);
                if constexpr (Q5 && FACT)                         // the four units' high-bit words
                    Hb[j] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(
                                wr, live ? ho[j] : OOB_VOFF, live ? (uint32_t)c * 256u : 0u, 2));
                else if constexpr (Q5)                            // the unit's high-bit word
                    Hb[j][0] = (uint32_t)__builtin_amdgcn_raw_buffer_load_b32(wr, live ? ho[j] : OOB_VOFF, live ? (uint32_t)c * 256u : 0u, 2);
            }
        }
    };
    // A operand: x row 16 i + (lane & 15), piece NS (lane >> 4) + s of stage st (Q8_0: 4 s + (lane >> 4)), the K values
    // the lane's weights hold
    auto a_op = [&](int st, int i, int s) __attribute__((always_inline)) {
        const int r = 16 * i + r16, p = (Q8 ? 4 * s + lg : NS * lg + s) ^ kgm_swz<PCS>(r);
        return *reinterpret_cast<const bf16x8_t*>(ring + st * STAGE + r * XB + (p << 4));
    };

    f32x4_t acc[MX][NTW];
#pragma unroll
    for (int i = 0; i < MX; ++i)
#pragma unroll
        for (int j = 0; j < NTW; ++j) acc[i][j] = f32x4_t{0.f, 0.f, 0.f, 0.f};
    u32x4 W[D][NTW];
    u32x4 H[QK || Q8 ? D : 1][NTW];                                       // K-quants: headers / scales; Q8_0: scales
    u32x4 Hb[Q5 ? D : 1][NTW];                                            // Q5_K: high-bit word(s)

    // Issue order: x0 w0 x1 w1 .. x(D-2) w(D-2) w(D-1), then step l issues x(l+D-1) and w(l+D). At step l's wait the
    // loads issued after x(l) (steady state) or w(l) (first steps) number VMT, so vmcnt <= VMT means both landed.
    // J < 0: a step of the unrolled loop. J >= 0: step J of the last steps % D, whose x and weights would be for steps
    // past the last, so it issues no DMA and no loads (loads nobody reads are dropped by the compiler, and the wait
    // must count what is issued): after x(l) come only the loads of the D - 1 - J loop steps before the tail.
    auto step = [&](auto U_, auto J_, int l) __attribute__((always_inline)) {
        constexpr int U = decltype(U_)::value;                            // l % D
        constexpr int J = decltype(J_)::value;
        wait_vm<J < 0 ? VMT : (D - 1 - J) * NWL + (D - 2 - J) * NX>();
        // stage U landed for every wave; stage (l - 1) % D is no longer read. With one row group a wave reads only the
        // stages it fills, but the block-wide barrier still measured faster (it keeps the waves' x reads together)
        barrier_nofence();
        __builtin_amdgcn_sched_barrier(0);
        if constexpr (J < 0) dma_x((U + D - 1) % D, l + D - 1);
        __builtin_amdgcn_sched_barrier(0);
        if constexpr (DIAG) {
            // the chunk's four K steps chain into one product per tile: output row 4 u + e of x tile i is x row 4 i + e
            // times sub-block u (the lane group's unit, whose scale the lane holds); the x sums by the same chain
            // against ones; then the lane's (d sc, offset) once per chunk
            const int j8 = 4 * (chunk_of(l) & 1) + lg;
            const bf16x8_t ones = __builtin_bit_cast(bf16x8_t, u32x4{BF16_ONES, BF16_ONES, BF16_ONES, BF16_ONES});
            f32x4_t P[MX][NTW], DX[MX];
#pragma unroll
            for (int i = 0; i < MX; ++i) {
                DX[i] = f32x4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
                for (int j = 0; j < NTW; ++j) P[i][j] = f32x4_t{0.f, 0.f, 0.f, 0.f};
            }
#pragma unroll
            for (int s = 0; s < NS; ++s) {
                bf16x8_t A[MX];
#pragma unroll
                for (int i = 0; i < MX; ++i) {
                    A[i] = a_op(U, i, s);
                    DX[i] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(A[i], ones, DX[i], 0, 0, 0);
                }
#pragma unroll
                for (int j = 0; j < NTW; ++j) {
                    const uint32_t w = W[U][j][s];
                    u32x4 o;
                    if constexpr (Q5) {
                        uint32_t lo, hi;
                        q5k_bytes(w, Hb[U][j][0], s, &lo, &hi);
                        const uint32_t c43 = in_vgpr(0x43434343u);
                        o = u32x4{b128_pair(lo, c43, 0), b128_pair(lo, c43, 1), b128_pair(hi, c43, 0), b128_pair(hi, c43, 1)};
                    } else {
                        const uint32_t m = in_vgpr(0x000F000Fu), e = in_vgpr(0x43004300u);
                        o = u32x4{(w & m) | e, ((w >> 4) & m) | e, ((w >> 8) & m) | e, ((w >> 12) & m) | e};
                    }
                    const bf16x8_t B = __builtin_bit_cast(bf16x8_t, o);
#pragma unroll
                    for (int i = 0; i < MX; ++i) P[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(A[i], B, P[i][j], 0, 0, 0);
                }
            }
#pragma unroll
            for (int j = 0; j < NTW; ++j) {
                float a, on;
                if constexpr (Q40) {
                    a = f16f(H[U][j][0]);
                    on = -136.f * a;                                             // d (q - 8) = d (128 + q) - 136 d
                } else {
                    const u32x4 hd = kgm_hdr(H[U][j][0]);
                    const WsScale c = Q5 ? ws_scale<T_Q5_K>(WsRaw<T_Q5_K>{W[U][j], hd, Hb[U][j][0]}, j8)
                                         : ws_scale<T_Q4_K>(WsRaw<T_Q4_K>{W[U][j], hd}, j8);
                    a = c.a;
                    on = -__builtin_fmaf(128.f, c.a, c.b);                       // -(128 d sc + dmin m)
                }
#pragma unroll
                for (int i = 0; i < MX; ++i)
#pragma unroll
                    for (int r = 0; r < 4; ++r)
                        acc[i][j][r] = __builtin_fmaf(on, DX[i][r], __builtin_fmaf(a, P[i][j][r], acc[i][j][r]));
            }
            __builtin_amdgcn_sched_barrier(0);
            if constexpr (J < 0) load_w(W[U], H[U], Hb[Q5 ? U : 0], l + D);
            return;
        }
        if constexpr (FACT) {
            // K step u = sub-block u of the chunk: lane group lg's x values are values 8 lg .. 8 lg + 7 of it (piece
            // 4 u + lg); the x sums of the four sub-blocks by MFMAs against ones, with x as the B operand, so that
            // lane l holds row 16 i + (l & 15)'s sum (the f32 MFMA's A operand takes sub-block lg's)
            // the super-block half of the chunk: c0 + kg + KG l has the parity of c0 + kg (KG is even)
            static_assert(KG % 2 == 0, "a K group's chunks keep their parity");
            const bool h = ((c0 + kg) & 1) != 0;
            const uint32_t km = h ? 0x0F0F0F0Fu : 0x3F3F3F3Fu, hm = h ? 0x30303030u : 0u;
            const bf16x8_t ones = __builtin_bit_cast(bf16x8_t, u32x4{BF16_ONES, BF16_ONES, BF16_ONES, BF16_ONES});
            bf16x8_t A[4][MX];
            float xs[MX];
#pragma unroll
            for (int i = 0; i < MX; ++i) {
#pragma unroll
                for (int u = 0; u < 4; ++u) {
                    const int r = 16 * i + r16, p = (4 * u + lg) ^ kgm_swz<PCS>(r);
                    A[u][i] = *reinterpret_cast<const bf16x8_t*>(ring + U * STAGE + r * XB + (p << 4));
                }
#pragma unroll
                for (int u = 0; u < 4; ++u) {
                    const f32x4_t t = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ones, A[u][i], f32x4_t{0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
                    xs[i] = u == 0 ? t[0] : (lg == u ? t[0] : xs[i]);
                }
            }
#pragma unroll
            for (int j = 0; j < NTW; ++j) {
                const u32x4 w = kgm_lg_transpose(W[U][j]);                 // dword u: values 8 lg .. of sub-block u
                float sc4[4], on;
                if constexpr (Q40)
                    kgm_q40_scales(H[U][j][0], H[U][j][1], lg, sc4, &on);
                else
                    kgm_kq_scales(kgm_hdr(H[U][j][0]), h, km, hm, lg, sc4, &on);
                f32x4_t P[4][MX];
#pragma unroll
                for (int u = 0; u < 4; ++u) {
                    u32x4 o;
                    if constexpr (Q5) {
                        uint32_t lo, hi;
                        q5k_bytes(w[u], Hb[U][j][u], lg, &lo, &hi);
                        const uint32_t c43 = in_vgpr(0x43434343u);
                        o = u32x4{b128_pair(lo, c43, 0), b128_pair(lo, c43, 1), b128_pair(hi, c43, 0), b128_pair(hi, c43, 1)};
                    } else {
                        // ((w >> 4p) & 0x000F000F) | 0x43004300: one v_and_or_b32 with both constants in registers
                        const uint32_t m = in_vgpr(0x000F000Fu), e = in_vgpr(0x43004300u);
                        o = u32x4{(w[u] & m) | e, ((w[u] >> 4) & m) | e, ((w[u] >> 8) & m) | e, ((w[u] >> 12) & m) | e};
                    }
                    const bf16x8_t B = __builtin_bit_cast(bf16x8_t, o);
#pragma unroll
                    for (int i = 0; i < MX; ++i)
                        P[u][i] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(A[u][i], B, f32x4_t{0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
                }
#pragma unroll
                for (int u = 0; u < 4; ++u)
#pragma unroll
                    for (int i = 0; i < MX; ++i)
#pragma unroll
                        for (int r = 0; r < 4; ++r) acc[i][j][r] = __builtin_fmaf(sc4[u], P[u][i][r], acc[i][j][r]);
#pragma unroll
                for (int i = 0; i < MX; ++i) acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x4f32(xs[i], on, acc[i][j], 0, 0, 0);
            }
            __builtin_amdgcn_sched_barrier(0);
            if constexpr (J < 0) load_w(W[U], H[U], Hb[Q5 ? U : 0], l + D);
            return;
        }
        // Q4_K: the lane's 16 bytes are one 32-value unit of its row, sub-block 4 (chunk % 2) + lg of the super-block;
        // its (d sc, dmin m) for the whole chunk
        WsScale qs[QK ? NTW : 1];
        if constexpr (Q6) {
#pragma unroll
            for (int j = 0; j < NTW; ++j) qs[j] = ws_scale<T_Q6_K>(q6raw(W[U][j], H[U][j]), 0);
        } else if constexpr (Q40) {
#pragma unroll
            for (int j = 0; j < NTW; ++j) {
                const float d = f16f(H[U][j][0]);
                qs[j] = WsScale{d, 8.f * d, d * 0.0625f, 0.f};          // d q - 8 d = (q - 8) d, exact in float32
            }
        } else if constexpr (Q5) {
            const int j8 = 4 * (chunk_of(l) & 1) + lg;
#pragma unroll
            for (int j = 0; j < NTW; ++j) qs[j] = ws_scale<T_Q5_K>(WsRaw<T_Q5_K>{W[U][j], kgm_hdr(H[U][j][0]), Hb[U][j][0]}, j8);
        } else if constexpr (QK) {
            const int j8 = 4 * (chunk_of(l) & 1) + lg;
#pragma unroll
            for (int j = 0; j < NTW; ++j) qs[j] = ws_scale<T_Q4_K>(WsRaw<T_Q4_K>{W[U][j], kgm_hdr(H[U][j][0])}, j8);
        }
#pragma unroll
        for (int s = 0; s < NS; ++s) {
            bf16x8_t A[MX];
#pragma unroll
            for (int i = 0; i < MX; ++i) A[i] = a_op(U, i, s);
            if constexpr (Q8 && MX <= 2) {
                // Q8_0, one or two x row tiles: every MFMA of the step first (their block products in P), then the
                // scale FMAs, so no FMA waits on the MFMA just issued
                f32x4_t P[MX][NTW];
#pragma unroll
                for (int j = 0; j < NTW; ++j) {
                    const uint32_t a = hide(W[U][j][2 * s]), b = hide(W[U][j][2 * s + 1]);
                    const u32x4 o{i8_pair(a, 0), i8_pair(a, 1), i8_pair(b, 0), i8_pair(b, 1)};
                    const bf16x8_t B = __builtin_bit_cast(bf16x8_t, o);
#pragma unroll
                    for (int i = 0; i < MX; ++i)
                        P[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(A[i], B, f32x4_t{0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
                }
#pragma unroll
                for (int j = 0; j < NTW; ++j) {
                    const float ds = f16f(s == 0 ? H[U][j][0] : H[U][j][0] >> 16);
#pragma unroll
                    for (int i = 0; i < MX; ++i)
#pragma unroll
                        for (int r = 0; r < 4; ++r) acc[i][j][r] = __builtin_fmaf(P[i][j][r], ds, acc[i][j][r]);
                }
                continue;
            }
#pragma unroll
            for (int j = 0; j < NTW; ++j) {
                bf16x8_t B;
                if constexpr (Q6) {
                    // values 8 s .. 8 s + 7 of the unit, (d sc) (q - 32) rounded to bfloat16 (the LDS GEMM's operand)
                    B = ws_bop<T_Q6_K>(q6raw(W[U][j], H[U][j]), qs[j], s);
                } else if constexpr (Q5) {
                    // values 8 s .. 8 s + 7 of the unit, (d sc) q - dmin m (one rounding) rounded to bfloat16
                    B = ws_bop<T_Q5_K>(WsRaw<T_Q5_K>{W[U][j], H[U][j], Hb[U][j][0]}, qs[j], s);
                } else if constexpr (QK) {
                    // values 8 s .. 8 s + 7 of the unit, (d sc) q - dmin m rounded to bfloat16 (the LDS GEMM's operand)
                    B = q4k_dword_bop(W[U][j][s], qs[j]);
                } else {
                    const uint32_t a = hide(W[U][j][2 * s]), b = hide(W[U][j][2 * s + 1]);
                    const u32x4 o{i8_pair(a, 0), i8_pair(a, 1), i8_pair(b, 0), i8_pair(b, 1)};
                    B = __builtin_bit_cast(bf16x8_t, o);
                }
                if constexpr (Q8) {
                    // K step s is block s of the chunk: its exact int8 product, then times the row's block scale
                    const float ds = f16f(s == 0 ? H[U][j][0] : H[U][j][0] >> 16);
#pragma unroll
                    for (int i = 0; i < MX; ++i) {
                        const f32x4_t p = __builtin_amdgcn_mfma_f32_16x16x32_bf16(A[i], B, f32x4_t{0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
#pragma unroll
                        for (int r = 0; r < 4; ++r) acc[i][j][r] = __builtin_fmaf(p[r], ds, acc[i][j][r]);
                    }
                } else {
#pragma unroll
                    for (int i = 0; i < MX; ++i) acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(A[i], B, acc[i][j], 0, 0, 0);
                }
            }
        }
        __builtin_amdgcn_sched_barrier(0);
        if constexpr (J < 0) load_w(W[U], H[QK || Q8 ? U : 0], Hb[Q5 ? U : 0], l + D);
    };

    if constexpr (RX) {
        // The wave's chunks' A operands stay in registers for the whole kernel (the diagonal mapping: lane (lg, r16)
        // holds x row r16 & 3's values of unit lg of the chunk when lg == r16 >> 2, else zero), so the K loop has no
        // LDS stage, DMA or barrier; weights run D chunks ahead. A chunk past the wave's count loads nothing (OOB).
        bf16x8_t AX[CHX][NS];
        {
            const int xrow = r16 & 3;
            const bool lv = lg == (r16 >> 2) && xrow < M;
#pragma unroll
            for (int ci = 0; ci < CHX; ++ci) {
                const bool live = lv && ci < mine && (KFULL || CW * chunk_of(ci) + 32 * lg < K);
                const uint32_t off = live ? (uint32_t)(((int64_t)xrow * K + CW * chunk_of(ci) + 32 * lg) * 2) : OOB_VOFF;
                // the scalar offset stays uniform (a per-lane choice there makes the compiler loop over its values):
                // a lane that loads nothing has OOB_VOFF + 16 u, still past the range
#pragma unroll
                for (int u = 0; u < NS; ++u)
                    AX[ci][u] = __builtin_bit_cast(bf16x8_t, __builtin_amdgcn_raw_buffer_load_b128(xr, off, 16u * u, 0));
            }
        }
#pragma unroll
        for (int p = 0; p < D; ++p) load_w(W[p], H[p], Hb[Q5 ? p : 0], p);
        // every weight load issues before the first wait for x (else the compiler hoists the x sums' MFMAs, and their
        // waits for x, above the weight loads, and the stream starts a round trip late)
        __builtin_amdgcn_sched_barrier(0);
        wait_vm<D * NWL>();                                               // the x loads (issued first) have landed
        const bf16x8_t ones = __builtin_bit_cast(bf16x8_t, u32x4{BF16_ONES, BF16_ONES, BF16_ONES, BF16_ONES});
        f32x4_t DX[CHX];
#pragma unroll
        for (int ci = 0; ci < CHX; ++ci) {
            DX[ci] = f32x4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int u = 0; u < NS; ++u) DX[ci] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(AX[ci][u], ones, DX[ci], 0, 0, 0);
        }
        kgm_each([&](auto CI) __attribute__((always_inline)) {
            constexpr int ci = decltype(CI)::value, U = ci % D;
            if (ci < mine) {                                              // wave-uniform; later chunks are dead too
                wait_vm<(D - 1 < CHX - 1 - ci ? D - 1 : CHX - 1 - ci) * NWL>();
                const int j8 = 4 * (chunk_of(ci) & 1) + lg;
#pragma unroll
                for (int j = 0; j < NTW; ++j) {
                    f32x4_t P = f32x4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
                    for (int u = 0; u < NS; ++u) {
                        const uint32_t w = W[U][j][u];
                        u32x4 o;
                        if constexpr (Q5) {
                            uint32_t lo, hi;
                            q5k_bytes(w, Hb[U][j][0], u, &lo, &hi);
                            const uint32_t c43 = in_vgpr(0x43434343u);
                            o = u32x4{b128_pair(lo, c43, 0), b128_pair(lo, c43, 1), b128_pair(hi, c43, 0), b128_pair(hi, c43, 1)};
                        } else {
                            const uint32_t m = in_vgpr(0x000F000Fu), e = in_vgpr(0x43004300u);
                            o = u32x4{(w & m) | e, ((w >> 4) & m) | e, ((w >> 8) & m) | e, ((w >> 12) & m) | e};
                        }
                        P = __builtin_amdgcn_mfma_f32_16x16x32_bf16(AX[ci][u], __builtin_bit_cast(bf16x8_t, o), P, 0, 0, 0);
                    }
                    float a, on;
                    if constexpr (Q40) {
                        a = f16f(H[U][j][0]);
                        on = -136.f * a;
                    } else {
                        const u32x4 hd = kgm_hdr(H[U][j][0]);
                        const WsScale c = Q5 ? ws_scale<T_Q5_K>(WsRaw<T_Q5_K>{W[U][j], hd, Hb[U][j][0]}, j8)
                                             : ws_scale<T_Q4_K>(WsRaw<T_Q4_K>{W[U][j], hd}, j8);
                        a = c.a;
                        on = -__builtin_fmaf(128.f, c.a, c.b);
                    }
#pragma unroll
                    for (int r = 0; r < 4; ++r) acc[0][j][r] = __builtin_fmaf(on, DX[ci][r], __builtin_fmaf(a, P[r], acc[0][j][r]));
                }
                if constexpr (ci + D < CHX) load_w(W[U], H[U], Hb[Q5 ? U : 0], ci + D);
            }
        }, std::make_integer_sequence<int, CHX>{});
        wait_vm<0>();
    } else if (steps > 0) {                                               // block-uniform
#pragma unroll
        for (int p = 0; p < D; ++p) {
            if (p < D - 1) dma_x(p, p);
            load_w(W[p], H[QK || Q8 ? p : 0], Hb[Q5 ? p : 0], p);
        }
        int l = 0;
        for (; l + D <= steps; l += D)
            kgm_each([&](auto P) __attribute__((always_inline)) {
                step(P, std::integral_constant<int, -1>{}, l + decltype(P)::value);
            }, std::make_integer_sequence<int, D>{});
        kgm_each([&](auto P) __attribute__((always_inline)) {
            if (l + decltype(P)::value < steps) step(P, P, l + decltype(P)::value);
        }, std::make_integer_sequence<int, D - 1>{});
        wait_vm<0>();                                                     // no DMA may land after the rings are reused
    }
    if constexpr (DIAG) {
        // lane group g holds sub-block g's share of each output: their sum, in lane group 0's rows 0-3 of each tile
#pragma unroll
        for (int i = 0; i < MX; ++i)
#pragma unroll
            for (int j = 0; j < NTW; ++j)
#pragma unroll
                for (int r = 0; r < 4; ++r) acc[i][j][r] = kgm_lg_sum(acc[i][j][r]);
    }
    __syncthreads();

    // Reduce-scatter of the K groups' accumulators through LDS, in rounds of TR tiles (a tile: one 16 x 16 float32
    // MFMA result, 1 KiB over the wave): every wave writes its tiles of the round, and the wave that owns a tile (tile tt
    // of row group q belongs to K group tt % KG) adds the KG copies in K-group order. Every wave then holds the block's
    // sums of its TPW tiles, and the split exchange and the stores below run on all 8 waves at once.
    constexpr int TT = MX * NTW, TR = kgm_round<MX, NTW>(), TPW = (TT + KG - 1) / KG;
    f32x4_t* red = reinterpret_cast<f32x4_t*>(kgm_lds_buf);
    f32x4_t fin[TPW];
#pragma unroll
    for (int u = 0; u < TPW; ++u) fin[u] = f32x4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int r0 = 0; r0 < TT; r0 += TR) {
#pragma unroll
        for (int i = 0; i < MX; ++i)
#pragma unroll
            for (int j = 0; j < NTW; ++j) {
                const int tt = i * NTW + j;
                if (tt >= r0 && tt < r0 + TR) red[((size_t)wave * TR + (tt - r0)) * 64 + lane] = acc[i][j];
            }
        __syncthreads();
#pragma unroll
        for (int u = 0; u < TPW; ++u) {
            const int tt = kg + KG * u;
            if (tt >= r0 && tt < r0 + TR && tt < TT) {                    // wave-uniform
                const f32x4_t* src = red + ((size_t)(q * KG) * TR + (tt - r0)) * 64 + lane;
                f32x4_t v = src[0];
#pragma unroll
                for (int k = 1; k < KG; ++k) v += src[(size_t)k * TR * 64];
                fin[u] = v;
            }
        }
        __syncthreads();
    }

    constexpr int E = kgm_elems<MX, RG, NTW>();
    if (g.S > 1) {
        // each wave stores its tiles of the block's partial, (range, split) -> E floats laid out [q][tile][lane]; the
        // split that arrives last adds the S partials of each tile in split order (its own from registers)
        const rsrc_t pr = make_rsrc(g.ws, g.ws_bytes);
        const uint32_t own = (uint32_t)(blockIdx.x * E) * 4u;
#pragma unroll
        for (int u = 0; u < TPW; ++u) {
            const int tt = kg + KG * u;
            const uint32_t off = tt < TT ? (uint32_t)((q * TT + tt) * 64 + lane) * 16u : OOB_VOFF;
            __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, fin[u]), pr, off, own, 16);
        }
        if (g.fenced) split_release();                                    // the partial is visible at agent scope
        else wait_vm<0>();
        __syncthreads();
        if (threadIdx.x == 0) {
            const int old = __hip_atomic_fetch_add(g.cnt + rr, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            kgm_last = old == g.S - 1;
            if (old == g.S - 1) __hip_atomic_store(g.cnt + rr, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
        __syncthreads();
        if (!kgm_last) return;
        if (g.fenced) split_acquire();                                    // the other blocks' partials, not stale lines
        const uint32_t first = (uint32_t)(rr * g.S * E) * 4u;
        f32x4_t sum[TPW] = {};
        // the loads of ZC splits in flight at once (every split of a plan of up to 8 when TPW <= 3: one round trip),
        // then their sums in split order
        constexpr int ZC = 24 / TPW >= 8 ? 8 : (24 / TPW < 1 ? 1 : 24 / TPW);
        for (int z0 = 0; z0 < g.S; z0 += ZC) {
            f32x4_t v[ZC][TPW];
#pragma unroll
            for (int c = 0; c < ZC; ++c)
#pragma unroll
                for (int u = 0; u < TPW; ++u) {
                    const int zz = z0 + c, tt = kg + KG * u;
                    const bool live = zz < g.S && zz != z && tt < TT;
                    v[c][u] = __builtin_bit_cast(f32x4_t, __builtin_amdgcn_raw_buffer_load_b128(
                                  pr, live ? (uint32_t)((q * TT + tt) * 64 + lane) * 16u : OOB_VOFF,
                                  live ? first + (uint32_t)(zz * E) * 4u : 0u, 16));
                }
#pragma unroll
            for (int c = 0; c < ZC; ++c) {
                const int zz = z0 + c;
                if (zz < g.S) {
#pragma unroll
                    for (int u = 0; u < TPW; ++u) {
                        const f32x4_t t = zz == z ? fin[u] : v[c][u];
                        sum[u] = zz == 0 ? t : sum[u] + t;
                    }
                }
            }
        }
#pragma unroll
        for (int u = 0; u < TPW; ++u) fin[u] = sum[u];
    }

    // stores: tile tt = i NTW + j of this wave's row group holds rows m = 16 i + 4 (lane >> 4) + r of x and column
    // n = 16 (t0 + j) + (lane & 15) of y; a store past M or outside [rq0, rq1) gets an offset out of y's range (no
    // write), so the stores run back to back with no branch and no wait between them
    const uint32_t esz = g.out_bf16 ? 2u : 4u;
    const rsrc_t yr = make_rsrc(g.y, (uint32_t)M * (uint32_t)N * esz);
#pragma unroll
    for (int u = 0; u < TPW; ++u) {
        const int tt = kg + KG * u, i = tt / NTW, j = tt - i * NTW;
        const int n = 16 * (t0 + j) + r16;
        const bool col = tt < TT && n >= rq0 && n < rq1;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            // diagonal x tiles: x row 4 i + r, stored by lane group 0 (every group holds the same sums)
            const int m = DIAG ? (lg == 0 ? 4 * i + r : M) : 16 * i + 4 * lg + r;
            const uint32_t off = (col && m < M) ? ((uint32_t)m * (uint32_t)N + (uint32_t)n) * esz : OOB_VOFF;
            const float v = fin[u][r] * (ok ? sc[u] : __builtin_nanf(""));    // a layer outside the stack: NaN
            if (g.out_bf16)
                __builtin_amdgcn_raw_buffer_store_b16((uint16_t)pack_bf16(v, 0.f), yr, off, 0, 0);
            else
                __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(v), yr, off, 0, 0);
        }
    }
}

// ------------------------------------------------------------------------------------------------------ planner
// A plan: K splits S, rows per block R, row groups RG, tiles per wave NTW and the kernel's x-tile parameter MT (kgm_mt).
struct KgmPlan { int S, R, RG, NTW, MT; };
constexpr int KGM_MAX_NTW = 6;
// most tiles per wave of a type, x-tile parameter (kgm_mt) and row-group count whose units and scales fit the registers
// without spilling at 256 per lane (two row groups keep three stages of weights in flight, one group two); from the
// compiler's register counts of every instance:
//   per-value dequantization: Q4_K / Q4_0 at 33-64 rows 5, Q6_K from 17 rows 5, Q5_K 5 (4 at 33-48 rows);
//   factored products (9-32 rows): Q4_K / Q4_0 6 (5 at 17-32 rows with two row groups); Q5_K one row group 6 (4 at
//   17-32 rows), two row groups 4 (3);
//   diagonal x tiles: at 1-4 rows (x in registers, one row group) 6; at 5-8 rows Q4_K / Q4_0 6 (with two row groups
//   4 / 5), Q5_K 5 (4).
constexpr int kgm_max_ntw(int t, int mt, int rg) {
    const bool q5 = t == T_Q5KT, q4 = t == T_Q4KT || t == T_Q40T;
    if (mt == -1) return rg == 1 ? KGM_MAX_NTW : 0;                        // x in registers: one row group only
    if (mt < 0) return q5 ? (rg == 1 ? 5 : 4) : rg == 1 ? KGM_MAX_NTW : (t == T_Q4KT ? 4 : 5);
    const bool fact = (q4 || q5) && mt <= 2;
    if (q5) return fact ? (rg == 1 ? (mt == 1 ? KGM_MAX_NTW : 4) : (mt == 1 ? 4 : 3)) : (mt == 3 ? 4 : 5);
    if (q4) return fact ? (mt == 2 && rg == 2 ? 5 : KGM_MAX_NTW) : 5;
    if (t == T_Q6KT) return mt >= 2 ? 5 : KGM_MAX_NTW;
    return KGM_MAX_NTW;
}

// the kernel's x-tile parameter for M activation rows: 16-row x tiles (1-4), or for the nibble tiles at up to 8 rows
// -1 / -2: one or two sub-block-diagonal x tiles of 4 rows each (the kernel's DIAG path)
constexpr int kgm_mt(int t, int64_t M) {
    return (t == T_Q4KT || t == T_Q5KT || t == T_Q40T) && M <= 8 ? (M <= 4 ? -1 : -2) : (int)((M + 15) / 16);
}
constexpr int kgm_abs(int v) { return v < 0 ? -v : v; }

// the most 16-row tiles a wave touches: over the blocks' row ranges [rr R, min(N, rr R + R)) and their RG row groups
// (every range but the last is full, and a full range's row groups span tiles by their starts modulo 16, which repeat
// every 16 ranges: the first 16 ranges and the last cover every case)
static int kgm_ntw(int64_t N, int64_t R, int RG) {
    const int64_t ranges = (N + R - 1) / R, RQ = (R + RG - 1) / RG;
    int64_t most = 0;
    auto range = [&](int64_t rr) {
        const int64_t r0 = rr * R, r1 = std::min(N, r0 + R);
        for (int q = 0; q < RG; ++q) {
            const int64_t a = std::min(r1, r0 + q * RQ), b = std::min(r1, a + RQ);
            if (b > a) most = std::max(most, (b - 1) / 16 - a / 16 + 1);
        }
    };
    for (int64_t rr = 0; rr < std::min<int64_t>(ranges, 16); ++rr) range(rr);
    if (ranges > 16) range(ranges - 1);
    return (int)most;
}

// The plan of least estimated cost, in bytes a CU moves per block (its weights, the x of its K range, and for S > 1
// its partial tile written plus, for the last arriver, S partials read) plus the MFMA rows spent on rows outside the
// block's range and the K groups left idle in a block's last step, times the rounds of blocks the CUs run; the weights
// reflect MI355X timings of the 7 projections of a 27B-class layer at 64 rows against forced split counts, over S in
// {1, 2, 3, 4, 6, 8} (only `force_s` when it is set) and RG in {1, 2} (those whose x rings fit the LDS). Rows per block
// are chosen so that the ranges fill the CUs once, or, for a weight whose ranges would then hold more tiles than a
// wave's registers take (more than about 96 rows per CU), the CUs' share times the fewest rounds whose ranges fit;
// split plans keep their partials within the static scratch of mbq_matmul_noalloc. Q4_K tiles: a row's chunk is 64
// bytes of quants and half a 16-byte header, and a tile row outside the range costs its dequantization (the vector
// work of the whole row), not only its MFMA row.
static KgmPlan kgm_choose_mt(int t, int MTS, int64_t M, int64_t N, int64_t K, int cus, int force_s) {
    const int CW = kgm_cw(t);
    const int64_t KC = (K + CW - 1) / CW;
    const int MT = kgm_abs(MTS);
    const double wpc = t == T_Q4KT ? 72.0 : t == T_Q40T ? 72.0 : t == T_Q5KT ? 88.0 : t == T_Q6KT ? 105.0 : t == T_Q8T ? 68.0 : 64.0;
    const double waste_w = (t == T_Q4KT || t == T_Q5KT || t == T_Q6KT || t == T_Q40T) ? 1.5 : t == T_Q8T ? 1.0 : 0.5;
    KgmPlan best{0, 0, 0, 0, MTS};
    double best_cost = 0;
    for (int S : {1, 2, 3, 4, 6, 8}) {
        if (force_s > 0) S = force_s;
        if (KC >= S) {
            const int64_t share = std::max<int64_t>(1, cus / S);
            const int64_t kcs = (KC + S - 1) / S;
            for (int RG : {1, 2}) {
                const int KG = 8 / RG;
                if (kgm_ring(t, MT, RG) > KGM_LDS_MAX) continue;
                const int maxn = kgm_max_ntw(t, MTS, RG);
                if (maxn == 0) continue;
                if (MTS == -1 && (kcs + KG - 1) / KG > kgm_rx_chunks()) continue;       // the chunks x registers hold
                // the fewest rounds of `share` ranges whose row groups fit a wave's tiles (16 rows always do), from a
                // bound below it: a row group of RQ rows spans at least RQ / 16 tiles
                int64_t rounds = std::max<int64_t>(1, N / (share * RG * 16 * maxn)), R = 0;
                int ntw = 0;
                for (;; ++rounds) {
                    R = (N + share * rounds - 1) / (share * rounds);
                    ntw = kgm_ntw(N, R, RG);
                    if (ntw <= maxn || R <= 16) break;
                }
                if (ntw > maxn) continue;
                const int64_t ranges = (N + R - 1) / R;
                if (S > 1 && (ranges > SCRATCH_TILES ||
                              (size_t)ranges * S * RG * MT * ntw * 1024 > SCRATCH_BYTES)) continue;
                const double w = (double)R * kcs * wpc;                         // weight bytes
                // x bytes (L2 hits: half weight); diagonal x tiles move only the batch's rows
                const double x = 0.5 * (MTS < 0 ? (double)M : 16.0 * MT) * 2 * CW * kcs;
                // partial tile written, and S read by the last arriver at the end of its work (twice the weight), and
                // the exchange's dependent round trips (store and wait, arrival count, partial loads): about 4 us at
                // 1-16 rows, a CU's share of 96 KB (MI355X, K-group plans of a 27B-class layer forced to 1-8 splits)
                const double part = S > 1 ? (double)RG * MT * ntw * 1024 * (1 + 2 * S) + (M <= 16 ? 96e3 : 0.0) : 0.0;
                const double waste = waste_w * (double)std::max<int64_t>(0, RG * ntw * 16 - R) * kcs * wpc;
                const double idle = (double)((kcs + KG - 1) / KG * KG - kcs) / (double)kcs;
                const double blocks_per_cu = std::ceil((double)(ranges * S) / (double)cus);
                const double cost = (w + x + part + waste) * (1.0 + idle) * blocks_per_cu;
                if (best.S == 0 || cost < best_cost) {
                    best = KgmPlan{S, (int)R, RG, ntw, MTS};
                    best_cost = cost;
                }
            }
        }
        if (force_s > 0) break;
    }
    return best;
}

// The plan for M activation rows: x tiles kgm_mt(t, M), or, where x in registers (1-4 rows of the nibble tiles) holds
// too few chunks for any split (K above 40960), the two diagonal x tiles staged in LDS
static KgmPlan kgm_choose(int t, int64_t M, int64_t N, int64_t K, int cus, int force_s) {
    const int MTS = kgm_mt(t, M);
    KgmPlan p = kgm_choose_mt(t, MTS, M, N, K, cus, force_s);
    if (p.S == 0 && MTS == -1) p = kgm_choose_mt(t, -2, M, N, K, cus, force_s);
    return p;
}

// ------------------------------------------------------------------------------------------------------ launchers
template <int T, int MT, int RG, int NTW, bool KFULL>
static int kgm_launch(const Args& a, const KgmPlan& p, const Workspace& w, hipStream_t s) {
    if constexpr (kgm_ring(T, kgm_abs(MT), RG) > KGM_LDS_MAX || NTW > kgm_max_ntw(T, MT, RG)) {
        return set_error(MBQ_BAD_ARG, "K-group GEMM: no kernel of %d row groups x %d tiles at %d activation rows", RG, NTW,
                         MT < 0 ? -4 * MT : 16 * MT);
    } else {
        auto kern = kgemm_kernel<T, MT, RG, NTW, KFULL>;
        const size_t lds = kgm_lds<T, kgm_abs(MT), RG, NTW>();
        static std::atomic<uint64_t> lds_set{0};
        if (set_lds_limit((const void*)kern, lds, lds_set) != hipSuccess)
            return set_error(MBQ_LAUNCH_FAIL, "K-group GEMM: %zu bytes of LDS refused", lds);
        const int64_t KC = (a.K + kgm_cw(T) - 1) / kgm_cw(T);
        const int kcs = (int)((KC + p.S - 1) / p.S);
        KgmArgs g{a.base, a.stride, a.layer_dev, a.nlayers, a.sc_off, a.wbytes, a.hi_off, a.d_off, a.x, (int)a.M, (int)a.N, (int)a.K, a.y,
                  a.out_bf16, p.R, p.S, kcs, w.ws, w.cnt, (uint32_t)w.bytes, w.fenced};
        const int64_t ranges = (a.N + p.R - 1) / p.R;
        kern<<<dim3((unsigned)(ranges * p.S)), KGM_THREADS, lds, s>>>(g);
        const hipError_t e = hipGetLastError();
        if (e != hipSuccess) return set_error(MBQ_LAUNCH_FAIL, "K-group GEMM launch: %s", hipGetErrorString(e));
        return 0;
    }
}

template <int T, int MT, int RG, bool KFULL>
static int kgm_launch_ntw(const Args& a, const KgmPlan& p, const Workspace& w, hipStream_t s) {
    switch (p.NTW) {
        case 1: return kgm_launch<T, MT, RG, 1, KFULL>(a, p, w, s);
        case 2: return kgm_launch<T, MT, RG, 2, KFULL>(a, p, w, s);
        case 3: return kgm_launch<T, MT, RG, 3, KFULL>(a, p, w, s);
        case 4: return kgm_launch<T, MT, RG, 4, KFULL>(a, p, w, s);
        case 5: return kgm_launch<T, MT, RG, 5, KFULL>(a, p, w, s);
        case 6: return kgm_launch<T, MT, RG, 6, KFULL>(a, p, w, s);
    }
    return set_error(MBQ_BAD_ARG, "K-group GEMM: %d tiles per wave", p.NTW);
}

template <int T, int MT, bool KFULL>
static int kgm_launch_rg(const Args& a, const KgmPlan& p, const Workspace& w, hipStream_t s) {
    if (p.RG == 1) return kgm_launch_ntw<T, MT, 1, KFULL>(a, p, w, s);
    return kgm_launch_ntw<T, MT, 2, KFULL>(a, p, w, s);
}

template <int T, bool KFULL>
static int kgm_launch_mt(const Args& a, const KgmPlan& p, const Workspace& w, hipStream_t s) {
    if constexpr (T == T_Q4KT || T == T_Q5KT || T == T_Q40T) {
        if (p.MT == -1) return kgm_launch_rg<T, -1, KFULL>(a, p, w, s);
        if (p.MT == -2) return kgm_launch_rg<T, -2, KFULL>(a, p, w, s);
    }
    switch (p.MT) {
        case 1: return kgm_launch_rg<T, 1, KFULL>(a, p, w, s);
        case 2: return kgm_launch_rg<T, 2, KFULL>(a, p, w, s);
        case 3: return kgm_launch_rg<T, 3, KFULL>(a, p, w, s);
        case 4: return kgm_launch_rg<T, 4, KFULL>(a, p, w, s);
    }
    return set_error(MBQ_BAD_ARG, "K-group GEMM: x-tile parameter %d for type %d", p.MT, T);
}

// bytes of the partial tiles of a plan
static size_t kgm_ws_bytes(int64_t N, const KgmPlan& p) {
    const int64_t ranges = (N + p.R - 1) / p.R;
    return (size_t)ranges * p.S * p.RG * kgm_abs(p.MT) * p.NTW * 256 * 4;
}

int kgemm_plan(int t, const Args& a, int force_s, int* rows_per_block, int* splits) {
    const KgmPlan p = kgm_choose(t, a.M, a.N, a.K, cus_of_device(), force_s);
    if (p.S == 0) return set_error(MBQ_BAD_ARG, "K-group GEMM: no plan for %lld x %lld x %lld (%d splits)", (long long)a.M,
                                   (long long)a.N, (long long)a.K, force_s);
    *rows_per_block = p.R;
    *splits = p.S;
    return 0;
}

int launch_kgemm(int t, const Args& a, int force_s, hipStream_t s) {
    if (!tiled_type(t)) return set_error(MBQ_BAD_ARG, "K-group GEMM: type %d is not a tiled plane type", t);
    if (a.M < 1 || a.M > 64) return set_error(MBQ_BAD_ARG, "K-group GEMM: M = %lld", (long long)a.M);
    if (a.wbytes > BUF_MAX_BYTES || a.M * a.K * 2 > BUF_MAX_BYTES || a.M * a.N * 4 > BUF_MAX_BYTES)
        return set_error(MBQ_BAD_ARG, "K-group GEMM operands over 2 GiB");
    if ((t == T_Q4KT || t == T_Q5KT || t == T_Q6KT) && a.K % 256) return set_error(MBQ_BAD_ARG, "K-group GEMM: K-quant K = %lld", (long long)a.K);
    const KgmPlan p = kgm_choose(t, a.M, a.N, a.K, cus_of_device(), force_s);
    if (p.S == 0) return set_error(MBQ_BAD_ARG, "K-group GEMM: no plan for %lld x %lld x %lld (%d splits)", (long long)a.M,
                                   (long long)a.N, (long long)a.K, force_s);
    Workspace w;
    if (p.S > 1) {
        const int64_t ranges = (a.N + p.R - 1) / p.R;
        if (int rc = split_workspace(a, ranges, kgm_ws_bytes(a.N, p), s, &w)) return rc;
    }
    if (t == T_Q4KT) return kgm_launch_mt<T_Q4KT, true>(a, p, w, s);                  // K % 128 == 0
    if (t == T_Q6KT) return kgm_launch_mt<T_Q6KT, true>(a, p, w, s);
    if (t == T_Q5KT) return kgm_launch_mt<T_Q5KT, true>(a, p, w, s);
    if (t == T_Q40T) return a.K % 128 == 0 ? kgm_launch_mt<T_Q40T, true>(a, p, w, s) : kgm_launch_mt<T_Q40T, false>(a, p, w, s);
    if (t == T_Q8T) return a.K % 64 == 0 ? kgm_launch_mt<T_Q8T, true>(a, p, w, s) : kgm_launch_mt<T_Q8T, false>(a, p, w, s);
    return a.K % 64 == 0 ? kgm_launch_mt<T_I8T, true>(a, p, w, s) : kgm_launch_mt<T_I8T, false>(a, p, w, s);
}

}  // namespace mbq
