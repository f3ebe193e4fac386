// Weight-direct MFMA operands, shared by the GEMMs that take their weights from HBM straight into registers
// (mbq_wsgemm.hip): one iteration = KI values of K (64 for int8 and Q8_0, 128 for Q4_0 and the
// K-quants), 64 contiguous bytes of each row of the quant plane (tiled int8 planes: the 16 rows' 64 bytes are one
// contiguous KiB). Lane l holds 16 bytes of row (l & 15) of a 16-row tile at byte 16 g
// (g = l >> 4, the lane group). The MFMA sums over K, so any K order works when x follows it: in K step s of an
// iteration, lane group g holds the 8 values K = k0 + g KI/4 + 8 s + e (e = 0..7) for both operands.
//   int8   16 quants = 2 K steps; bf16(q) is exact; the per-row scale multiplies the float32 sum in the epilogue.
//   Q8_0   16 quants of block (k0 + 16 g) / 32; the B operand is q * d (exact in float32) rounded to nearest even
//          bfloat16, the value the LDS GEMM stores.
//   Q4_K   one 16-byte unit = the 32 quants of sub-block k0/32 + g = 4 K steps; the B operand is (d sc) q - dmin m
//          (exact in float32) rounded to nearest even bfloat16.
//   Q4_0   one 16-byte unit = the 32 quants of block k0/32 + g (the Q4_K order); the B operand is d (q - 8) (exact in
//          float32) rounded to nearest even bfloat16.
//   Q5_K   the same 32 values: 16 bytes of low nibbles, the 4-byte high-bit word and the super-block's scales; the B
//          operand is (d sc) q - dmin m (one rounding) rounded to nearest even bfloat16.
//   Q6_K   the same 32 values: 16 bytes of low nibbles, 8 bytes of high bits, the two 16-value scales and the
//          super-block scale; the B operand is (d sc) (q - 32) (exact in float32) rounded to nearest even bfloat16.
// Weights: reference src/mashbox/ops/reference.py:66-70 (Q4_0), :101-103 (Q8_0), :132-149 (Q4_K), :150-159 (Q5_K), :164-173 (Q6_K); plane layouts:
// mbq_layout.h.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "mbq_device.h"
#include "mbq_layout.h"

namespace mbq {

template <int T> constexpr int ws_ki() { return unit32(T) ? 128 : 64; }
inline int ws_ki_of(int t) { return unit32(t) ? 128 : 64; }

// raw bytes of one iteration of one 16-row tile, as one lane holds them
template <int T> struct WsRaw;
template <> struct WsRaw<T_INT8> { u32x4 q; };
template <> struct WsRaw<T_I8T> { u32x4 q; };
template <> struct WsRaw<T_Q8_0> { u32x4 q; uint32_t d; };
template <> struct WsRaw<T_Q4_K> { u32x4 q, meta; };
template <> struct WsRaw<T_Q4_0> { u32x4 q; uint32_t d; };
template <> struct WsRaw<T_Q6_K> { u32x4 q; u32x2 h; uint32_t s, d; };
template <> struct WsRaw<T_Q5_K> { u32x4 q, meta; uint32_t h; };
template <int T> constexpr int ws_wloads() { return int8_type(T) ? 1 : T == T_Q6_K ? 4 : T == T_Q5_K ? 3 : 2; }   // buffer loads per tile per iteration

// per-lane byte offsets of one weight row's planes (the iteration's part goes in the scalar offset)
struct WsOff { uint32_t q, s, h, d; };
template <int T>
__device__ __forceinline__ WsOff ws_off(uint32_t row, int K, int lg, int64_t sc_off, int64_t hi_off, int64_t d_off) {
    WsOff o{row * (uint32_t)(unit32(T) ? K / 2 : K) + 16u * lg, 0u, 0u, 0u};
    if constexpr (T == T_I8T) o.q = (uint32_t)i8t_off(row, K, 0) + 16u * lg;          // one contiguous KiB per tile
    if constexpr (T == T_Q8_0) o.s = (uint32_t)sc_off + row * (uint32_t)(K / 32) * 2u + 2u * (lg >> 1);
    if constexpr (T == T_Q4_0) o.s = (uint32_t)sc_off + row * (uint32_t)(K / 32) * 2u + 2u * lg;
    if constexpr (T == T_Q4_K || T == T_Q5_K) o.s = (uint32_t)sc_off + row * (uint32_t)(K / 256) * 16u;
    if constexpr (T == T_Q5_K) o.h = (uint32_t)hi_off + row * (uint32_t)(K / 8) + 4u * lg;
    if constexpr (T == T_Q6_K) {
        o.s = (uint32_t)sc_off + row * (uint32_t)(K / 16) + 2u * lg;
        o.h = (uint32_t)hi_off + row * (uint32_t)(K / 4) + 8u * lg;
        o.d = (uint32_t)d_off + row * (uint32_t)(K / 256) * 2u;
    }
    return o;
}

// the lane's bytes of the iteration at K offset kk (non-temporal quant loads); with KFULL false a Q4_0 / Q8_0 block
// past K gets scale 0 (the x it meets is zero, its quants may be any bytes)
template <int T, bool KFULL>
__device__ __forceinline__ void ws_load(WsRaw<T>& w, rsrc_t wr, const WsOff& o, int kk, int K, int lg) {
    const uint32_t qk = T == T_I8T ? (uint32_t)kk * 16u : (uint32_t)(unit32(T) ? kk / 2 : kk);   // T_I8T: KiB per 64 values
    w.q = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(wr, o.q, qk, 2));
    if constexpr (T == T_Q8_0) {
        w.d = bload2(wr, o.s, (uint32_t)(kk / 32) * 2u);
        if constexpr (!KFULL) w.d = (kk + 16 * lg < K) ? w.d : 0u;
    }
    if constexpr (T == T_Q4_0) {
        w.d = bload2(wr, o.s, (uint32_t)(kk / 32) * 2u);
        if constexpr (!KFULL) w.d = (kk + 32 * lg < K) ? w.d : 0u;
    }
    if constexpr (T == T_Q4_K || T == T_Q5_K) w.meta = bload16(wr, o.s, (uint32_t)(kk / 256) * 16u);
    if constexpr (T == T_Q5_K) w.h = (uint32_t)__builtin_amdgcn_raw_buffer_load_b32(wr, o.h, (uint32_t)(kk / 8), 2);
    if constexpr (T == T_Q6_K) {
        w.h = __builtin_bit_cast(u32x2, __builtin_amdgcn_raw_buffer_load_b64(wr, o.h, (uint32_t)(kk / 4), 2));
        w.s = bload2(wr, o.s, (uint32_t)(kk / 16));
        w.d = bload2(wr, o.d, (uint32_t)(kk / 256) * 2u);
    }
}

// per-lane dequant constants of one tile's unit
// Q8_0: d; Q4_K, Q5_K: d*sc, dmin*m, d*sc/16; Q4_0: d, 8 d, d/16; Q6_K: d*sc0, 32 d*sc0, d*sc1, 32 d*sc1
struct WsScale { float a, b, c, e; };

template <int T>
__device__ __forceinline__ WsScale ws_scale(const WsRaw<T>& w, int j) {
    WsScale s{1.f, 0.f, 0.f, 0.f};
    if constexpr (T == T_Q6_K) {
        const float d = f16f(w.d);
        s.a = d * (float)(int8_t)(w.s & 0xFFu);           // exact
        s.b = 32.f * s.a;
        s.c = d * (float)(int8_t)((w.s >> 8) & 0xFFu);
        s.e = 32.f * s.c;
    } else if constexpr (T == T_Q8_0) {
        s.a = f16f(w.d);
    } else if constexpr (T == T_Q4_0) {
        s.a = f16f(w.d);
        s.b = 8.f * s.a;                            // q d - 8 d = (q - 8) d, exact in float32
        s.c = s.a * 0.0625f;
    } else if constexpr (T == T_Q4_K || T == T_Q5_K) {
        uint32_t sc, mn;
        q4k_scale_min_sel(w.meta[1], w.meta[2], w.meta[3], q4k_sel(j), &sc, &mn);
        s.a = f16f(w.meta[0]) * (float)sc;          // exact
        s.b = f16f(w.meta[0] >> 16) * (float)mn;    // exact
        s.c = s.a * 0.0625f;                        // exact: a power-of-two scale
    }
    return s;
}

// dword p (0..3) of the B operand of K step s: bfloat16 values 2p, 2p + 1 of the lane's 8 (s, p constants once the
// caller's loops are unrolled); each dword is independent of the others, so a caller can spread them between MFMAs
template <int T>
__device__ __forceinline__ uint32_t ws_bpair(const WsRaw<T>& w, const WsScale& sc, int s, int p) {
    if constexpr (T == T_Q6_K) {
        // values 8s .. 8s+3 (p = 0, 1) and 8s+4 .. 8s+7 (p = 2, 3) of the unit as bytes; (q - 32) (d sc) is one exact FMA
        uint32_t lo, hi;
        q6k_bytes(w.q[s], w.h[s >> 1], s, &lo, &hi);
        const uint32_t v = p < 2 ? lo : hi;
        const int sh = (p & 1) * 16;
        const float ds = s < 2 ? sc.a : sc.c, m = s < 2 ? sc.b : sc.e;
        return pack_bf16(__builtin_fmaf((float)((v >> sh) & 0xFFu), ds, -m), __builtin_fmaf((float)((v >> (sh + 8)) & 0xFFu), ds, -m));
    } else if constexpr (T == T_Q5_K) {
        // values 8s .. 8s+3 (p = 0, 1) and 8s+4 .. 8s+7 (p = 2, 3) of the unit as bytes; (d sc) q - dmin m is one FMA
        uint32_t lo, hi;
        q5k_bytes(w.q[s], w.h, s, &lo, &hi);
        const uint32_t v = p < 2 ? lo : hi;
        const int sh = (p & 1) * 16;
        return pack_bf16(__builtin_fmaf((float)((v >> sh) & 0xFFu), sc.a, -sc.b), __builtin_fmaf((float)((v >> (sh + 8)) & 0xFFu), sc.a, -sc.b));
    } else if constexpr (nib4(T)) {
        // dword s of the unit: quant 8s+2p in bits 4p..4p+3, quant 8s+2p+1 in bits 16+4p.. (mbq_layout.h); the odd
        // nibble positions come out 16 times too large and take the scale d*sc/16
        const uint32_t v = w.q[s];
        if (p == 0) {
            const uint32_t m = opaque(v & 0x000F000Fu);
            return pack_bf16(__builtin_fmaf((float)(m & 0xFFu), sc.a, -sc.b), __builtin_fmaf((float)((m >> 16) & 0xFFu), sc.a, -sc.b));
        } else if (p == 1) {
            const uint32_t m = opaque(v & 0x00F000F0u);
            return pack_bf16(__builtin_fmaf((float)(m & 0xFFu), sc.c, -sc.b), __builtin_fmaf((float)((m >> 16) & 0xFFu), sc.c, -sc.b));
        } else if (p == 2) {
            const uint32_t m = opaque(v & 0x0F000F00u);
            return pack_bf16(__builtin_fmaf((float)((m >> 8) & 0xFFu), sc.a, -sc.b), __builtin_fmaf((float)(m >> 24), sc.a, -sc.b));
        } else {
            const uint32_t m = opaque(v & 0xF000F000u);
            return pack_bf16(__builtin_fmaf((float)((m >> 8) & 0xFFu), sc.c, -sc.b), __builtin_fmaf((float)(m >> 24), sc.c, -sc.b));
        }
    } else {
        // 16 quants = dwords 2s, 2s + 1 of K step s; q * d is exact in float32 (at most 19 significant bits)
        const uint32_t v = hide(w.q[2 * s + (p >> 1)]);
        const int sh = (p & 1) * 16;
        float f0 = (float)(int8_t)((v >> sh) & 0xFFu), f1 = (float)(int8_t)((v >> (sh + 8)) & 0xFFu);
        if constexpr (T == T_Q8_0) f0 *= sc.a, f1 *= sc.a;
        return pack_bf16(f0, f1);
    }
}

// The 8 values of one Q4_K unit dword (quant 2p in bits 4p..4p+3, quant 2p+1 in bits 16+4p..: mbq_layout.h) as the
// bfloat16 B operand (d sc) q - dmin m, the values of ws_bop<T_Q4_K> bit for bit with two masks per dword instead of
// four: v & 0x0F0F0F0F leaves bytes (q0, q4, q1, q5), v & 0xF0F0F0F0 bytes (16 q2, 16 q6, 16 q3, 16 q7), which take
// the scale d sc / 16
__device__ __forceinline__ bf16x8_t q4k_dword_bop(uint32_t v, const WsScale& sc) {
    const uint32_t lo = opaque(v & 0x0F0F0F0Fu), hi = opaque(v & 0xF0F0F0F0u);
    auto f = [](uint32_t w, int b) { return (float)((w >> (8 * b)) & 0xFFu); };
    const u32x4 o{pack_bf16(__builtin_fmaf(f(lo, 0), sc.a, -sc.b), __builtin_fmaf(f(lo, 2), sc.a, -sc.b)),
                  pack_bf16(__builtin_fmaf(f(hi, 0), sc.c, -sc.b), __builtin_fmaf(f(hi, 2), sc.c, -sc.b)),
                  pack_bf16(__builtin_fmaf(f(lo, 1), sc.a, -sc.b), __builtin_fmaf(f(lo, 3), sc.a, -sc.b)),
                  pack_bf16(__builtin_fmaf(f(hi, 1), sc.c, -sc.b), __builtin_fmaf(f(hi, 3), sc.c, -sc.b))};
    return __builtin_bit_cast(bf16x8_t, o);
}

// B operand of K step s: the 8 values of the lane's row, as bfloat16
template <int T>
__device__ __forceinline__ bf16x8_t ws_bop(const WsRaw<T>& w, const WsScale& sc, int s) {
    const u32x4 o{ws_bpair<T>(w, sc, s, 0), ws_bpair<T>(w, sc, s, 1), ws_bpair<T>(w, sc, s, 2), ws_bpair<T>(w, sc, s, 3)};
    return __builtin_bit_cast(bf16x8_t, o);
}

}  // namespace mbq
