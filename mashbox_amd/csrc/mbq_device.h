// Device helpers shared by the gfx950 kernels (vector types, exact conversions, Q4_K scale unpack, wave sums).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "mbq_layout.h"

namespace mbq {

typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

// ----------------------------------------------------------------------------------------------------- helpers
__device__ __forceinline__ u32x4 ld16(const void* p) { return *reinterpret_cast<const u32x4*>(p); }
__device__ __forceinline__ void st16(void* p, u32x4 v) { *reinterpret_cast<u32x4*>(p) = v; }

// fp16 bits -> float32, exact (subnormal, inf and NaN kept): reference src/mashbox/ops/reference.py:49-51
__device__ __forceinline__ float f16f(uint32_t h) { return (float)__builtin_bit_cast(_Float16, (uint16_t)(h & 0xFFFFu)); }

// float32 -> bfloat16 bits, round to nearest even; NaN stays NaN (quiet). One v_cvt_pk_bf16_f32: on every one of the
// 2^32 inputs it gives the bits of the integer form bf16_bits_int (mbq_probe_bf16 checks that on the device at hand;
// on MI355X no input differs), where the integer form's branch for NaN cost about 20 instructions per value.
__device__ __forceinline__ uint32_t bf16_bits_int(float f) {
    const uint32_t u = __float_as_uint(f);
    if ((u & 0x7FFFFFFFu) > 0x7F800000u) return (u >> 16) | 0x40u;
    return (u + 0x7FFFu + ((u >> 16) & 1u)) >> 16;
}
__device__ __forceinline__ uint32_t bf16_bits(float f) {
    const bf16x2_t p = {(__bf16)f, (__bf16)0.f};
    return __builtin_bit_cast(uint32_t, p) & 0xFFFFu;
}

__device__ __forceinline__ float dot2(uint32_t a, uint32_t b, float c) {
    return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, a), __builtin_bit_cast(bf16x2_t, b), c, false);
}

// Q4_K unit dword -> bfloat16 pair (128 + q[8t+2p], 128 + q[8t+2p+1]); exact (mbq_layout.h)
__device__ __forceinline__ uint32_t nib_pair(uint32_t w, int p) { return ((w >> (4 * p)) & 0x000F000Fu) | 0x43004300u; }

// Q6_K unit (mbq_layout.h): the 6-bit quants of values 8t .. 8t+3 (*lo) and 8t+4 .. 8t+7 (*hi) as the bytes of two
// dwords, from dword t of the low-nibble plane (ql) and dword t / 2 of the high-bit plane (qh)
__device__ __forceinline__ void q6k_bytes(uint32_t ql, uint32_t qh, int t, uint32_t* lo, uint32_t* hi) {
    const uint32_t m = 0x30303030u;
    const uint32_t h0 = (t & 1) ? (qh & m) : ((qh << 4) & m);
    const uint32_t h1 = (t & 1) ? ((qh >> 2) & m) : ((qh << 2) & m);
    *lo = (ql & 0x0F0F0F0Fu) | h0;
    *hi = ((ql >> 4) & 0x0F0F0F0Fu) | h1;
}

// Q5_K unit (mbq_layout.h): the 5-bit quants of values 8t .. 8t+3 (*lo) and 8t+4 .. 8t+7 (*hi) as the bytes of two
// dwords, from dword t of the low-nibble plane (ql) and the unit's high-bit dword (qh): a rotate brings bit 2t (2t + 1)
// of every qh byte to bit 4, and a bit-field insert joins it to the low nibbles
__device__ __forceinline__ void q5k_bytes(uint32_t ql, uint32_t qh, int t, uint32_t* lo, uint32_t* hi) {
    const uint32_t m = 0x10101010u;
    const uint32_t a = __builtin_amdgcn_alignbit(qh, qh, (uint32_t)(2 * t + 28) & 31u);
    const uint32_t b = __builtin_amdgcn_alignbit(qh, qh, (uint32_t)(2 * t + 29) & 31u);
    *lo = (a & m) | (ql & 0x0F0F0F0Fu);
    *hi = (b & m) | ((ql >> 4) & 0x0F0F0F0Fu);
}

// bytes 2p, 2p+1 (each < 128) of w -> bfloat16 pair (128 + byte, 128 + byte'), exact: one byte permute against the
// exponent byte 0x43 held in every byte of c43
__device__ __forceinline__ uint32_t b128_pair(uint32_t w, uint32_t c43, int p) {
    return __builtin_amdgcn_perm(c43, w, p ? 0x04030402u : 0x04010400u);
}

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

// the factor a kernel applies to output row n's float32 sum: the int8 per-row scale (T_INT8: the caller's scale array;
// T_I8T: the planes' scale plane of the weight read, base + lo its first byte), else 1
template <int T>
__device__ __forceinline__ float row_scale(const float* srow, const uint8_t* wbase, int64_t sc_off, int n) {
    if constexpr (T == T_INT8) return srow[n];
    else if constexpr (T == T_I8T) return reinterpret_cast<const float*>(wbase + sc_off)[n];
    else return 1.f;
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

// buffer resources: loads carry a 32-bit per-lane offset and a scalar offset, and read zero past num_records
typedef __amdgpu_buffer_rsrc_t rsrc_t;
// A buffer-load offset beyond every buffer this library addresses (their byte ranges are at most BUF_MAX_BYTES, checked
// by each launcher): the load returns zero without touching memory. With a scalar offset below 2^31 the sum cannot wrap.
constexpr uint32_t OOB_VOFF = 0x7FFFFFF0u;
__device__ __forceinline__ rsrc_t make_rsrc(const void* p, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p), (short)0, (int)bytes, 0x00020000);
}
__device__ __forceinline__ u32x4 bload16(rsrc_t r, uint32_t voff, uint32_t soff) {
    return __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(r, voff, soff, 0));
}
__device__ __forceinline__ uint32_t bload2(rsrc_t r, uint32_t voff, uint32_t soff) {
    return (uint32_t)__builtin_amdgcn_raw_buffer_load_b16(r, voff, soff, 0);
}

// 16 bytes per lane from global memory straight into LDS (buffer_load ... lds): lane l writes lds_wave + 16 l
// (lds_wave wave-uniform); it counts in vmcnt like a load
__device__ __forceinline__ void dma16(rsrc_t r, uint16_t* lds_wave, uint32_t voff, uint32_t soff) {
    __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (__attribute__((address_space(3))) void*)lds_wave, 16, voff, soff, 0, 0);
}

// s_waitcnt vmcnt(N), expcnt and lgkmcnt not waited (gfx9 encoding: vmcnt bits 3:0 and 15:14)
template <int N>
__device__ __forceinline__ void wait_vm() {
    static_assert(N >= 0 && N < 64, "vmcnt range");
    __builtin_amdgcn_s_waitcnt((N & 15) | 0x0F70 | ((N >> 4) << 14));
}

// s_waitcnt lgkmcnt(0) (vmcnt and expcnt not waited): a wave's own LDS writes have completed. A barrier does not wait
// for them (the AMDGPU memory model releases LDS writes at workgroup scope with this wait), so a wave that writes LDS
// for other waves waits for its writes before it passes the barrier they wait at (measured on MI355X: without it,
// dequantized weight chunks written just before a barrier were read stale by the waves past it)
__device__ __forceinline__ void wait_lgkm0() { __builtin_amdgcn_s_waitcnt(0xC07F); }

// Workgroup barrier without the memory fence of __syncthreads, which waits for every load in flight (LDS DMA
// included) and so empties a load pipeline at each step. The caller has waited (vmcnt) for the loads whose LDS writes
// the other waves read after the barrier, and (wait_lgkm0) for its own LDS writes that they read; the empty asm
// statements keep the compiler from moving memory accesses across.
__device__ __forceinline__ void barrier_nofence() {
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
}

constexpr uint32_t BF16_ONES = 0x3F803F80u;  // bfloat16 pair (1, 1)

// a value the compiler treats as unknown, so that it keeps one AND of a two-quant mask instead of splitting it per byte
__device__ __forceinline__ uint32_t opaque(uint32_t v) {
    asm volatile("" : "+v"(v));
    return v;
}

// v_mfma_f32_16x16x32_bf16 on an accumulator pinned to accumulation registers and updated in place. For kernels whose
// accumulators fill the accumulation registers: the compiler's own MFMA there writes its result to other registers
// than its accumulator input and copies the accumulators back every iteration. The compiler sees an opaque
// instruction, so the asm pads on entry the hazard such kernels meet (2 wait states after a VALU write of an A or B
// operand register), and a kernel must wait out the last MFMA (mfma_drain) before its VALU instructions read the
// accumulators, and must not leave conditional blocks between these MFMAs (the compiler may move accumulators between
// registers at block boundaries, right after an MFMA that is still writing them).
__device__ __forceinline__ void mfma_acc(f32x4_t& acc, const bf16x8_t& a, const bf16x8_t& b) {
    asm("s_nop 1\n\tv_mfma_f32_16x16x32_bf16 %0, %1, %2, %0" : "+a"(acc) : "v"(a), "v"(b));
}

// the same with the accumulator in (arch) vector registers, for kernels whose accumulators exceed the accumulation
// registers of their occupancy (the compiler splits a wave's registers evenly between the two files)
__device__ __forceinline__ void mfma_accv(f32x4_t& acc, const bf16x8_t& a, const bf16x8_t& b) {
    asm("s_nop 1\n\tv_mfma_f32_16x16x32_bf16 %0, %1, %2, %0" : "+v"(acc) : "v"(a), "v"(b));
}

// v_mfma_f32_32x32x16_bf16, the same two forms. Lane l: A row l % 32, B column l % 32, both K values 8 (l / 32) .. +7;
// accumulator element 4 i + r is row 8 i + 4 (l / 32) + r, column l % 32 (checked on MI355X).
__device__ __forceinline__ void mfma32_acc(f32x16_t& acc, const bf16x8_t& a, const bf16x8_t& b) {
    asm("s_nop 1\n\tv_mfma_f32_32x32x16_bf16 %0, %1, %2, %0" : "+a"(acc) : "v"(a), "v"(b));
}
__device__ __forceinline__ void mfma32_accv(f32x16_t& acc, const bf16x8_t& a, const bf16x8_t& b) {
    asm("s_nop 1\n\tv_mfma_f32_32x32x16_bf16 %0, %1, %2, %0" : "+v"(acc) : "v"(a), "v"(b));
}

// 24 wait states: the last mfma_acc / mfma32_acc (16 passes) has written its accumulator before the next instruction
// reads it
__device__ __forceinline__ void mfma_drain() {
    __builtin_amdgcn_sched_barrier(0);
    asm volatile("s_nop 7\n\ts_nop 7\n\ts_nop 7" ::: "memory");
    __builtin_amdgcn_sched_barrier(0);
}

// Split-K partial exchange between the blocks of a tile, by the MI355X memory model at agent scope. The blocks that
// store a partial release it before their arrival atomic: buffer_wbl2 sc1 writes the XCD's L2 dirty lines back, and
// the s_waitcnt vmcnt(0) that follows waits for it and for the stores. The last block acquires before it reads the
// partials: buffer_inv sc1 drops its XCD's L2 lines, which another XCD may have written since. Device-coherent (sc1)
// stores and loads alone do not order this: a partial can still be dirty in the writer's L2 when the last block reads
// it from memory (seen on MI355X as stale 64-byte sectors of a partial).
__device__ __forceinline__ void split_release() { __builtin_amdgcn_fence(__ATOMIC_RELEASE, "agent"); }
__device__ __forceinline__ void split_acquire() { __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent"); }

// v as a register value the compiler cannot look through (so byte extracts stay register ops on it), without the
// ordering constraints of a volatile asm
__device__ __forceinline__ uint32_t hide(uint32_t v) {
    asm("" : "+v"(v));
    return v;
}

// two float32 -> bfloat16 pair (lo, hi), round to nearest even (v_cvt_pk_bf16_f32)
__device__ __forceinline__ uint32_t pack_bf16(float lo, float hi) {
    const bf16x2_t p = {(__bf16)lo, (__bf16)hi};
    return __builtin_bit_cast(uint32_t, p);
}

}  // namespace mbq
