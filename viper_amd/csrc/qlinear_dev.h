// Device helpers shared by the gfx950 quantized-linear kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#include "viper_qlinear.h"

namespace vq {

typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));

constexpr int NT = 256;            // threads per workgroup (generic kernels)
constexpr int CPL = 8;             // chunk slots per lane per row segment (generic kernel)
constexpr int LDS_MAX = 65536;     // dynamic LDS budget per workgroup

template <int F> struct Fmt;
// G: quantization group, OFF: offset of the stored code, CK: weights per
// 16-byte chunk of the main plane, HIW: u32 high-plane words per chunk.
template <> struct Fmt<4> { static constexpr int G = 64, OFF = 8, CK = 32, HIW = 0; };
template <> struct Fmt<5> { static constexpr int G = 64, OFF = 16, CK = 32, HIW = 1; };
template <> struct Fmt<6> { static constexpr int G = 64, OFF = 32, CK = 32, HIW = 2; };
template <> struct Fmt<8> { static constexpr int G = 32, OFF = 0, CK = 16, HIW = 0; };

// ---------------------------------------------------------------- helpers

constexpr int DPP_SWAP1 = 0xB1;        // quad_perm [1,0,3,2]
constexpr int DPP_SWAP2 = 0x4E;        // quad_perm [2,3,0,1]
constexpr int DPP_HALF_MIRROR = 0x141; // lane i <- 7-i within 8
constexpr int DPP_MIRROR = 0x140;      // lane i <- 15-i within 16

template <int CTRL>
__device__ __forceinline__ int dpp_i(int v) {
    return __builtin_amdgcn_mov_dpp(v, CTRL, 0xF, 0xF, true);
}
template <int CTRL>
__device__ __forceinline__ float dpp_f(float v) {
    return __int_as_float(dpp_i<CTRL>(__float_as_int(v)));
}

__device__ __forceinline__ float bf16f(uint32_t h) { return __uint_as_float(h << 16); }
__device__ __forceinline__ float f16f(uint32_t h) {
    return (float)__builtin_bit_cast(_Float16, (uint16_t)h);
}
// fp32 -> bf16, round to nearest even, NaN kept quiet with its top payload
// bits.  The arithmetic statement is f2bf_sw; the kernels use gfx950's
// v_cvt_pk_bf16_f32 (two values per instruction where the caller has two),
// which equals f2bf_sw on all 2^32 inputs (viper_hip_check_bf16_rounding
// checks that exhaustively on the device).
__device__ __forceinline__ uint16_t f2bf_sw(float f) {
    uint32_t u = __float_as_uint(f);
    if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40u);
    u += 0x7fffu + ((u >> 16) & 1u);
    return (uint16_t)(u >> 16);
}
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef float f32x2_t __attribute__((ext_vector_type(2)));
// {bf16(a), bf16(b)} packed as (a in the low half): one v_cvt_pk_bf16_f32
__device__ __forceinline__ uint32_t f2bf2(float a, float b) {
    return __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2_t){a, b}, bf16x2_t));
}
__device__ __forceinline__ uint16_t f2bf(float f) { return (uint16_t)f2bf2(f, 0.0f); }
__device__ __forceinline__ int sdot4(uint32_t a, uint32_t b, int c) {
    return __builtin_amdgcn_sdot4((int)a, (int)b, c, false);
}
// Low bytes of four words -> one packed word [a0, b0, c0, d0].
__device__ __forceinline__ uint32_t bytes4(uint32_t a, uint32_t b, uint32_t c, uint32_t d) {
    const uint32_t ab = __builtin_amdgcn_perm(b, a, 0x0c0c0400u);
    const uint32_t cd = __builtin_amdgcn_perm(d, c, 0x0c0c0400u);
    return __builtin_amdgcn_perm(cd, ab, 0x05040100u);
}

// Max / sum over the LANES (2, 4 or 8; sums 4 or 8) consecutive lanes that
// hold one group.
template <int LANES>
__device__ __forceinline__ float group_max(float v) {
    v = fmaxf(v, dpp_f<DPP_SWAP1>(v));
    if constexpr (LANES >= 4) v = fmaxf(v, dpp_f<DPP_SWAP2>(v));
    if constexpr (LANES == 8) v = fmaxf(v, dpp_f<DPP_HALF_MIRROR>(v));
    return v;
}
template <int LANES>
__device__ __forceinline__ int group_sum(int v) {
    v += dpp_i<DPP_SWAP1>(v);
    v += dpp_i<DPP_SWAP2>(v);
    if constexpr (LANES == 8) v += dpp_i<DPP_HALF_MIRROR>(v);
    return v;
}

// Sum over a team of TS consecutive lanes; every lane of the team gets it.
template <int TS>
__device__ __forceinline__ float team_sum(float v) {
    if constexpr (TS >= 2) v += dpp_f<DPP_SWAP1>(v);
    if constexpr (TS >= 4) v += dpp_f<DPP_SWAP2>(v);
    if constexpr (TS >= 8) v += dpp_f<DPP_HALF_MIRROR>(v);
    if constexpr (TS >= 16) v += dpp_f<DPP_MIRROR>(v);
    if constexpr (TS >= 32) v += __shfl_xor(v, 16, 64);
    if constexpr (TS >= 64) v += __shfl_xor(v, 32, 64);
    return v;
}

// Logical block of workgroup b in a grid of g: the dispatcher deals
// workgroups to the 8 XCDs in turn (b -> XCD b % 8), so numbering the
// blocks XCD by XCD gives each XCD one contiguous range of output rows.  Its
// y stores then fill whole cache lines of one L2 instead of sharing lines
// with the neighbouring XCDs (M = 1 north star 4.07 -> 4.03 us).  Any g works: XCD
// k holds g / 8 blocks, one more when k < g % 8.  The mapping only permutes
// blocks, so results do not depend on how the hardware deals them.
__device__ __forceinline__ int xcd_block(int b, int g) {
    const int k = b & 7;
    return k * (g >> 3) + min(k, g & 7) + (b >> 3);
}

// Workgroup barrier that orders LDS only: the weight loads still in flight
// are not waited for (a full __syncthreads() would drain them first).
__device__ __forceinline__ void lds_barrier() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

// silu(g) * u as the swiglu producers compute it: g * rcp(1 + exp(-g)) * u with
// the hardware exp and reciprocal (each within 1 ulp; the reference computes
// g / (1 + __expf(-g)) * u under fast math, swiglu_quantize.cu:39-41).  The
// bf16-rounded result stays within one bf16 ulp of the IEEE-divide value.
__device__ __forceinline__ float silu_mul(float g, float u) {
    return g * __builtin_amdgcn_rcpf(1.0f + __expf(-g)) * u;
}

// ------------------------------------------------------------- quantizer

constexpr float RND_MAGIC = 12582912.0f;  // 1.5 * 2^23

// Bits of RNE(x/s) + 1.5*2^23: the low byte is the quantized int8.
__device__ __forceinline__ uint32_t qbits(float x, float s, float r) {
    const float q0 = __fmul_rn(x, r);
    const float e = __builtin_fmaf(-q0, s, x);
    const float q1 = __builtin_fmaf(e, r, q0);
    return __float_as_uint(__fadd_rn(q1, RND_MAGIC));
}

// s = max(amax / 127, 1e-8) exactly (it is the stored activation scale); r
// the hardware reciprocal of s: the correction step in qbits still gives the
// exact RNE(x / s) for every finite bf16 pair (amax, x), as the device
// self-check shows exhaustively (10 VALU per group fewer than an IEEE 1 / s).
__device__ __forceinline__ void group_scale(float amax, float& s, float& r) {
    s = fmaxf(amax / 127.0f, 1e-8f);
    r = __builtin_amdgcn_rcpf(s);
}

// Quantize the 8 bf16 values of one octet (k = 8o..8o+7).  PERM stores them
// as [k even | k odd] (the nibble formats' dot order), else in k order.  The
// G/8 lanes of a group must call this together (DPP max over the group).
template <int G, bool PERM>
__device__ __forceinline__ void quantize_octet(const u32x4& v, uint32_t& d0, uint32_t& d1, float& s) {
    const float f0 = bf16f(v.x & 0xffffu), f1 = bf16f(v.x >> 16);
    const float f2 = bf16f(v.y & 0xffffu), f3 = bf16f(v.y >> 16);
    const float f4 = bf16f(v.z & 0xffffu), f5 = bf16f(v.z >> 16);
    const float f6 = bf16f(v.w & 0xffffu), f7 = bf16f(v.w >> 16);
    float a = fmaxf(fmaxf(fmaxf(fabsf(f0), fabsf(f1)), fmaxf(fabsf(f2), fabsf(f3))),
                    fmaxf(fmaxf(fabsf(f4), fabsf(f5)), fmaxf(fabsf(f6), fabsf(f7))));
    a = group_max<G / 8>(a);
    float r;
    group_scale(a, s, r);
    const uint32_t t0 = qbits(f0, s, r), t1 = qbits(f1, s, r), t2 = qbits(f2, s, r),
                   t3 = qbits(f3, s, r), t4 = qbits(f4, s, r), t5 = qbits(f5, s, r),
                   t6 = qbits(f6, s, r), t7 = qbits(f7, s, r);
    if constexpr (PERM) {
        d0 = bytes4(t0, t2, t4, t6);
        d1 = bytes4(t1, t3, t5, t7);
    } else {
        d0 = bytes4(t0, t1, t2, t3);
        d1 = bytes4(t4, t5, t6, t7);
    }
}

// Two consecutive octets of one lane (16 bf16 values of a group held by
// G / 16 lanes): the same group amax, scale and bytes as quantize_octet on
// each octet (d0, d1 the first octet, d2, d3 the second; PERM: even k then
// odd k within each octet, as quantize_octet<G, true>).
template <int G, bool PERM = false>
__device__ __forceinline__ void quantize_octet_pair(const u32x4& v0, const u32x4& v1, uint32_t& d0, uint32_t& d1,
                                                    uint32_t& d2, uint32_t& d3, float& s) {
    const uint32_t wd[8] = {v0.x, v0.y, v0.z, v0.w, v1.x, v1.y, v1.z, v1.w};
    float f[16];
    float a = 0.0f;
#pragma unroll
    for (int e = 0; e < 16; ++e) {
        f[e] = bf16f((wd[e >> 1] >> (16 * (e & 1))) & 0xffffu);
        a = fmaxf(a, fabsf(f[e]));
    }
    a = group_max<G / 16>(a);
    float r;
    group_scale(a, s, r);
    uint32_t t[16];
#pragma unroll
    for (int e = 0; e < 16; ++e) t[e] = qbits(f[e], s, r);
    if constexpr (PERM) {
        d0 = bytes4(t[0], t[2], t[4], t[6]);
        d1 = bytes4(t[1], t[3], t[5], t[7]);
        d2 = bytes4(t[8], t[10], t[12], t[14]);
        d3 = bytes4(t[9], t[11], t[13], t[15]);
    } else {
        d0 = bytes4(t[0], t[1], t[2], t[3]);
        d1 = bytes4(t[4], t[5], t[6], t[7]);
        d2 = bytes4(t[8], t[9], t[10], t[11]);
        d3 = bytes4(t[12], t[13], t[14], t[15]);
    }
}

// Sum of the 8 int8 values held in two packed words.
__device__ __forceinline__ int bytesum8(uint32_t d0, uint32_t d1) {
    return sdot4(d0, 0x01010101u, sdot4(d1, 0x01010101u, 0));
}

__device__ __forceinline__ int sdot8(uint32_t a, uint32_t b, int c) {
    return __builtin_amdgcn_sdot8((int)a, (int)b, c, false);
}
__device__ __forceinline__ uint32_t udot8(uint32_t a, uint32_t b, uint32_t c) {
    return __builtin_amdgcn_udot8(a, b, c, false);
}

// Low nibbles of the 8 bytes of (d0, d1), packed: nibble n = byte n & 15.
__device__ __forceinline__ uint32_t nibbles8(uint32_t d0, uint32_t d1) {
    const uint32_t t0 = d0 & 0x0F0F0F0Fu, t1 = d1 & 0x0F0F0F0Fu;
    return __builtin_amdgcn_perm(t1 | (t1 >> 4), t0 | (t0 >> 4), 0x06040200u);
}

// --------------------------------------------------------- weight decode

template <int S>
__device__ __forceinline__ uint32_t shl(uint32_t v) {
    if constexpr (S >= 0) return v << S;
    else return v >> (-S);
}

// Unpack one 16-byte chunk into the 8 (Q4/Q5/Q6) or 4 (W8) dot4 operands.
// For the nibble formats word 2i holds the codes of k = 8i+{0,2,4,6} and
// word 2i+1 those of k = 8i+{1,3,5,7}; h0/h1 are the chunk's high-plane words.
template <int F, int I>
__device__ __forceinline__ void decode_word(uint32_t p, uint32_t h0, uint32_t h1, uint32_t* wd) {
    uint32_t lo = p & 0x0F0F0F0Fu;
    uint32_t hi = (p >> 4) & 0x0F0F0F0Fu;
    if constexpr (F == 5) {
        lo |= shl<4 - 2 * I>(h0) & 0x10101010u;
        hi |= shl<3 - 2 * I>(h0) & 0x10101010u;
    } else if constexpr (F == 6) {
        const uint32_t H = (I < 2) ? h0 : h1;
        lo |= shl<4 - 4 * (I & 1)>(H) & 0x30303030u;
        hi |= shl<2 - 4 * (I & 1)>(H) & 0x30303030u;
    }
    wd[2 * I] = lo;
    wd[2 * I + 1] = hi;
}
template <int F>
__device__ __forceinline__ void decode(const u32x4& p, uint32_t h0, uint32_t h1, uint32_t* wd) {
    if constexpr (F == 8) {
        wd[0] = p.x;
        wd[1] = p.y;
        wd[2] = p.z;
        wd[3] = p.w;
    } else {
        decode_word<F, 0>(p.x, h0, h1, wd);
        decode_word<F, 1>(p.y, h0, h1, wd);
        decode_word<F, 2>(p.z, h0, h1, wd);
        decode_word<F, 3>(p.w, h0, h1, wd);
    }
}

// Dot of one 16-byte weight chunk with its activations a (32 int8 for the
// nibble formats, 16 for W8), accumulated onto acc.
template <int F>
__device__ __forceinline__ int chunk_dot(const u32x4& p, uint32_t h0, uint32_t h1, const u32x4& a0,
                                         const u32x4& a1, int acc) {
    uint32_t wd[8];
    decode<F>(p, h0, h1, wd);
    acc = sdot4(wd[0], a0.x, acc);
    acc = sdot4(wd[1], a0.y, acc);
    acc = sdot4(wd[2], a0.z, acc);
    acc = sdot4(wd[3], a0.w, acc);
    if constexpr (F != 8) {
        acc = sdot4(wd[4], a1.x, acc);
        acc = sdot4(wd[5], a1.y, acc);
        acc = sdot4(wd[6], a1.z, acc);
        acc = sdot4(wd[7], a1.w, acc);
    }
    return acc;
}

// Q4_G64 chunk against nibble-split activations.  Each activation q is split
// as q = 16*qh + ql (qh = q >> 4 signed 4-bit, ql = q & 15 unsigned 4-bit);
// with the stored code u = w + 8 and w = u ^ 8 read as signed 4-bit,
//   sum w*q = 16 * sum w*qh + sum u*ql - 8 * sum ql,
// i.e. one v_dot8_i32_i4 and one v_dot8_u32_u4 per 8 weights, no unpacking.
// a0 = (QL0, QH0, QL1, QH1), a1 = (QL2, QH2, QL3, QH3) for the chunk's four
// dwords; corr = -8 * sum ql over the chunk.
__device__ __forceinline__ int chunk_dot_q4(const u32x4& p, const u32x4& a0, const u32x4& a1,
                                            int corr) {
    uint32_t lo = (uint32_t)corr;
    int hi = 0;
    lo = udot8(p.x, a0.x, lo);
    hi = sdot8(p.x ^ 0x88888888u, a0.y, hi);
    lo = udot8(p.y, a0.z, lo);
    hi = sdot8(p.y ^ 0x88888888u, a0.w, hi);
    lo = udot8(p.z, a1.x, lo);
    hi = sdot8(p.z ^ 0x88888888u, a1.y, hi);
    lo = udot8(p.w, a1.z, lo);
    hi = sdot8(p.w ^ 0x88888888u, a1.w, hi);
    return (int)((uint32_t)hi * 16u + lo);
}

// chunk_dot_q4 with the sign-flipped words px = p ^ 0x88888888 computed once
// by the caller (shared by the activation rows of a multi-row dot).
__device__ __forceinline__ int chunk_dot_q4x(const u32x4& p, const u32x4& px, const u32x4& a0, const u32x4& a1,
                                             int corr) {
    uint32_t lo = (uint32_t)corr;
    int hi = 0;
    lo = udot8(p.x, a0.x, lo);
    hi = sdot8(px.x, a0.y, hi);
    lo = udot8(p.y, a0.z, lo);
    hi = sdot8(px.y, a0.w, hi);
    lo = udot8(p.z, a1.x, lo);
    hi = sdot8(px.z, a1.y, hi);
    lo = udot8(p.w, a1.z, lo);
    hi = sdot8(px.w, a1.w, hi);
    return (int)((uint32_t)hi * 16u + lo);
}

// Raw buffer loads: the resource's byte range bounds every access, and an
// out-of-range lane reads 0 without touching memory, so the kernel issues
// all its loads unconditionally and the compiler counts them exactly.
typedef int i32x4 __attribute__((ext_vector_type(4)));
typedef int i32x2 __attribute__((ext_vector_type(2)));
constexpr int BUF_CFG = 0x00020000;  // dword 3 of a raw buffer resource on gfx9
constexpr int AUX_NT = 2;            // non-temporal (streamed once)
constexpr int AUX_SC1 = 16;          // device scope: written through the XCD's L2 (no dirty line left)
constexpr int OOB = 0x7ffffff0;      // an offset past any range used here

__device__ __forceinline__ __amdgpu_buffer_rsrc_t buf(const void* base, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes, BUF_CFG);
}
// Buffer stores (out-of-range offsets are dropped by the resource bounds).
// Written-through stores (AUX_SC1) leave no dirty L2 line for the end-of-kernel
// write-back, which shortens small producer kernels whose consumer follows.
template <int AUX = 0>
__device__ __forceinline__ void bstore16(__amdgpu_buffer_rsrc_t r, int off, const u32x4& v) {
    __builtin_amdgcn_raw_buffer_store_b128(i32x4{(int)v.x, (int)v.y, (int)v.z, (int)v.w}, r, off, 0, AUX);
}
template <int AUX = 0>
__device__ __forceinline__ void bstore8(__amdgpu_buffer_rsrc_t r, int off, const u32x2& v) {
    __builtin_amdgcn_raw_buffer_store_b64(i32x2{(int)v.x, (int)v.y}, r, off, 0, AUX);
}
template <int AUX = 0>
__device__ __forceinline__ void bstore4(__amdgpu_buffer_rsrc_t r, int off, uint32_t v) {
    __builtin_amdgcn_raw_buffer_store_b32((int)v, r, off, 0, AUX);
}

template <int AUX = 0>
__device__ __forceinline__ u32x4 bload16(__amdgpu_buffer_rsrc_t r, int off) {
    const i32x4 v = __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, AUX);
    return u32x4{(uint32_t)v.x, (uint32_t)v.y, (uint32_t)v.z, (uint32_t)v.w};
}
template <int AUX = 0>
__device__ __forceinline__ u32x2 bload8(__amdgpu_buffer_rsrc_t r, int off) {
    const i32x2 v = __builtin_amdgcn_raw_buffer_load_b64(r, off, 0, AUX);
    return u32x2{(uint32_t)v.x, (uint32_t)v.y};
}
template <int AUX = 0>
__device__ __forceinline__ uint32_t bload4(__amdgpu_buffer_rsrc_t r, int off) {
    return (uint32_t)__builtin_amdgcn_raw_buffer_load_b32(r, off, 0, AUX);
}
// Compiler-only fence for memory operations: loads issued before it stay
// before it, so the weight stream cannot be hoisted above the activation
// loads.  (Activation pointers are also kept free of __restrict__: a load
// through a restrict-qualified read-only pointer counts as invariant, and
// the register allocator then re-issues it at its first use, after the
// weight loads, where the wait for it waits for the whole weight stream -
// loads retire in issue order.)
__device__ __forceinline__ void issue_fence() { asm volatile("" ::: "memory"); }

__device__ __forceinline__ uint32_t bload2(__amdgpu_buffer_rsrc_t r, int off) {
    return (uint32_t)(uint16_t)__builtin_amdgcn_raw_buffer_load_b16(r, off, 0, 0);
}

}  // namespace vq
