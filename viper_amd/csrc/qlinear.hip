// Quantized linear for MI355X (gfx950): y = bf16( sum_g ws*xs*D_g [+ res] ).
//
// Semantics follow the reference's int8 decode path (itzrnvr/viper):
// activation quantize as kernels/ops/rmsnorm_quantize.cu:71-104 and
// linear_multim.cu:21-61 (per-row, per-group amax/127 floored at 1e-8,
// round-to-nearest-even of x/scale), group dot + fp32 combine as
// kernels/ops/dp4a_smem_kernel.cu:25-74 and linear_multim.cu:64-130, weight
// layout as tools/convert/convert.cpp:91-127.  The design is gfx950's own.
//
// M = 1 (qgemv_m1_kernel, the decode GEMV):
//  * a team of TS lanes (a power of two) streams one output row; a lane owns
//    whole quantization groups (32 bytes of the main plane = two 16-byte
//    non-temporal loads, plus the group's high-plane bytes and scale);
//  * every lane first issues its activation loads, then all its weight loads
//    (the vector-memory counter retires in issue order, so the activation
//    arrives first), then quantizes the bf16 activation into LDS while the
//    weight bytes are still in flight;
//  * nibbles are not sign-converted: v_dot4 runs on the offset codes u (u in
//    [0, 63] read as int8) and each group's -OFF * sum(q) correction is
//    computed once per workgroup into LDS, so the int32 group dot D is exact;
//  * fp32 (ws*xs)*D is accumulated per lane and the team is reduced with DPP
//    row operations in a fixed order (deterministic).
//
// M = 2..16 and prequantized activations (qgemm_pre_kernel): activations are
// quantized once into a caller workspace (quantize_act_kernel) or supplied by
// the caller, staged into LDS per workgroup, and every weight byte is read
// once for all M rows.
//
// The activation quantizer never divides per element: with s the group scale
// and r = 1/s (both IEEE divides, once per group), q0 = x*r and
// q1 = fma(fma(-q0, s, x), r, q0); adding 1.5*2^23 rounds q1 to the nearest
// even integer and leaves it, two's complement, in the low byte.  For every
// finite bf16 pair (amax, x) the byte equals RNE(x/s); check_quantizer_kernel
// and the CPU oracle verify that exhaustively.

#include <hip/hip_ext.h>
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
__device__ __forceinline__ uint16_t f2bf(float f) {
    uint32_t u = __float_as_uint(f);
    if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40u);
    u += 0x7fffu + ((u >> 16) & 1u);
    return (uint16_t)(u >> 16);
}
__device__ __forceinline__ int sdot4(uint32_t a, uint32_t b, int c) {
    return __builtin_amdgcn_sdot4((int)a, (int)b, c, false);
}
// Low bytes of four words -> one packed word [a0, b0, c0, d0].
__device__ __forceinline__ uint32_t bytes4(uint32_t a, uint32_t b, uint32_t c, uint32_t d) {
    const uint32_t ab = __builtin_amdgcn_perm(b, a, 0x0c0c0400u);
    const uint32_t cd = __builtin_amdgcn_perm(d, c, 0x0c0c0400u);
    return __builtin_amdgcn_perm(cd, ab, 0x05040100u);
}

// Max / sum over the LANES (4 or 8) consecutive lanes that hold one group.
template <int LANES>
__device__ __forceinline__ float group_max(float v) {
    v = fmaxf(v, dpp_f<DPP_SWAP1>(v));
    v = fmaxf(v, dpp_f<DPP_SWAP2>(v));
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

// Workgroup barrier that orders LDS only: the weight loads still in flight
// are not waited for (a full __syncthreads() would drain them first).
__device__ __forceinline__ void lds_barrier() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
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

__device__ __forceinline__ void group_scale(float amax, float& s, float& r) {
    s = fmaxf(amax / 127.0f, 1e-8f);
    r = 1.0f / s;
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

// ------------------------------------------------------- M = 1, fused quantize
//
// A team of TS lanes streams one output row: in each load instruction lane l
// reads 16-byte chunk c = base + l of the row, so every instruction reads
// whole contiguous row segments.  A chunk is half a quantization group; the
// two halves meet by a DPP lane swap of the int32 partial, and the even lane
// of the pair applies the group's scales.
//
// LDS: xq [K] int8 (octets in the format's dot order) and, per chunk,
// {-OFF * sum(q) over the chunk (int32), xs (fp32)}.

constexpr int M1_CPL = 10;  // chunk slots per lane per row segment
constexpr int M1_XS = 4;    // activation octets per thread loaded before the weights
constexpr int M1_DELAY = 4; // weight-issue delay, s_sleep units

template <int F>
__host__ __device__ constexpr size_t m1_lds_bytes(int K) {
    return (size_t)K + (size_t)(K / Fmt<F>::CK) * 8;
}

// Raw buffer loads: the resource's byte range bounds every access, and an
// out-of-range lane reads 0 without touching memory, so the kernel issues
// all its loads unconditionally and the compiler counts them exactly.
typedef int i32x4 __attribute__((ext_vector_type(4)));
typedef int i32x2 __attribute__((ext_vector_type(2)));
constexpr int BUF_CFG = 0x00020000;  // dword 3 of a raw buffer resource on gfx9
constexpr int AUX_NT = 2;            // non-temporal (streamed once)
constexpr int OOB = 0x7ffffff0;      // an offset past any range used here

__device__ __forceinline__ __amdgpu_buffer_rsrc_t buf(const void* base, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes, BUF_CFG);
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
__device__ __forceinline__ uint32_t bload2(__amdgpu_buffer_rsrc_t r, int off) {
    return (uint32_t)(uint16_t)__builtin_amdgcn_raw_buffer_load_b16(r, off, 0, 0);
}

// EXACT: every lane's chunks of every slot lie inside its row (the row has
// exactly TS * M1_CPL chunks), so no chunk needs masking.
// DELAY: s_sleep units (64 clocks) between issuing the activation loads and
// the weight loads.  The activation is a few KB read by every workgroup; a
// short head start lets its requests through the memory pipeline before the
// weight stream saturates it, which moves every workgroup's barrier earlier.
template <int F, int TS, int NTT, int SENC, bool PART, bool EXACT, int DELAY>
__global__ void __launch_bounds__(NTT)
qgemv_m1_kernel(const uint8_t* __restrict__ w, const uint16_t* __restrict__ ws,
                const uint16_t* __restrict__ x, uint16_t* y,
                const uint16_t* res, int32_t* __restrict__ part, int N, int K) {
    using FT = Fmt<F>;
    constexpr int CPL = M1_CPL;
    constexpr int XS = M1_XS;
    constexpr int ROWS = NTT / TS;
    constexpr int HB = FT::HIW * 4;  // high-plane bytes per chunk: Q5 4, Q6 8
    constexpr int OPC = FT::CK / 8;  // octets per chunk (4, or 2 for W8)
    extern __shared__ __align__(16) uint8_t smem[];
    const int CPR = K / FT::CK;      // chunks per row
    const int NGR = K / FT::G;       // groups per row
    int8_t* lxq = (int8_t*)smem;
    u32x2* lcs = (u32x2*)(smem + K);

    const int tid = (int)threadIdx.x;
    const int l = tid % TS;
    const int rr = tid / TS;  // row within the workgroup
    const int row0 = (int)blockIdx.x * ROWS;
    const int row = row0 + rr;
    const int nrows = min(ROWS, N - row0);
    const bool row_ok = rr < nrows;

    // 1. activation octets, then every weight byte and group scale of the
    //    first row segment, all in flight at once
    const int noct = K / 8;
    const auto xr = buf(x, (uint32_t)K * 2);
    u32x4 xv[XS];
#pragma unroll
    for (int i = 0; i < XS; ++i) xv[i] = bload16(xr, (tid + NTT * i) * 16);
    const auto sr = buf(ws + (size_t)row0 * NGR, (uint32_t)(nrows * NGR) * 2);
    const bool lead = (l & 1) == 0;  // the even lane of a chunk pair owns the group

    const uint32_t rbytes = (uint32_t)CPR * 16;
    const auto wr = buf(w + (size_t)row0 * rbytes, (uint32_t)nrows * rbytes);
    const auto hr = buf(w + (size_t)N * (K / 2) + (size_t)row0 * CPR * HB, (uint32_t)nrows * CPR * HB);
    const int segw = TS * CPL;
    const int nseg = EXACT ? 1 : (CPR + segw - 1) / segw;
    u32x4 wv[CPL];
    uint32_t h0[CPL], h1[CPL], sv[CPL];
    auto load_seg = [&](int seg) {
#pragma unroll
        for (int j = 0; j < CPL; ++j) {
            const int c = seg * segw + j * TS + l;
            const bool in = EXACT || c < CPR;
            wv[j] = bload16<AUX_NT>(wr, in ? rr * (int)rbytes + c * 16 : OOB);
            // odd lanes and chunks past the row read scale 0, which zeroes
            // their term without any select
            sv[j] = bload2(sr, (in && lead) ? (rr * NGR + (c >> 1)) * 2 : OOB);
            h0[j] = 0u;
            h1[j] = 0u;
            if constexpr (FT::HIW == 1) {
                h0[j] = bload4<AUX_NT>(hr, in ? (rr * CPR + c) * HB : OOB);
            } else if constexpr (FT::HIW == 2) {
                const u32x2 hh = bload8<AUX_NT>(hr, in ? (rr * CPR + c) * HB : OOB);
                h0[j] = hh.x;
                h1[j] = hh.y;
            }
        }
    };
    if constexpr (DELAY > 0) __builtin_amdgcn_s_sleep(DELAY);
    load_seg(0);

    // 2. quantize the activation into LDS (trip counts are workgroup-uniform,
    //    so every DPP group reduction sees whole groups).  Q4 stores each
    //    octet as (ql nibbles, qh nibbles); Q5/Q6 as [k even | k odd] int8;
    //    W8 in k order.
    const int xiters = (noct + NTT - 1) / NTT;
    auto quant_store = [&](int o, const u32x4& v) {
        uint32_t d0, d1;
        float s;
        quantize_octet<FT::G, (F == 5 || F == 6)>(v, d0, d1, s);
        int corr = 0;
        if constexpr (F == 4) {
            const uint32_t ql = nibbles8(d0, d1), qh = nibbles8(d0 >> 4, d1 >> 4);
            d0 = ql;
            d1 = qh;
            corr = -8 * group_sum<OPC>((int)udot8(ql, 0x11111111u, 0u));
        } else if constexpr (FT::OFF != 0) {
            corr = -FT::OFF * group_sum<OPC>(bytesum8(d0, d1));
        }
        if (o < noct) {
            *(u32x2*)(lxq + (size_t)o * 8) = u32x2{d0, d1};
            if (o % OPC == 0) lcs[o / OPC] = u32x2{(uint32_t)corr, __float_as_uint(s)};
        }
    };
    const int wave0 = tid & ~63;  // waves with no octet skip the quantize
#pragma unroll
    for (int i = 0; i < XS; ++i)
        if (i < xiters && wave0 + NTT * i < noct) quant_store(tid + NTT * i, xv[i]);
    for (int i = XS; i < xiters; ++i)
        if (wave0 + NTT * i < noct) quant_store(tid + NTT * i, bload16(xr, (tid + NTT * i) * 16));

    lds_barrier();

    // 3. chunk dots, group sums, fp32 combine; each chunk waits only for its
    //    own weights and scale
    float acc = 0.0f;
    for (int seg = 0; seg < nseg; ++seg) {
        if (seg) load_seg(seg);
#pragma unroll
        for (int j = 0; j < CPL; ++j) {
            const int c = seg * segw + j * TS + l;
            const bool ok = EXACT || c < CPR;
            const int cc = EXACT ? c : min(c, CPR - 1);
            const u32x2 cs = lcs[cc];
            const u32x4* a = (const u32x4*)(lxq + (size_t)cc * FT::CK);
            int dot;
            if constexpr (F == 4) dot = chunk_dot_q4(wv[j], a[0], a[1], (int)cs.x);
            else dot = chunk_dot<F>(wv[j], h0[j], h1[j], a[0], FT::OFF ? a[1] : a[0], (int)cs.x);
            dot += dpp_i<DPP_SWAP1>(dot);
            const int g = cc >> 1;
            if constexpr (PART)
                if (ok && lead && row_ok) part[(size_t)row * NGR + g] = dot;
            const float wsf = SENC ? bf16f(sv[j]) : f16f(sv[j]);
            acc = __builtin_fmaf(wsf * __uint_as_float(cs.y), (float)dot, acc);
        }
    }
    acc = team_sum<TS>(acc);
    if (l == 0 && row_ok) {
        if (res != nullptr) acc += bf16f(res[row]);
        y[row] = f2bf(acc);
    }
}

// --------------------------------------------- M <= 16, prequantized activations
//
// LDS holds, for M activation rows: xq [M][K] int8 (for the nibble formats
// each octet stored as [even k | odd k], matching decode()), corr [M][K/32]
// int32 = -OFF * (sum of q over each 32-element chunk) (nibble formats only),
// xs [M][K/G] fp32.  A team of TS lanes streams one row, one 16-byte chunk
// (half a group) per lane and slot; the halves of a group meet by a DPP swap.

template <int F>
__device__ void stage_prequant(const int8_t* __restrict__ xq, const float* __restrict__ xs, int M,
                               int K, int8_t* lxq, int32_t* lcorr, float* lxs) {
    using FT = Fmt<F>;
    const int oct_total = M * K / 8;
    const int iters = (oct_total + NT - 1) / NT;
    for (int it = 0; it < iters; ++it) {
        const int o = it * NT + (int)threadIdx.x;
        const bool ok = o < oct_total;
        u32x2 v = {0u, 0u};
        if (ok) v = *(const u32x2*)(xq + (size_t)o * 8);
        uint32_t d0 = v.x, d1 = v.y;
        if constexpr (FT::OFF != 0) {
            d0 = __builtin_amdgcn_perm(v.y, v.x, 0x06040200u);
            d1 = __builtin_amdgcn_perm(v.y, v.x, 0x07050301u);
            const int csum = group_sum<4>(bytesum8(v.x, v.y));
            if (ok) {
                *(u32x2*)(lxq + (size_t)o * 8) = u32x2{d0, d1};
                if ((o & 3) == 0) lcorr[o / 4] = -FT::OFF * csum;
            }
        } else if (ok) {
            *(u32x2*)(lxq + (size_t)o * 8) = u32x2{d0, d1};
        }
    }
    const int ns = M * (K / FT::G);
    for (int i = (int)threadIdx.x; i < ns; i += NT) lxs[i] = xs[i];
}

template <int F, int MT, int TS>
__global__ void __launch_bounds__(NT)
qgemm_pre_kernel(const uint8_t* __restrict__ w, const uint16_t* __restrict__ ws, int senc,
                 const int8_t* __restrict__ xq, const float* __restrict__ xs,
                 uint16_t* y, const uint16_t* res,
                 int32_t* __restrict__ part, int N, int K, int M) {
    using FT = Fmt<F>;
    extern __shared__ __align__(16) uint8_t smem[];
    const int CPR = K / FT::CK;
    const int NG = K / FT::G;
    int8_t* lxq = (int8_t*)smem;
    int32_t* lcorr = (int32_t*)(smem + (size_t)M * K);
    float* lxs = (float*)(smem + (size_t)M * K + (FT::OFF ? (size_t)M * (K / 32) * 4 : 0));

    const int tid = (int)threadIdx.x;
    const int l = tid % TS;
    const int row = (int)blockIdx.x * (NT / TS) + tid / TS;
    const bool row_ok = row < N;
    const size_t rstride = (F == 8) ? (size_t)K : (size_t)K / 2;
    const uint8_t* wrow = w + (size_t)row * rstride;
    const uint8_t* hrow = w + (size_t)N * (K / 2) + (size_t)row * (K / 32) * 4 * FT::HIW;
    const uint16_t* srow = ws + (size_t)row * NG;
    const int segw = TS * CPL;
    const int nseg = (CPR + segw - 1) / segw;

    u32x4 wv[CPL];
    uint32_t h0[CPL], h1[CPL], sv[CPL];

    auto load_seg = [&](int seg) {
#pragma unroll
        for (int j = 0; j < CPL; ++j) {
            const int c = seg * segw + j * TS + l;
            const bool ok = row_ok && c < CPR;
            wv[j] = u32x4{0u, 0u, 0u, 0u};
            h0[j] = 0u;
            h1[j] = 0u;
            sv[j] = 0u;
            if (ok) {
                wv[j] = __builtin_nontemporal_load((const u32x4*)(wrow + (size_t)c * 16));
                if constexpr (FT::HIW == 1) {
                    h0[j] = __builtin_nontemporal_load((const uint32_t*)(hrow + (size_t)c * 4));
                } else if constexpr (FT::HIW == 2) {
                    const u32x2 hh = __builtin_nontemporal_load((const u32x2*)(hrow + (size_t)c * 8));
                    h0[j] = hh.x;
                    h1[j] = hh.y;
                }
                sv[j] = srow[c >> 1];
            }
        }
    };

    load_seg(0);
    stage_prequant<F>(xq, xs, M, K, lxq, lcorr, lxs);
    __syncthreads();

    float acc[MT];
#pragma unroll
    for (int m = 0; m < MT; ++m) acc[m] = 0.0f;

    for (int seg = 0; seg < nseg; ++seg) {
        if (seg) load_seg(seg);
#pragma unroll
        for (int j = 0; j < CPL; ++j) {
            const int c = seg * segw + j * TS + l;
            const bool ok = row_ok && c < CPR;
            const int cc = ok ? c : 0;
            const int g = cc >> 1;
            const float wsf = senc ? bf16f(sv[j]) : f16f(sv[j]);
            const bool lead = (l & 1) == 0;
#pragma unroll
            for (int m = 0; m < MT; ++m) {
                if (m < M) {
                    const int8_t* a = lxq + (size_t)m * K + (size_t)cc * (FT::OFF ? 32 : 16);
                    const u32x4 a0 = *(const u32x4*)a;
                    u32x4 a1 = a0;
                    int dot = 0;
                    if constexpr (FT::OFF != 0) {
                        a1 = *(const u32x4*)(a + 16);
                        dot = lcorr[m * (K / 32) + cc];
                    }
                    dot = chunk_dot<F>(wv[j], h0[j], h1[j], a0, a1, dot);
                    int D = dot + dpp_i<DPP_SWAP1>(dot);
                    D = ok ? D : 0;
                    if (part != nullptr && ok && lead) part[((size_t)m * N + row) * NG + g] = D;
                    const float f = lead ? wsf * lxs[m * NG + g] : 0.0f;
                    acc[m] = __builtin_fmaf(f, (float)D, acc[m]);
                }
            }
        }
    }

#pragma unroll
    for (int m = 0; m < MT; ++m) {
        if (m < M) {
            float v = team_sum<TS>(acc[m]);
            if (l == 0 && row_ok) {
                if (res != nullptr) v += bf16f(res[(size_t)m * N + row]);
                y[(size_t)m * N + row] = f2bf(v);
            }
        }
    }
}

// ------------------------------------------------ standalone activation quantize

template <int G>
__global__ void __launch_bounds__(NT)
quantize_act_kernel(const uint16_t* __restrict__ x, int8_t* __restrict__ xq,
                    float* __restrict__ xs, int oct_total) {
    const int o = (int)blockIdx.x * NT + (int)threadIdx.x;
    const bool ok = o < oct_total;
    u32x4 v = {0u, 0u, 0u, 0u};
    if (ok) v = *(const u32x4*)(x + (size_t)o * 8);
    uint32_t d0, d1;
    float s;
    quantize_octet<G, false>(v, d0, d1, s);
    if (ok) {
        *(u32x2*)(xq + (size_t)o * 8) = u32x2{d0, d1};
        if ((o & (G / 8 - 1)) == 0) xs[(size_t)o * 8 / G] = s;
    }
}

// --------------------------------------------------- quantizer self-check

__global__ void __launch_bounds__(NT) check_quantizer_kernel(int ab0, int32_t* __restrict__ counts) {
    __shared__ int red[NT];
    const int ab = ab0 + (int)blockIdx.x;
    const float amax = bf16f((uint32_t)ab);
    float s, r;
    group_scale(amax, s, r);
    const float s_ieee = fmaxf(amax / 127.0f, 1e-8f);
    int bad = s != s_ieee;
    for (int xb = (int)threadIdx.x; xb <= ab; xb += NT) {
        const float xv = bf16f((uint32_t)xb);
        const int fast = (int8_t)(qbits(xv, s, r) & 0xffu);
        const int fastn = (int8_t)(qbits(-xv, s, r) & 0xffu);
        const float ex = fminf(fmaxf(__builtin_rintf(xv / s_ieee), -127.0f), 127.0f);
        bad += fast != (int)ex;
        bad += fastn != -(int)ex;
    }
    red[threadIdx.x] = bad;
    __syncthreads();
    for (int step = NT / 2; step > 0; step >>= 1) {
        if ((int)threadIdx.x < step) red[threadIdx.x] += red[threadIdx.x + step];
        __syncthreads();
    }
    if (threadIdx.x == 0) counts[blockIdx.x] = red[0];
}

// ------------------------------------------------------------------ host side

static int status_of(hipError_t e) {
    if (e == hipSuccess) return VIPER_OK;
    if (e == hipErrorOutOfMemory) return VIPER_OUT_OF_MEMORY;
    return VIPER_DEVICE_ERROR;
}

static int group_of(int qtype) {
    switch (qtype) {
        case VIPER_QTYPE_Q4_G64:
        case VIPER_QTYPE_Q5_G64:
        case VIPER_QTYPE_Q6_G64: return 64;
        case VIPER_QTYPE_W8_G32: return 32;
        default: return 0;
    }
}

static size_t align16(size_t v) { return (v + 15) & ~(size_t)15; }

// LDS of the prequantized kernel for M rows
static size_t lds_pre(int qtype, int M, int K) {
    const size_t G = (size_t)group_of(qtype);
    size_t b = (size_t)M * K + (size_t)M * (K / G) * 4;
    if (qtype != VIPER_QTYPE_W8_G32) b += (size_t)M * (K / 32) * 4;
    return b;
}

static bool misaligned(const void* p, size_t a) { return ((uintptr_t)p % a) != 0; }

static int validate_weights(int qtype, const void* w, const void* s, int senc, int group, int N,
                            int K, int M) {
    if (qtype == VIPER_QTYPE_BF16 || qtype == VIPER_QTYPE_FP32) return VIPER_UNIMPLEMENTED;
    const int G = group_of(qtype);
    if (G == 0) return VIPER_INVALID_ARGUMENT;
    if (w == nullptr || s == nullptr) return VIPER_INVALID_ARGUMENT;
    if (senc != VIPER_SCALE_FP16 && senc != VIPER_SCALE_BF16) return VIPER_INVALID_ARGUMENT;
    if (group != G) return VIPER_INVALID_ARGUMENT;
    if (N <= 0 || K <= 0 || M <= 0 || M > VIPER_QLINEAR_MAX_M) return VIPER_INVALID_ARGUMENT;
    if (K % G != 0) return VIPER_INVALID_ARGUMENT;
    if ((int64_t)M * K > INT32_MAX / 2) return VIPER_INVALID_ARGUMENT;
    if (misaligned(w, 16) || misaligned(s, 2)) return VIPER_INVALID_ARGUMENT;
    return VIPER_OK;
}

static void launch(const void* fn, unsigned grid, unsigned block, size_t lds, hipStream_t st,
                   void** args, hipEvent_t ev0, hipEvent_t ev1) {
    // Events (when given) are attached to this dispatch, so they time the
    // kernel itself rather than the host-side launch.
    if (ev0 == nullptr && ev1 == nullptr)
        (void)hipLaunchKernel(fn, dim3(grid), dim3(block), args, lds, st);
    else
        (void)hipExtLaunchKernel(fn, dim3(grid), dim3(block), args, lds, st, ev0, ev1, 0);
}

// ---- M = 1 fused

typedef void (*m1_fn)(const uint8_t*, const uint16_t*, const uint16_t*, uint16_t*,
                      const uint16_t*, int32_t*, int, int);

struct M1Shape {
    int ts, ntt;
};

// Launch shapes instantiated for the fused M = 1 kernel.
template <int F, int SENC, bool PART, bool EXACT>
static m1_fn m1_kernel_v(int ts, int ntt) {
#define VQ_M1(TS_, NTT_) \
    if (ts == TS_ && ntt == NTT_) return qgemv_m1_kernel<F, TS_, NTT_, SENC, PART, EXACT, M1_DELAY>;
    VQ_M1(8, 320) VQ_M1(16, 256) VQ_M1(16, 640) VQ_M1(32, 320) VQ_M1(32, 640) VQ_M1(64, 640)
#undef VQ_M1
    return nullptr;
}
template <int F, bool EXACT>
static m1_fn m1_kernel_e(int ts, int ntt, int senc, bool part) {
    if (senc == VIPER_SCALE_BF16)
        return part ? m1_kernel_v<F, 1, true, EXACT>(ts, ntt) : m1_kernel_v<F, 1, false, EXACT>(ts, ntt);
    return part ? m1_kernel_v<F, 0, true, EXACT>(ts, ntt) : m1_kernel_v<F, 0, false, EXACT>(ts, ntt);
}
template <int F>
static m1_fn m1_kernel(int ts, int ntt, int senc = 0, bool part = false, bool exact = false) {
    return exact ? m1_kernel_e<F, true>(ts, ntt, senc, part) : m1_kernel_e<F, false>(ts, ntt, senc, part);
}

// Team size: the smallest of 8..64 lanes covering a row in at most M1_CPL
// chunks per lane (longer rows loop over segments of 64 lanes).  Workgroup
// size: among the instantiated ones for that team, the one whose per-CU row
// load ceil(ceil(N/rows)/CUs)*rows is smallest (ties: more rows per group,
// i.e. fewer redundant activation quantizations).
static M1Shape m1_shape(int cpr, int N, int cus) {
    int ts = 8;
    while (ts < 64 && ts * M1_CPL < cpr) ts *= 2;
    static const int cand[] = {256, 320, 640};
    M1Shape best{ts, 0};
    long best_load = -1;
    for (int ntt : cand) {
        if (m1_kernel<4>(ts, ntt) == nullptr) continue;
        const long rows = ntt / ts;
        const long groups = (N + rows - 1) / rows;
        const long load = ((groups + cus - 1) / cus) * rows;
        if (best_load < 0 || load < best_load || (load == best_load && ntt > best.ntt)) {
            best_load = load;
            best.ntt = ntt;
        }
    }
    return best;
}

static int device_cus() {
    int dev = 0, cus = 0;
    if (hipGetDevice(&dev) != hipSuccess) return 256;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0)
        return 256;
    return cus;
}

static size_t lds_m1(int qtype, int K) {
    switch (qtype) {
        case VIPER_QTYPE_Q4_G64: return m1_lds_bytes<4>(K);
        case VIPER_QTYPE_Q5_G64: return m1_lds_bytes<5>(K);
        case VIPER_QTYPE_Q6_G64: return m1_lds_bytes<6>(K);
        default: return m1_lds_bytes<8>(K);
    }
}

static int launch_m1(int qtype, const void* w, const void* s, int senc, int N, int K,
                     const void* x, void* y, const void* res, int32_t* part, hipStream_t st,
                     hipEvent_t ev0, hipEvent_t ev1) {
    const int ck = qtype == VIPER_QTYPE_W8_G32 ? 16 : 32;
    const M1Shape sh = m1_shape(K / ck, N, device_cus());
    m1_fn fn;
    const bool want_part = part != nullptr;
    const bool exact = (K / ck) == sh.ts * M1_CPL;
    switch (qtype) {
        case VIPER_QTYPE_Q4_G64: fn = m1_kernel<4>(sh.ts, sh.ntt, senc, want_part, exact); break;
        case VIPER_QTYPE_Q5_G64: fn = m1_kernel<5>(sh.ts, sh.ntt, senc, want_part, exact); break;
        case VIPER_QTYPE_Q6_G64: fn = m1_kernel<6>(sh.ts, sh.ntt, senc, want_part, exact); break;
        default: fn = m1_kernel<8>(sh.ts, sh.ntt, senc, want_part, exact); break;
    }
    if (fn == nullptr) return VIPER_INTERNAL;
    const int rows = sh.ntt / sh.ts;
    const size_t lds = lds_m1(qtype, K);
    if (lds > (size_t)LDS_MAX) return VIPER_INVALID_ARGUMENT;
    const unsigned grid = (unsigned)((N + rows - 1) / rows);
    const uint8_t* a0 = (const uint8_t*)w;
    const uint16_t* a1 = (const uint16_t*)s;
    const uint16_t* a3 = (const uint16_t*)x;
    uint16_t* a4 = (uint16_t*)y;
    const uint16_t* a5 = (const uint16_t*)res;
    void* args[] = {&a0, &a1, &a3, &a4, &a5, &part, &N, &K};
    launch((const void*)fn, grid, (unsigned)sh.ntt, lds, st, args, ev0, ev1);
    return status_of(hipGetLastError());
}

// ---- M <= 16 prequantized

typedef void (*pre_fn)(const uint8_t*, const uint16_t*, int, const int8_t*, const float*,
                       uint16_t*, const uint16_t*, int32_t*, int, int, int);

template <int F, int MT>
static pre_fn pick_pre_ts(int ts) {
    switch (ts) {
        case 16: return qgemm_pre_kernel<F, MT, 16>;
        case 32: return qgemm_pre_kernel<F, MT, 32>;
        default: return qgemm_pre_kernel<F, MT, 64>;
    }
}
template <int F>
static pre_fn pick_pre(int mt, int ts) {
    switch (mt) {
        case 1: return pick_pre_ts<F, 1>(ts);
        case 2: return pick_pre_ts<F, 2>(ts);
        case 4: return pick_pre_ts<F, 4>(ts);
        case 8: return pick_pre_ts<F, 8>(ts);
        default: return pick_pre_ts<F, 16>(ts);
    }
}

static int launch_pre(int qtype, const void* w, const void* s, int senc, int N, int K,
                      const void* xq, const void* xs, int M, void* y, const void* res,
                      int32_t* part, hipStream_t st, hipEvent_t ev0, hipEvent_t ev1) {
    const size_t lds = lds_pre(qtype, M, K);
    if (lds > (size_t)LDS_MAX) return VIPER_INVALID_ARGUMENT;
    const int cpr = K / (qtype == VIPER_QTYPE_W8_G32 ? 16 : 32);
    const int ts = cpr <= 16 * CPL ? 16 : cpr <= 32 * CPL ? 32 : 64;
    const int mt = M <= 1 ? 1 : M <= 2 ? 2 : M <= 4 ? 4 : M <= 8 ? 8 : 16;
    pre_fn fn;
    switch (qtype) {
        case VIPER_QTYPE_Q4_G64: fn = pick_pre<4>(mt, ts); break;
        case VIPER_QTYPE_Q5_G64: fn = pick_pre<5>(mt, ts); break;
        case VIPER_QTYPE_Q6_G64: fn = pick_pre<6>(mt, ts); break;
        default: fn = pick_pre<8>(mt, ts); break;
    }
    const int rows = NT / ts;
    const unsigned grid = (unsigned)((N + rows - 1) / rows);
    const uint8_t* a0 = (const uint8_t*)w;
    const uint16_t* a1 = (const uint16_t*)s;
    const int8_t* a3 = (const int8_t*)xq;
    const float* a4 = (const float*)xs;
    uint16_t* a5 = (uint16_t*)y;
    const uint16_t* a6 = (const uint16_t*)res;
    void* args[] = {&a0, &a1, &senc, &a3, &a4, &a5, &a6, &part, &N, &K, &M};
    launch((const void*)fn, grid, NT, lds, st, args, ev0, ev1);
    return status_of(hipGetLastError());
}

static int launch_quantize(int group, const void* x, int M, int K, void* xq, void* xs,
                           hipStream_t st) {
    const int oct_total = M * K / 8;
    const unsigned grid = (unsigned)((oct_total + NT - 1) / NT);
    const uint16_t* a0 = (const uint16_t*)x;
    int8_t* a1 = (int8_t*)xq;
    float* a2 = (float*)xs;
    void* args[] = {&a0, &a1, &a2, (void*)&oct_total};
    const void* fn = group == 64 ? (const void*)quantize_act_kernel<64>
                                 : (const void*)quantize_act_kernel<32>;
    launch(fn, grid, NT, 0, st, args, nullptr, nullptr);
    return status_of(hipGetLastError());
}

// M = 1 is fused when the quantized activation and its per-chunk records fit
// the LDS budget.
static bool fused_ok(int qtype, int M, int K) {
    return M == 1 && lds_m1(qtype, K) <= (size_t)LDS_MAX;
}

static size_t workspace_need(int qtype, int K, int M) {
    const int G = group_of(qtype);
    if (G == 0 || M <= 0 || K <= 0) return 0;
    if (fused_ok(qtype, M, K)) return 0;
    return align16((size_t)M * K) + align16((size_t)M * (K / G) * 4);
}

static int qlinear_common(int qtype, const void* w, const void* s, int senc, int group, int N,
                          int K, const void* x, int M, void* y, const void* res, void* wsp,
                          size_t wsp_bytes, int32_t* part, void* stream,
                          hipEvent_t ev0 = nullptr, hipEvent_t ev1 = nullptr) {
    int rc = validate_weights(qtype, w, s, senc, group, N, K, M);
    if (rc != VIPER_OK) return rc;
    if (x == nullptr || y == nullptr) return VIPER_INVALID_ARGUMENT;
    if (misaligned(x, 16) || misaligned(y, 2) || misaligned(res, 2) || misaligned(part, 4))
        return VIPER_INVALID_ARGUMENT;
    hipStream_t st = (hipStream_t)stream;
    if (fused_ok(qtype, M, K)) return launch_m1(qtype, w, s, senc, N, K, x, y, res, part, st, ev0, ev1);
    const size_t need = workspace_need(qtype, K, M);
    if (wsp == nullptr || wsp_bytes < need || misaligned(wsp, 16)) return VIPER_INVALID_ARGUMENT;
    if (lds_pre(qtype, M, K) > (size_t)LDS_MAX) return VIPER_INVALID_ARGUMENT;
    uint8_t* xq = (uint8_t*)wsp;
    float* xs = (float*)(xq + align16((size_t)M * K));
    rc = launch_quantize(group, x, M, K, xq, xs, st);
    if (rc != VIPER_OK) return rc;
    return launch_pre(qtype, w, s, senc, N, K, xq, xs, M, y, res, part, st, ev0, ev1);
}

}  // namespace vq

// ------------------------------------------------------------------- C ABI

extern "C" int viper_hip_abi_version(void) { return VIPER_QLINEAR_ABI_VERSION; }

extern "C" int viper_hip_group_size(int qtype) { return vq::group_of(qtype); }

extern "C" size_t viper_hip_qlinear_workspace_bytes(int qtype, int N, int K, int M) {
    (void)N;
    return vq::workspace_need(qtype, K, M);
}

extern "C" int viper_hip_qlinear(int qtype, const void* w_packed, const void* w_scales,
                                 int scale_enc, int group, int N, int K, const void* x_bf16, int M,
                                 void* y_bf16, const void* residual_bf16, void* workspace,
                                 size_t workspace_bytes, void* stream) {
    return vq::qlinear_common(qtype, w_packed, w_scales, scale_enc, group, N, K, x_bf16, M, y_bf16,
                              residual_bf16, workspace, workspace_bytes, nullptr, stream);
}

extern "C" int viper_hip_qlinear_timed(int qtype, const void* w_packed, const void* w_scales,
                                       int scale_enc, int group, int N, int K, const void* x_bf16,
                                       int M, void* y_bf16, const void* residual_bf16,
                                       void* workspace, size_t workspace_bytes, void* start_event,
                                       void* stop_event, void* stream) {
    return vq::qlinear_common(qtype, w_packed, w_scales, scale_enc, group, N, K, x_bf16, M, y_bf16,
                              residual_bf16, workspace, workspace_bytes, nullptr, stream,
                              (hipEvent_t)start_event, (hipEvent_t)stop_event);
}

extern "C" int viper_hip_qlinear_partials(int qtype, const void* w_packed, const void* w_scales,
                                          int scale_enc, int group, int N, int K,
                                          const void* x_bf16, int M, void* y_bf16,
                                          const void* residual_bf16, void* workspace,
                                          size_t workspace_bytes, int32_t* partials,
                                          void* stream) {
    if (partials == nullptr) return VIPER_INVALID_ARGUMENT;
    return vq::qlinear_common(qtype, w_packed, w_scales, scale_enc, group, N, K, x_bf16, M, y_bf16,
                              residual_bf16, workspace, workspace_bytes, partials, stream);
}

extern "C" int viper_hip_quantize_act(int group, const void* x_bf16, int M, int K, void* xq,
                                      void* xs, void* stream) {
    if (group != 64 && group != 32) return VIPER_INVALID_ARGUMENT;
    if (x_bf16 == nullptr || xq == nullptr || xs == nullptr) return VIPER_INVALID_ARGUMENT;
    if (M <= 0 || K <= 0 || K % group != 0) return VIPER_INVALID_ARGUMENT;
    if ((int64_t)M * K > INT32_MAX / 2) return VIPER_INVALID_ARGUMENT;
    if (vq::misaligned(x_bf16, 16) || vq::misaligned(xq, 8) || vq::misaligned(xs, 4))
        return VIPER_INVALID_ARGUMENT;
    return vq::launch_quantize(group, x_bf16, M, K, xq, xs, (hipStream_t)stream);
}

extern "C" int viper_hip_qlinear_prequantized(int qtype, const void* w_packed,
                                              const void* w_scales, int scale_enc, int group,
                                              int N, int K, const void* xq, const void* xs, int M,
                                              void* y_bf16, const void* residual_bf16,
                                              void* stream) {
    int rc = vq::validate_weights(qtype, w_packed, w_scales, scale_enc, group, N, K, M);
    if (rc != VIPER_OK) return rc;
    if (xq == nullptr || xs == nullptr || y_bf16 == nullptr) return VIPER_INVALID_ARGUMENT;
    if (vq::misaligned(xq, 8) || vq::misaligned(xs, 4) || vq::misaligned(y_bf16, 2) ||
        vq::misaligned(residual_bf16, 2))
        return VIPER_INVALID_ARGUMENT;
    return vq::launch_pre(qtype, w_packed, w_scales, scale_enc, N, K, xq, xs, M, y_bf16,
                          residual_bf16, nullptr, (hipStream_t)stream, nullptr, nullptr);
}

extern "C" int viper_hip_check_quantizer(int exp_lo, int exp_hi, int32_t* counts, void* stream) {
    if (counts == nullptr || exp_lo < 0 || exp_hi > 254 || exp_lo > exp_hi)
        return VIPER_INVALID_ARGUMENT;
    if (vq::misaligned(counts, 4)) return VIPER_INVALID_ARGUMENT;
    int ab0 = exp_lo << 7;
    int32_t* c = counts;
    void* args[] = {&ab0, &c};
    const unsigned grid = (unsigned)((exp_hi - exp_lo + 1) << 7);
    vq::launch((const void*)vq::check_quantizer_kernel, grid, vq::NT, 0, (hipStream_t)stream, args,
               nullptr, nullptr);
    return vq::status_of(hipGetLastError());
}
