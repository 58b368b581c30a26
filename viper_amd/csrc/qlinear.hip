// Quantized linear for MI355X (gfx950): y = bf16( sum_g ws*xs*D_g [+ res] ).
//
// Semantics follow the reference's int8 decode path (itzrnvr/viper):
// activation quantize as kernels/ops/rmsnorm_quantize.cu:71-104 and
// linear_multim.cu:21-61 (per-row, per-group amax/127 floored at 1e-8,
// round-to-nearest-even of x/scale), group dot + fp32 combine as
// kernels/ops/dp4a_smem_kernel.cu:25-74 and linear_multim.cu:64-130, weight
// layout as tools/convert/convert.cpp:91-127.  The design is gfx950's own:
//
//  * one workgroup of 256 lanes owns 256/TS output rows; a team of TS lanes
//    (16/32/64) streams one row with 16-byte non-temporal loads, so each load
//    instruction reads TS*16 contiguous bytes of a row;
//  * every lane issues all its weight, high-plane and scale loads first and
//    only then quantizes the activations into LDS, so the HBM latency of the
//    first loads hides the prologue;
//  * a 16-byte chunk is half a quantization group.  Nibbles are not
//    sign-converted: the dot runs on offset codes u (v_dot4 with u in
//    [0, 63] read as int8) and the chunk's -OFF * sum(q) correction is
//    precomputed once per workgroup in LDS, so D stays exact;
//  * the two halves of a group meet with one DPP lane swap, giving the exact
//    int32 group sum D, then fp32 (ws*xs)*D is accumulated per lane and the
//    team is reduced with DPP row operations (fixed order, deterministic).
//
// The activation quantize replaces the IEEE divide x/s by q0 = x*r,
// q1 = fma(fma(-q0, s, x), r, q0) with r = 1/s (IEEE).  For every finite
// bf16 pair (amax, x) the rounded integer equals rint(x/s); the device
// self-check kernel below and the CPU oracle verify that exhaustively.

#include <hip/hip_ext.h>
#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#include "viper_qlinear.h"

namespace vq {

typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));

constexpr int NT = 256;            // threads per workgroup
constexpr int CPL = 8;             // chunk slots per lane per row segment
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
    return __builtin_amdgcn_update_dpp(0, v, CTRL, 0xF, 0xF, true);
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
__device__ __forceinline__ uint32_t pack4(int a, int b, int c, int d) {
    return (uint32_t)(a & 0xff) | ((uint32_t)(b & 0xff) << 8) | ((uint32_t)(c & 0xff) << 16) |
           ((uint32_t)(d & 0xff) << 24);
}
__device__ __forceinline__ int sdot4(uint32_t a, uint32_t b, int c) {
    return __builtin_amdgcn_sdot4((int)a, (int)b, c, false);
}

// Max over the LANES (4 or 8) consecutive lanes that hold one group.
template <int LANES>
__device__ __forceinline__ float group_max(float v) {
    v = fmaxf(v, dpp_f<DPP_SWAP1>(v));
    v = fmaxf(v, dpp_f<DPP_SWAP2>(v));
    if (LANES == 8) v = fmaxf(v, dpp_f<DPP_HALF_MIRROR>(v));
    return v;
}
__device__ __forceinline__ int quad_sum(int v) {
    v += dpp_i<DPP_SWAP1>(v);
    v += dpp_i<DPP_SWAP2>(v);
    return v;
}

// Sum over a team of TS consecutive lanes; every lane of the team gets it.
template <int TS>
__device__ __forceinline__ float team_sum(float v) {
    v += dpp_f<DPP_SWAP1>(v);
    v += dpp_f<DPP_SWAP2>(v);
    v += dpp_f<DPP_HALF_MIRROR>(v);
    v += dpp_f<DPP_MIRROR>(v);
    if (TS >= 32) v += __shfl_xor(v, 16, 64);
    if (TS >= 64) v += __shfl_xor(v, 32, 64);
    return v;
}

// RNE(x / s) clamped to +-127, without a divide (see the file comment).
__device__ __forceinline__ int quant1(float x, float s, float r) {
    const float q0 = __fmul_rn(x, r);
    const float e = __builtin_fmaf(-q0, s, x);
    const float q1 = __builtin_fmaf(e, r, q0);
    const float q = fminf(fmaxf(__builtin_rintf(q1), -127.0f), 127.0f);
    return (int)q;
}

template <int S>
__device__ __forceinline__ uint32_t shl(uint32_t v) {
    if constexpr (S >= 0) return v << S;
    else return v >> (-S);
}

// Unpack one 16-byte chunk into the 8 (Q4/Q5/Q6) or 4 (W8) dot4 operands.
// For the nibble formats word 2i holds the codes of k = 8i+{0,2,4,6} and
// word 2i+1 those of k = 8i+{1,3,5,7}.
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

// ------------------------------------------------------- LDS activation stage
//
// LDS holds, for M activation rows: xq [M][K] int8 (for the nibble formats
// each 8-element octet is stored as [even k | odd k], matching decode()),
// corr [M][K/32] int32 = -OFF * (sum of q over each 32-element chunk)
// (nibble formats only), xs [M][K/G] fp32.

template <int F>
__device__ __forceinline__ void store_octet(int o, bool ok, int q0, int q1, int q2, int q3, int q4,
                                            int q5, int q6, int q7, float s, int8_t* lxq,
                                            int32_t* lcorr, float* lxs) {
    using FT = Fmt<F>;
    uint32_t d0, d1;
    int csum = 0;
    if constexpr (FT::OFF != 0) {
        d0 = pack4(q0, q2, q4, q6);
        d1 = pack4(q1, q3, q5, q7);
        csum = quad_sum(q0 + q1 + q2 + q3 + q4 + q5 + q6 + q7);
    } else {
        d0 = pack4(q0, q1, q2, q3);
        d1 = pack4(q4, q5, q6, q7);
    }
    if (ok) {
        *(u32x2*)(lxq + (size_t)o * 8) = u32x2{d0, d1};
        if constexpr (FT::OFF != 0)
            if ((o & 3) == 0) lcorr[o / 4] = -FT::OFF * csum;
        if ((o & (FT::G / 8 - 1)) == 0) lxs[(o * 8) / FT::G] = s;
    }
}

// Fused prologue: quantize x[M][K] bf16 into LDS.  The loop trip count is
// uniform over the workgroup so the DPP group reductions see whole groups.
template <int F>
__device__ void stage_quantize(const uint16_t* __restrict__ x, int M, int K, int8_t* lxq,
                               int32_t* lcorr, float* lxs) {
    using FT = Fmt<F>;
    const int oct_total = M * K / 8;
    const int iters = (oct_total + NT - 1) / NT;
    for (int it = 0; it < iters; ++it) {
        const int o = it * NT + (int)threadIdx.x;
        const bool ok = o < oct_total;
        u32x4 v = {0u, 0u, 0u, 0u};
        if (ok) v = *(const u32x4*)(x + (size_t)o * 8);
        float f[8];
        f[0] = bf16f(v.x & 0xffffu);
        f[1] = bf16f(v.x >> 16);
        f[2] = bf16f(v.y & 0xffffu);
        f[3] = bf16f(v.y >> 16);
        f[4] = bf16f(v.z & 0xffffu);
        f[5] = bf16f(v.z >> 16);
        f[6] = bf16f(v.w & 0xffffu);
        f[7] = bf16f(v.w >> 16);
        float a = 0.0f;
#pragma unroll
        for (int j = 0; j < 8; ++j) a = fmaxf(a, fabsf(f[j]));
        a = group_max<FT::G / 8>(a);
        const float s = fmaxf(a / 127.0f, 1e-8f);
        const float r = 1.0f / s;
        int q[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) q[j] = quant1(f[j], s, r);
        store_octet<F>(o, ok, q[0], q[1], q[2], q[3], q[4], q[5], q[6], q[7], s, lxq, lcorr, lxs);
    }
}

// Prequantized prologue: copy xq[M][K] (natural order) and xs into LDS.
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
            const int csum = quad_sum(sdot4(v.x, 0x01010101u, 0) + sdot4(v.y, 0x01010101u, 0));
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

// ------------------------------------------------------------ GEMV / GEMM
//
// M <= MT activation rows, every weight byte read once.  Grid: one
// workgroup per NT/TS output rows.

template <int F, int MT, int TS, bool PRE>
__global__ void __launch_bounds__(NT)
qgemm_dot4_kernel(const uint8_t* __restrict__ w, const uint16_t* __restrict__ ws, int senc,
                  const uint16_t* __restrict__ x, const int8_t* __restrict__ xq,
                  const float* __restrict__ xs, uint16_t* __restrict__ y,
                  const uint16_t* __restrict__ res, int32_t* __restrict__ part, int N, int K,
                  int M) {
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
    if constexpr (PRE) stage_prequant<F>(xq, xs, M, K, lxq, lcorr, lxs);
    else stage_quantize<F>(x, M, K, lxq, lcorr, lxs);
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
            uint32_t wd[8];
            decode<F>(wv[j], h0[j], h1[j], wd);
            const float wsf = senc ? bf16f(sv[j]) : f16f(sv[j]);
            const bool lead = (l & 1) == 0;
#pragma unroll
            for (int m = 0; m < MT; ++m) {
                if (m < M) {
                    const int8_t* a = lxq + (size_t)m * K + (size_t)cc * (FT::OFF ? 32 : 16);
                    int dot;
                    if constexpr (FT::OFF != 0) {
                        const u32x4 a0 = *(const u32x4*)a;
                        const u32x4 a1 = *(const u32x4*)(a + 16);
                        dot = lcorr[m * (K / 32) + cc];
                        dot = sdot4(wd[0], a0.x, dot);
                        dot = sdot4(wd[1], a0.y, dot);
                        dot = sdot4(wd[2], a0.z, dot);
                        dot = sdot4(wd[3], a0.w, dot);
                        dot = sdot4(wd[4], a1.x, dot);
                        dot = sdot4(wd[5], a1.y, dot);
                        dot = sdot4(wd[6], a1.z, dot);
                        dot = sdot4(wd[7], a1.w, dot);
                    } else {
                        const u32x4 a0 = *(const u32x4*)a;
                        dot = sdot4(wd[0], a0.x, 0);
                        dot = sdot4(wd[1], a0.y, dot);
                        dot = sdot4(wd[2], a0.z, dot);
                        dot = sdot4(wd[3], a0.w, dot);
                    }
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
    float f[8];
    f[0] = bf16f(v.x & 0xffffu);
    f[1] = bf16f(v.x >> 16);
    f[2] = bf16f(v.y & 0xffffu);
    f[3] = bf16f(v.y >> 16);
    f[4] = bf16f(v.z & 0xffffu);
    f[5] = bf16f(v.z >> 16);
    f[6] = bf16f(v.w & 0xffffu);
    f[7] = bf16f(v.w >> 16);
    float a = 0.0f;
#pragma unroll
    for (int j = 0; j < 8; ++j) a = fmaxf(a, fabsf(f[j]));
    a = group_max<G / 8>(a);
    const float s = fmaxf(a / 127.0f, 1e-8f);
    const float r = 1.0f / s;
    int q[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) q[j] = quant1(f[j], s, r);
    if (ok) {
        *(u32x2*)(xq + (size_t)o * 8) = u32x2{pack4(q[0], q[1], q[2], q[3]), pack4(q[4], q[5], q[6], q[7])};
        if ((o & (G / 8 - 1)) == 0) xs[(size_t)o * 8 / G] = s;
    }
}

// --------------------------------------------------- quantizer self-check

__global__ void __launch_bounds__(NT) check_quantizer_kernel(int ab0, int32_t* __restrict__ counts) {
    __shared__ int red[NT];
    const int ab = ab0 + (int)blockIdx.x;
    const float amax = bf16f((uint32_t)ab);
    const float s = fmaxf(amax / 127.0f, 1e-8f);
    const float r = 1.0f / s;
    int bad = 0;
    for (int xb = (int)threadIdx.x; xb <= ab; xb += NT) {
        const float xv = bf16f((uint32_t)xb);
        const int fast = quant1(xv, s, r);
        const float ex = fminf(fmaxf(__builtin_rintf(xv / s), -127.0f), 127.0f);
        bad += fast != (int)ex;
        const int fastn = quant1(-xv, s, r);
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

static size_t lds_bytes(int qtype, int M, int K) {
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
    if (misaligned(w, 16) || misaligned(s, 2)) return VIPER_INVALID_ARGUMENT;
    return VIPER_OK;
}

typedef void (*gemm_fn)(const uint8_t*, const uint16_t*, int, const uint16_t*, const int8_t*,
                        const float*, uint16_t*, const uint16_t*, int32_t*, int, int, int);

template <int F, int MT, bool PRE>
static gemm_fn pick_ts(int ts) {
    switch (ts) {
        case 16: return qgemm_dot4_kernel<F, MT, 16, PRE>;
        case 32: return qgemm_dot4_kernel<F, MT, 32, PRE>;
        default: return qgemm_dot4_kernel<F, MT, 64, PRE>;
    }
}

template <int F>
static gemm_fn pick_mt(int mt, int ts, bool pre) {
    if (!pre) return pick_ts<F, 1, false>(ts);
    switch (mt) {
        case 1: return pick_ts<F, 1, true>(ts);
        case 2: return pick_ts<F, 2, true>(ts);
        case 4: return pick_ts<F, 4, true>(ts);
        case 8: return pick_ts<F, 8, true>(ts);
        default: return pick_ts<F, 16, true>(ts);
    }
}

static gemm_fn pick_gemm(int qtype, int mt, int ts, bool pre) {
    switch (qtype) {
        case VIPER_QTYPE_Q4_G64: return pick_mt<4>(mt, ts, pre);
        case VIPER_QTYPE_Q5_G64: return pick_mt<5>(mt, ts, pre);
        case VIPER_QTYPE_Q6_G64: return pick_mt<6>(mt, ts, pre);
        default: return pick_mt<8>(mt, ts, pre);
    }
}

// Team size: the smallest of 16/32/64 lanes that covers a row in at most
// CPL chunks per lane (longer rows loop over segments with 64 lanes).
static int choose_ts(int cpr) {
    if (cpr <= 16 * CPL) return 16;
    if (cpr <= 32 * CPL) return 32;
    return 64;
}

// ev0/ev1 (may be null) are attached to this dispatch, so they time the
// kernel itself rather than the host-side launch.
static int launch_gemm(int qtype, const void* w, const void* s, int senc, int N, int K,
                       const void* x, const void* xq, const void* xs, int M, void* y,
                       const void* res, int32_t* part, bool pre, hipStream_t st,
                       hipEvent_t ev0 = nullptr, hipEvent_t ev1 = nullptr) {
    const size_t lds = lds_bytes(qtype, M, K);
    if (lds > (size_t)LDS_MAX) return VIPER_INVALID_ARGUMENT;
    const int ck = qtype == VIPER_QTYPE_W8_G32 ? 16 : 32;
    const int ts = choose_ts(K / ck);
    const int mt = M <= 1 ? 1 : M <= 2 ? 2 : M <= 4 ? 4 : M <= 8 ? 8 : 16;
    const int rows_per_wg = NT / ts;
    const unsigned grid = (unsigned)((N + rows_per_wg - 1) / rows_per_wg);
    gemm_fn fn = pick_gemm(qtype, mt, ts, pre);
    if (ev0 == nullptr && ev1 == nullptr)
        hipLaunchKernelGGL(fn, dim3(grid), dim3(NT), lds, st, (const uint8_t*)w,
                           (const uint16_t*)s, senc, (const uint16_t*)x, (const int8_t*)xq,
                           (const float*)xs, (uint16_t*)y, (const uint16_t*)res, part, N, K, M);
    else
        hipExtLaunchKernelGGL(fn, dim3(grid), dim3(NT), (uint32_t)lds, st, ev0, ev1, 0u,
                              (const uint8_t*)w, (const uint16_t*)s, senc, (const uint16_t*)x,
                              (const int8_t*)xq, (const float*)xs, (uint16_t*)y,
                              (const uint16_t*)res, part, N, K, M);
    return status_of(hipGetLastError());
}

static int launch_quantize(int group, const void* x, int M, int K, void* xq, void* xs,
                           hipStream_t st) {
    const int oct_total = M * K / 8;
    const unsigned grid = (unsigned)((oct_total + NT - 1) / NT);
    if (group == 64)
        hipLaunchKernelGGL(quantize_act_kernel<64>, dim3(grid), dim3(NT), 0, st,
                           (const uint16_t*)x, (int8_t*)xq, (float*)xs, oct_total);
    else
        hipLaunchKernelGGL(quantize_act_kernel<32>, dim3(grid), dim3(NT), 0, st,
                           (const uint16_t*)x, (int8_t*)xq, (float*)xs, oct_total);
    return status_of(hipGetLastError());
}

static bool fused_ok(int qtype, int M, int K) {
    return M == 1 && lds_bytes(qtype, 1, K) <= (size_t)LDS_MAX;
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
    if (fused_ok(qtype, M, K))
        return launch_gemm(qtype, w, s, senc, N, K, x, nullptr, nullptr, M, y, res, part, false, st,
                           ev0, ev1);
    const size_t need = workspace_need(qtype, K, M);
    if (wsp == nullptr || wsp_bytes < need || misaligned(wsp, 16)) return VIPER_INVALID_ARGUMENT;
    if (lds_bytes(qtype, M, K) > (size_t)LDS_MAX) return VIPER_INVALID_ARGUMENT;
    uint8_t* xq = (uint8_t*)wsp;
    float* xs = (float*)(xq + align16((size_t)M * K));
    rc = launch_quantize(group, x, M, K, xq, xs, st);
    if (rc != VIPER_OK) return rc;
    return launch_gemm(qtype, w, s, senc, N, K, nullptr, xq, xs, M, y, res, part, true, st, ev0,
                       ev1);
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
    if ((int64_t)M * K > INT32_MAX) return VIPER_INVALID_ARGUMENT;
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
    return vq::launch_gemm(qtype, w_packed, w_scales, scale_enc, N, K, nullptr, xq, xs, M, y_bf16,
                           residual_bf16, nullptr, true, (hipStream_t)stream);
}

extern "C" int viper_hip_check_quantizer(int exp_lo, int exp_hi, int32_t* counts, void* stream) {
    if (counts == nullptr || exp_lo < 0 || exp_hi > 254 || exp_lo > exp_hi)
        return VIPER_INVALID_ARGUMENT;
    if (vq::misaligned(counts, 4)) return VIPER_INVALID_ARGUMENT;
    const int ab0 = exp_lo << 7;
    const unsigned grid = (unsigned)((exp_hi - exp_lo + 1) << 7);
    hipLaunchKernelGGL(vq::check_quantizer_kernel, dim3(grid), dim3(vq::NT), 0,
                       (hipStream_t)stream, ab0, counts);
    return vq::status_of(hipGetLastError());
}
