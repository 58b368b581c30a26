// M = 1 quantized GEMV kernel (one template, instantiated per format in
// qgemv_m1_q4.hip ... qgemv_m1_w8.hip so the formats compile in parallel).
#pragma once

#include "qlinear_host.h"

namespace vq {

// ------------------------------------------------------- M = 1, fused quantize
//
// The activation arrives as bf16 and is quantized in the prologue, or (PRE)
// arrives already quantized (int8 in k order + fp32 group scales, the
// layout of viper_hip_quantize_act) and is only rearranged into LDS.
//
// Two matrices of one shape may share a launch (the reference's fused2):
// workgroups [0, nb0) work on (w, ws, y), the rest on (w1, ws1, y1).
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

// EXACT: every lane's chunks of every slot lie inside its row (the row has
// exactly TS * M1_CPL chunks), so no chunk needs masking.
// DELAY: s_sleep units (64 clocks) between issuing the activation loads and
// the weight loads.  The activation is a few KB read by every workgroup; a
// short head start lets its requests through the memory pipeline before the
// weight stream saturates it, which moves every workgroup's barrier earlier.
template <int F, int TS, int NTT, int SENC, bool PART, bool EXACT, bool PRE, int DELAY>
__global__ void __launch_bounds__(NTT)
qgemv_m1_kernel(const uint8_t* __restrict__ w, const uint16_t* __restrict__ ws,
                const void* __restrict__ x, const float* __restrict__ xsc, uint16_t* y,
                const uint16_t* res, int32_t* __restrict__ part, int N, int K,
                const uint8_t* __restrict__ w1, const uint16_t* __restrict__ ws1, uint16_t* y1,
                int nb0) {
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
    int bid = (int)blockIdx.x;
    if (bid >= nb0) {  // second matrix of a fused pair
        bid -= nb0;
        w = w1;
        ws = ws1;
        y = y1;
    }
    const int row0 = bid * ROWS;
    const int row = row0 + rr;
    const int nrows = min(ROWS, N - row0);
    const bool row_ok = rr < nrows;

    // 1. activation octets, then every weight byte and group scale of the
    //    first row segment, all in flight at once
    const int noct = K / 8;
    constexpr int OPG = FT::G / 8;   // octets per group
    const auto xr = buf(x, (uint32_t)K * (PRE ? 1 : 2));
    const auto xsr = buf(xsc, PRE ? (uint32_t)(K / FT::G) * 4 : 0u);
    // bf16 octet, or {int8 octet, int8 octet, group scale of a chunk's first octet}
    auto load_x = [&](int o) -> u32x4 {
        if constexpr (PRE) {
            const u32x2 q = bload8(xr, o * 8);
            const uint32_t sb = bload4(xsr, (o % OPC == 0) ? (o / OPG) * 4 : OOB);
            return u32x4{q.x, q.y, sb, 0u};
        } else {
            return bload16(xr, o * 16);
        }
    };
    u32x4 xv[XS];
#pragma unroll
    for (int i = 0; i < XS; ++i) xv[i] = load_x(tid + NTT * i);
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
        if constexpr (PRE) {
            d0 = v.x;
            d1 = v.y;
            if constexpr (F == 5 || F == 6) {
                d0 = __builtin_amdgcn_perm(v.y, v.x, 0x06040200u);
                d1 = __builtin_amdgcn_perm(v.y, v.x, 0x07050301u);
            }
            s = __uint_as_float(v.z);
        } else {
            quantize_octet<FT::G, (F == 5 || F == 6)>(v, d0, d1, s);
        }
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
        if (wave0 + NTT * i < noct) quant_store(tid + NTT * i, load_x(tid + NTT * i));

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

typedef void (*m1_fn)(const uint8_t*, const uint16_t*, const void*, const float*, uint16_t*,
                      const uint16_t*, int32_t*, int, int, const uint8_t*, const uint16_t*, uint16_t*,
                      int);

// Launch shapes instantiated for every format: (team size, workgroup size).
constexpr int M1_SHAPES[][2] = {{8, 320}, {16, 256}, {16, 640}, {32, 320}, {32, 640}, {64, 640}};

template <int F, int SENC, bool PART, bool EXACT, bool PRE>
m1_fn m1_kernel_v(int ts, int ntt) {
#define VQ_M1(TS_, NTT_) \
    if (ts == TS_ && ntt == NTT_) return qgemv_m1_kernel<F, TS_, NTT_, SENC, PART, EXACT, PRE, M1_DELAY>;
    VQ_M1(8, 320) VQ_M1(16, 256) VQ_M1(16, 640) VQ_M1(32, 320) VQ_M1(32, 640) VQ_M1(64, 640)
#undef VQ_M1
    return nullptr;
}

// Kernel for format F (defined in that format's translation unit).
template <int F>
m1_fn m1_pick(int ts, int ntt, int senc, bool part, bool exact, bool pre);

#define VQ_M1_PICK(F)                                                                              \
    template <bool PRE>                                                                            \
    static m1_fn m1_pick_e(int ts, int ntt, int senc, bool part, bool exact) {                     \
        if (exact) {                                                                               \
            if (senc) return part ? m1_kernel_v<F, 1, true, true, PRE>(ts, ntt)                    \
                                  : m1_kernel_v<F, 1, false, true, PRE>(ts, ntt);                  \
            return part ? m1_kernel_v<F, 0, true, true, PRE>(ts, ntt)                              \
                        : m1_kernel_v<F, 0, false, true, PRE>(ts, ntt);                            \
        }                                                                                          \
        if (senc) return part ? m1_kernel_v<F, 1, true, false, PRE>(ts, ntt)                       \
                              : m1_kernel_v<F, 1, false, false, PRE>(ts, ntt);                     \
        return part ? m1_kernel_v<F, 0, true, false, PRE>(ts, ntt)                                 \
                    : m1_kernel_v<F, 0, false, false, PRE>(ts, ntt);                               \
    }                                                                                              \
    template <>                                                                                    \
    m1_fn m1_pick<F>(int ts, int ntt, int senc, bool part, bool exact, bool pre) {                 \
        return pre ? m1_pick_e<true>(ts, ntt, senc, part, exact)                                   \
                   : m1_pick_e<false>(ts, ntt, senc, part, exact);                                 \
    }

}  // namespace vq
