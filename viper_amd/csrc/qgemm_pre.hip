#include "qlinear_host.h"

namespace vq {

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

int launch_pre(int qtype, const void* w, const void* s, int senc, int N, int K,
                      const void* xq, const void* xs, int M, void* y, const void* res,
                      int32_t* part, hipStream_t st) {
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
    launch((const void*)fn, grid, NT, lds, st, args);
    return status_of(hipGetLastError());
}

}  // namespace vq
