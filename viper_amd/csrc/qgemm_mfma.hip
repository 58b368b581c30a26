// M = 2..16: quantized skinny GEMM on the i8 matrix cores of gfx950, for K a
// multiple of two groups that the row-contiguous kernels (qgemm_rc.h, K a
// multiple of four groups) do not take.
//
// Semantics are those of the reference's multi-row path
// (kernels/ops/linear_multim.cu:64-130): per group, the int32 dot of the
// weight codes with the int8 activations, scaled by ws * xs in fp32 and
// summed over groups.
//
// Operands.  v_mfma_i32_16x16x64_i8 (Q4/Q5/Q6: one 64-weight group per
// instruction) and v_mfma_i32_16x16x32_i8 (W8: one 32-weight group): lane l
// supplies 16 (resp. 8) k-values of row l%16 of A and of column l%16 of B, in
// k-slot l/16 (A and B use the same k-slot layout), and receives
// C[4*(l/16) + r][l%16], r = 0..3.  A is the activation tile (row m, rows
// m >= M read as zero) and B the weight tile (column n), so the lane that
// loads row n's weights and scales also owns output column n.
//
// Data movement.  A group pair is four 16-byte chunks of a weight row; lane
// slot kb = l/16 loads chunk 4p + kb with one 16-byte load, so an instruction
// reads 64 contiguous bytes of each of 16 rows.  After decoding its chunk the
// lane swaps half of it with lane l ^ 32 (v_permlane32_swap), after which
// every lane holds a quarter of group 2p and a quarter of group 2p + 1.  Lane
// slot kb's quarter starts at k = Q * (2 * (kb & 1) + (kb >> 1)) within the
// group (Q = 16, or 8 for W8), and the lane loads its activation fragment
// from there.
//
// Offset codes.  Q4/Q5/Q6 codes u = w + OFF in [0, 2*OFF) are multiplied as
// they are; one extra MFMA per group with every byte of B equal to -OFF
// starts the accumulator at -OFF * sum(q) for every column, so C is the exact
// int32 group dot.  That MFMA depends on the activations only and is shared
// by all weight tiles of the wave.
//
// Work split.  A workgroup owns T tiles of 16 weight rows and W waves; wave v
// takes group pairs p = v, v + W, v + 2W, ... (adjacent waves read adjacent
// 64-byte pieces of every row), and the W partial sums are added in wave
// order through LDS, so results do not depend on timing.  Two matrices
// of one shape may share a launch (the reference's fused2): workgroups
// [0, nb0) work on (w, ws, y), the rest on (w1, ws1, y1).

#include "qlinear_host.h"

namespace vq {

// Group pairs per wave per load segment: a single segment, or the
// double-buffered segments of the looping variant (two sets in registers).
constexpr int MF_PS_ONE = 5;
constexpr int MF_PS_LOOP = 3;
// 16-byte staging loads per thread for the activation scales (SLX) and the
// weight scales (SLW) of the staged variant.
constexpr int MF_SLX = 3;
constexpr int MF_SLW = 2;

// Activation layouts.
//  * natural (XNAT): xq [M][K] int8 in k order, xs [M][K/G] fp32, the layout
//    of viper_hip_quantize_act and of the prequantized entry point; the kernel
//    gathers fragments and scales with per-lane loads.
//  * fragment order (written by quantize_act_kernel<G, true>): for group g,
//    k-slot kb and row m, the lane's 16 (W8: 8) int8 at
//    ((g * 4 + kb) * 16 + m) * Q, octets of the nibble formats stored as
//    [even k | odd k]; one wave instruction reads a group's fragments as one
//    contiguous 1 KB (512 B).  xs as [K/G][16] fp32.  Both scale arrays are
//    staged into LDS once per workgroup with contiguous loads.
// Rows m >= M of either layout are never read into an output.

__device__ __forceinline__ void lane_swap32(uint32_t& a, uint32_t& b) {
    // lanes 32..63 of a <-> lanes 0..31 of b
    const auto r = __builtin_amdgcn_permlane32_swap(a, b, false, false);
    a = r[0];
    b = r[1];
}

// 16 activation bytes in k order -> [even | odd] per octet (the order decode()
// leaves the nibble formats' weights in).
__device__ __forceinline__ u32x4 octet_perm(const u32x4& v) {
    return u32x4{__builtin_amdgcn_perm(v.y, v.x, 0x06040200u), __builtin_amdgcn_perm(v.y, v.x, 0x07050301u),
                 __builtin_amdgcn_perm(v.w, v.z, 0x06040200u), __builtin_amdgcn_perm(v.w, v.z, 0x07050301u)};
}

__device__ __forceinline__ i32x4 as_i32x4(const u32x4& v) {
    return i32x4{(int)v.x, (int)v.y, (int)v.z, (int)v.w};
}
__device__ __forceinline__ long as_i64(uint32_t lo, uint32_t hi) {
    return (long)(((uint64_t)hi << 32) | lo);
}

__device__ __forceinline__ float scale_f(uint32_t h, int senc) {
    return senc ? bf16f(h) : f16f(h);
}

template <int F, int T, int PS>
struct MfSeg {
    u32x4 a[PS][2];    // activation fragments of groups 2p, 2p+1
    u32x4 xs[PS][2];   // natural layout: xs of rows 4*kb + r, groups 2p, 2p+1
    u32x4 w[PS][T];    // weight chunk 4p + kb of each tile row
    uint32_t h0[PS][T], h1[PS][T];  // its high-plane words (Q5, Q6)
    uint32_t s[PS][T];  // natural layout: weight scales of groups 2p (low half), 2p+1
};

// LDS of the staged variant: [red W*T*1 KB][xs NG*64][weight scales 16T*NG*2 + 16]
__host__ __device__ constexpr size_t mf_lds_bytes(bool xnat, int W, int T, int NG) {
    return (size_t)W * T * 1024 + (xnat ? 0 : (size_t)NG * 64 + (size_t)16 * T * NG * 2 + 16);
}

// ONE: every wave's pairs fit one segment (ceil(NP / W) <= MF_PS_ONE).
// XNAT: natural activation layout (else fragment order, scales staged in LDS).
// PART: also store every int32 group dot (test and debug entry point).
// Arguments: what the common path reads fits the 14 preloaded argument
// dwords (a later one is a scalar load the wave waits for): N, M - 1 and the
// scale encoding share one word (nm: N in bits 0..26, M - 1 in 27..30, the
// encoding in bit 31) and the first matrix's workgroup count is derived
// from N (both matrices of a pair have N rows).
template <int F, int T, int W, bool ONE, bool XNAT, bool PART>
__global__ void __launch_bounds__(64 * W)
qgemm_mfma_kernel(const int8_t* xq, const float* xs, const uint8_t* __restrict__ w,
                  const uint16_t* __restrict__ ws, uint16_t* y, int K, unsigned nm, const uint16_t* res,
                  int32_t* __restrict__ part, const uint8_t* __restrict__ w1, const uint16_t* __restrict__ ws1,
                  uint16_t* y1) {
    using FT = Fmt<F>;
    constexpr int PS = ONE ? MF_PS_ONE : MF_PS_LOOP;
    constexpr bool NIB = F != 8;
    constexpr int HB = FT::HIW * 4;   // high-plane bytes per chunk
    constexpr int QB = NIB ? 16 : 8;  // activation bytes per lane per group
    constexpr uint32_t BOFF = (uint32_t)(uint8_t)(-FT::OFF) * 0x01010101u;
    extern __shared__ __align__(16) uint8_t smem[];
    float* red = (float*)smem;  // [W][T][4][64]

    const int tid = (int)threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int nl = lane & 15, kb = lane >> 4;
    const int NG = K / FT::G;
    const int NP = NG / 2;
    const int CPR = K / FT::CK;
    const int cnt = (NP + W - 1) / W;
    const int nseg = ONE ? 1 : (cnt + PS - 1) / PS;
    const int N = (int)(nm & ((1u << 27) - 1)), M = (int)((nm >> 27) & 15u) + 1;
    const int senc = (int)(nm >> 31);
    const int nb0 = (N + 16 * T - 1) / (16 * T);
    int bid = (int)blockIdx.x;
    if (__builtin_expect(bid >= nb0, 0)) {  // second matrix of a fused pair
        bid -= nb0;
        w = w1;
        ws = ws1;
        y = y1;
    }
    const int row0 = bid * 16 * T;
    const int nrows = min(16 * T, N - row0);
    const uint32_t rbytes = (uint32_t)CPR * 16;
    const auto wr = buf(w + (size_t)row0 * rbytes, (uint32_t)nrows * rbytes);
    const auto hr = buf(w + (size_t)N * (K / 2) + (size_t)row0 * CPR * HB, (uint32_t)(nrows * CPR * HB));
    const bool m_ok = nl < M;

    // Staged variant: the workgroup's activation scales and weight-scale rows
    // are contiguous blocks; their loads go first (they are the first data
    // every pair needs), then every activation fragment and weight chunk.
    float* lxs = (float*)(smem + (size_t)W * T * 1024);
    uint8_t* lws = smem + (size_t)W * T * 1024 + (size_t)NG * 64;
    const uintptr_t wsa = (uintptr_t)(ws + (size_t)row0 * NG);
    const int wsd = (int)(wsa & 15);  // the block's offset in its first 16 bytes
    u32x4 stx[MF_SLX], stw[MF_SLW];
    if constexpr (!XNAT) {
        const auto xsr = buf(xs, (uint32_t)NG * 64);
        const auto sr = buf((const void*)(wsa - wsd), (uint32_t)(wsd + nrows * NG * 2));
#pragma unroll
        for (int i = 0; i < MF_SLX; ++i) stx[i] = bload16(xsr, (tid + 64 * W * i) * 16);
#pragma unroll
        for (int i = 0; i < MF_SLW; ++i) stw[i] = bload16(sr, (tid + 64 * W * i) * 16);
    }

    const auto xr = buf(xq, XNAT ? (uint32_t)(M * K) : (uint32_t)NG * 64 * QB);
    const auto xsr_nat = buf(xs, (uint32_t)(M * NG) * 4);
    const auto sr_nat = buf(ws + (size_t)row0 * NG, (uint32_t)(nrows * NG) * 2);
    const int qoff = QB * (2 * (kb & 1) + (kb >> 1));

    auto load = [&](MfSeg<F, T, PS>& S, int seg) {
#pragma unroll
        for (int j = 0; j < PS; ++j) {
            const int p = wave + W * (seg * PS + j);
            const bool pok = p < NP;
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                const int g = 2 * p + h;
                int ao;
                if constexpr (XNAT) ao = (pok && m_ok) ? nl * K + g * FT::G + qoff : OOB;
                else ao = (pok && m_ok) ? (g * 64 + lane) * QB : OOB;
                if constexpr (NIB) {
                    S.a[j][h] = bload16(xr, ao);
                } else {
                    const u32x2 v = bload8(xr, ao);
                    S.a[j][h] = u32x4{v.x, v.y, 0u, 0u};
                }
                if constexpr (XNAT) {
                    uint32_t v[4];
#pragma unroll
                    for (int r = 0; r < 4; ++r)
                        v[r] = bload4(xsr_nat, (pok && 4 * kb + r < M) ? ((4 * kb + r) * NG + g) * 4 : OOB);
                    S.xs[j][h] = u32x4{v[0], v[1], v[2], v[3]};
                }
            }
#pragma unroll
            for (int t = 0; t < T; ++t) {
                const int nr = 16 * t + nl;
                const bool ok = pok && nr < nrows;
                const int c = 4 * p + kb;
                S.w[j][t] = bload16<AUX_NT>(wr, ok ? nr * (int)rbytes + c * 16 : OOB);
                if constexpr (XNAT) S.s[j][t] = bload4(sr_nat, ok ? (nr * NG + 2 * p) * 2 : OOB);
                S.h0[j][t] = 0u;
                S.h1[j][t] = 0u;
                if constexpr (FT::HIW == 1) {
                    S.h0[j][t] = bload4<AUX_NT>(hr, ok ? (nr * CPR + c) * HB : OOB);
                } else if constexpr (FT::HIW == 2) {
                    const u32x2 hh = bload8<AUX_NT>(hr, ok ? (nr * CPR + c) * HB : OOB);
                    S.h0[j][t] = hh.x;
                    S.h1[j][t] = hh.y;
                }
            }
        }
    };

    float acc[T][4];
#pragma unroll
    for (int t = 0; t < T; ++t)
#pragma unroll
        for (int r = 0; r < 4; ++r) acc[t][r] = 0.0f;

    auto compute = [&](MfSeg<F, T, PS>& S, int seg) {
#pragma unroll
        for (int j = 0; j < PS; ++j) {
            const int p = wave + W * (seg * PS + j);
            if (p < NP) {
                i32x4 A[2], C0[2];
                u32x4 xv[2];
#pragma unroll
                for (int h = 0; h < 2; ++h) {
                    A[h] = as_i32x4((XNAT && NIB) ? octet_perm(S.a[j][h]) : S.a[j][h]);
                    C0[h] = i32x4{0, 0, 0, 0};
                    if constexpr (FT::OFF != 0)
                        C0[h] = __builtin_amdgcn_mfma_i32_16x16x64_i8(
                            A[h], i32x4{(int)BOFF, (int)BOFF, (int)BOFF, (int)BOFF}, C0[h], 0, 0, 0);
                    if constexpr (XNAT) xv[h] = S.xs[j][h];
                    else xv[h] = *(const u32x4*)(lxs + (2 * p + h) * 16 + 4 * kb);
                }
#pragma unroll
                for (int t = 0; t < T; ++t) {
                    uint32_t wd[8];
                    decode<F>(S.w[j][t], S.h0[j][t], S.h1[j][t], wd);
                    i32x4 C[2];
                    if constexpr (NIB) {
                        lane_swap32(wd[0], wd[4]);
                        lane_swap32(wd[1], wd[5]);
                        lane_swap32(wd[2], wd[6]);
                        lane_swap32(wd[3], wd[7]);
                        C[0] = __builtin_amdgcn_mfma_i32_16x16x64_i8(
                            A[0], i32x4{(int)wd[0], (int)wd[1], (int)wd[2], (int)wd[3]}, C0[0], 0, 0, 0);
                        C[1] = __builtin_amdgcn_mfma_i32_16x16x64_i8(
                            A[1], i32x4{(int)wd[4], (int)wd[5], (int)wd[6], (int)wd[7]}, C0[1], 0, 0, 0);
                    } else {
                        lane_swap32(wd[0], wd[2]);
                        lane_swap32(wd[1], wd[3]);
                        C[0] = __builtin_amdgcn_mfma_i32_16x16x32_i8(
                            as_i64((uint32_t)A[0].x, (uint32_t)A[0].y), as_i64(wd[0], wd[1]), C0[0], 0, 0, 0);
                        C[1] = __builtin_amdgcn_mfma_i32_16x16x32_i8(
                            as_i64((uint32_t)A[1].x, (uint32_t)A[1].y), as_i64(wd[2], wd[3]), C0[1], 0, 0, 0);
                    }
                    const int n = row0 + 16 * t + nl;
                    uint32_t sv;
                    if constexpr (XNAT) sv = S.s[j][t];
                    else sv = *(const uint32_t*)(lws + wsd + ((16 * t + nl) * NG + 2 * p) * 2);
#pragma unroll
                    for (int h = 0; h < 2; ++h) {
                        const float wsf = scale_f(h ? (sv >> 16) : (sv & 0xffffu), senc);
                        const float xf[4] = {__uint_as_float(xv[h].x), __uint_as_float(xv[h].y),
                                             __uint_as_float(xv[h].z), __uint_as_float(xv[h].w)};
#pragma unroll
                        for (int r = 0; r < 4; ++r)
                            acc[t][r] = __builtin_fmaf(wsf * xf[r], (float)C[h][r], acc[t][r]);
                        if constexpr (PART) {
                            if (n < N) {
                                const int g = 2 * p + h;
#pragma unroll
                                for (int r = 0; r < 4; ++r)
                                    if (4 * kb + r < M) part[((size_t)(4 * kb + r) * N + n) * NG + g] = C[h][r];
                            }
                        }
                    }
                }
            }
        }
    };

    auto stage = [&]() {
        if constexpr (!XNAT) {
            const int nws = (wsd + nrows * NG * 2 + 15) / 16;
#pragma unroll
            for (int i = 0; i < MF_SLX; ++i) {
                const int u = tid + 64 * W * i;
                if (u < NG * 4) *(u32x4*)((uint8_t*)lxs + u * 16) = stx[i];
            }
#pragma unroll
            for (int i = 0; i < MF_SLW; ++i) {
                const int u = tid + 64 * W * i;
                if (u < nws) *(u32x4*)(lws + u * 16) = stw[i];
            }
            lds_barrier();
        }
    };

    if constexpr (ONE) {
        MfSeg<F, T, PS> S;
        load(S, 0);
        stage();
        compute(S, 0);
    } else {
        MfSeg<F, T, PS> S0, S1;
        load(S0, 0);
        stage();
        for (int seg = 0; seg < nseg; seg += 2) {
            load(S1, seg + 1);  // past the last segment every load is out of range: no traffic
            compute(S0, seg);
            load(S0, seg + 2);
            compute(S1, seg + 1);
        }
    }

    // cross-wave sum in wave order
#pragma unroll
    for (int t = 0; t < T; ++t)
#pragma unroll
        for (int r = 0; r < 4; ++r) red[((wave * T + t) * 4 + r) * 64 + lane] = acc[t][r];
    __syncthreads();
    for (int sl = wave; sl < 4 * T; sl += W) {
        const int t = sl >> 2, r = sl & 3;
        float v = 0.0f;
#pragma unroll
        for (int u = 0; u < W; ++u) v += red[((u * T + t) * 4 + r) * 64 + lane];
        const int m = 4 * kb + r, n = row0 + 16 * t + nl;
        if (m < M && n < N) {
            const size_t o = (size_t)m * N + n;
            if (res != nullptr) v += bf16f(res[o]);
            y[o] = f2bf(v);
        }
    }
}

// ------------------------------------------------------------------ host side

typedef void (*mf_fn)(const int8_t*, const float*, const uint8_t*, const uint16_t*, uint16_t*, int, unsigned,
                      const uint16_t*, int32_t*, const uint8_t*, const uint16_t*, uint16_t*);

struct MfShape {
    int t, w;
};

template <int F, bool ONE, bool XNAT, bool PART>
static mf_fn mf_kernel_v(int t, int w) {
#define VQ_MF(T_, W_) \
    if (t == T_ && w == W_) return qgemm_mfma_kernel<F, T_, W_, ONE, XNAT, PART>;
    VQ_MF(1, 4) VQ_MF(1, 8) VQ_MF(2, 4) VQ_MF(2, 8)
#undef VQ_MF
    return nullptr;
}
template <int F, bool PART>
static mf_fn mf_kernel_p(int t, int w, bool one, bool xnat) {
    if (one) return xnat ? mf_kernel_v<F, true, true, PART>(t, w) : mf_kernel_v<F, true, false, PART>(t, w);
    return xnat ? mf_kernel_v<F, false, true, PART>(t, w) : mf_kernel_v<F, false, false, PART>(t, w);
}
template <int F>
static mf_fn mf_kernel(int t, int w, bool one, bool xnat, bool part) {
    return part ? mf_kernel_p<F, true>(t, w, one, xnat) : mf_kernel_p<F, false>(t, w, one, xnat);
}

// Tiles of 16 rows per workgroup and waves per workgroup: two tiles per wave
// when that still leaves at least 2 workgroups per CU, then the fewest waves
// whose pairs fit one load segment (else 8).
static MfShape mf_shape(int N, int NP, int cus) {
    const int tiles = (N + 15) / 16;
    MfShape s{tiles >= 4 * cus ? 2 : 1, 8};
    if ((NP + 3) / 4 <= MF_PS_ONE) s.w = 4;
    return s;
}

bool mfma_ok(int qtype, int K, int M, const void* s) {
    const int G = group_of(qtype);
    return M >= 2 && G != 0 && K % (2 * G) == 0 && !misaligned(s, 4);
}

// The staged variant holds the workgroup's scales in LDS and loads them with
// MF_SLX + MF_SLW 16-byte loads per thread.
static bool staged_fits(int NG, MfShape sh) {
    const int nthr = 64 * sh.w;
    return NG * 4 <= MF_SLX * nthr && (16 * sh.t * NG * 2 + 16 + 15) / 16 <= MF_SLW * nthr &&
           mf_lds_bytes(false, sh.w, sh.t, NG) <= (size_t)LDS_MAX;
}

bool mfma_staged(int qtype, int N, int K) {
    if (rc_ok(qtype, K)) return true;  // reads fragments straight from the workspace
    const int G = group_of(qtype);
    if (G == 0) return false;
    const int NG = K / G;
    return staged_fits(NG, mf_shape(N, NG / 2, device_cus()));
}

int launch_mfma(int qtype, const void* w, const void* s, int senc, int N, int K, const void* xq,
                const void* xs, bool xnat, int M, void* y, const void* res, int32_t* part,
                const void* w1, const void* s1, void* y1, hipStream_t st, uint64_t* sp, unsigned* sc) {
    if (!mfma_ok(qtype, K, M, s)) return VIPER_INTERNAL;
    if (rc_ok(qtype, K))
        return launch_rc(qtype, w, s, senc, N, K, xq, xs, xnat ? RC_NAT : RC_FRAG, M, y, res, part, w1, s1, y1, st, sp, sc);
    if (sp != nullptr) return VIPER_INTERNAL;
    const int NG = K / group_of(qtype);
    const int NP = NG / 2;
    const MfShape sh = mf_shape(N, NP, device_cus());
    if (!xnat && !staged_fits(NG, sh)) return VIPER_INTERNAL;
    const bool one = (NP + sh.w - 1) / sh.w <= MF_PS_ONE;
    mf_fn fn;
    switch (qtype) {
        case VIPER_QTYPE_Q4_G64: fn = mf_kernel<4>(sh.t, sh.w, one, xnat, part != nullptr); break;
        case VIPER_QTYPE_Q5_G64: fn = mf_kernel<5>(sh.t, sh.w, one, xnat, part != nullptr); break;
        case VIPER_QTYPE_Q6_G64: fn = mf_kernel<6>(sh.t, sh.w, one, xnat, part != nullptr); break;
        default: fn = mf_kernel<8>(sh.t, sh.w, one, xnat, part != nullptr); break;
    }
    if (fn == nullptr) return VIPER_INTERNAL;
    int nb0 = (N + 16 * sh.t - 1) / (16 * sh.t);
    const unsigned grid = (unsigned)(w1 != nullptr ? 2 * nb0 : nb0);
    const size_t lds = mf_lds_bytes(xnat, sh.w, sh.t, NG);
    const uint8_t* a0 = (const uint8_t*)w;
    const uint16_t* a1 = (const uint16_t*)s;
    const int8_t* a3 = (const int8_t*)xq;
    const float* a4 = (const float*)xs;
    uint16_t* a5 = (uint16_t*)y;
    const uint16_t* a6 = (const uint16_t*)res;
    const uint8_t* b0 = (const uint8_t*)w1;
    const uint16_t* b1 = (const uint16_t*)s1;
    uint16_t* b2 = (uint16_t*)y1;
    if (N >= (1 << 27)) return VIPER_INVALID_ARGUMENT;  // N shares a word with M and the encoding
    unsigned nm = (unsigned)N | ((unsigned)(M - 1) << 27) | (senc ? 1u << 31 : 0u);
    void* args[] = {&a3, &a4, &a0, &a1, &a5, &K, &nm, &a6, &part, &b0, &b1, &b2};
    launch((const void*)fn, grid, (unsigned)(64 * sh.w), lds, st, args);
    return status_of(hipGetLastError());
}

}  // namespace vq
