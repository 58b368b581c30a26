// M = 2..16 skinny GEMM on the i8 matrix cores with row-contiguous weight
// loads (one template, instantiated per format in qgemm_rc_{q4,q5,q6,w8}.hip).
//
// Semantics are those of the reference's multi-row path
// (kernels/ops/linear_multim.cu:64-130): per group, the int32 dot of the
// weight codes with the int8 activations, scaled by ws * xs in fp32 and
// summed over groups.
//
// Why row-contiguous loads.  The MFMA operand layout (lane l holds 16 k-values
// of column l % 16) makes a direct 16-byte load per lane read 64 contiguous
// bytes of each of 16 weight rows per instruction; on MI355X that pattern
// streams 14 MB in 4.2 us where 8 rows x 128 bytes take 3.5 us.  Here every
// main-plane load instruction reads 8 rows x 128 bytes (lane l: row l / 8,
// 16-byte chunk l % 8), and each wave moves its 16 rows x 128 bytes through a
// wave-private LDS buffer into the operand layout (no workgroup barrier: a
// wave's own LDS accesses are ordered).  The high planes of Q5/Q6 (32 / 64
// bytes per row per quad) take the same route through a second buffer.
//
// Work split.  A workgroup owns 8 * RB weight rows (one workgroup per CU on
// the north-star shape: 40 rows, tiles of 16, 16 and 8 rows) so the activation
// is read once per CU; its W waves split K by quads of 4 groups (128 bytes of
// every row's main plane), wave v taking quads v, v + W, ...  QW quads of a
// wave form a load segment; with several segments (long K) the next
// segment's loads are issued before the current one is computed.  A quad's
// operands are one activation fragment per group (the fragment order written
// by the fragment quantize, or gathered from the natural layout), the fp32
// activation scales of the lane's 4 output rows, the lane's 4 weight scales
// (8 bytes) and the weight rows; the small operands are requested first.
//
// Operands.  v_mfma_i32_16x16x64_i8 (Q4/Q5/Q6: one 64-group) or
// v_mfma_i32_16x16x32_i8 (W8: one 32-group): lane l supplies k-slot
// kb = l / 16 of A row l % 16 (the activation) and of B column l % 16 (the
// weight row); the fragment of k-slot kb is quarter qi = bit-swap(kb) of the
// group (octets of the nibble formats as [even k | odd k], the order the
// low/high nibble split of packed bytes produces).  Offset codes u = w + OFF
// are multiplied as they are; one extra MFMA per group with B = -OFF starts
// the accumulator at -OFF * sum(q) (exact int32 group dot).  Lane l receives
// C[4 * kb + r][l % 16], r = 0..3.  The W partial sums are added in wave order
// through LDS, so results do not depend on timing.  Two matrices of one shape
// may share a launch (fused pair): workgroups [0, nb0) use (w, ws, y), the
// rest (w1, ws1, y1).
#pragma once

#include "qlinear_host.h"

namespace vq {

// Per format: A-fragment bytes per lane and group, high-plane bytes per row
// per quad (and their LDS row stride), code offset.
template <int F> struct RcFmt;
template <> struct RcFmt<4> { static constexpr int QB = 16, HQ = 0, HSTR = 0, OFF = 8; };
template <> struct RcFmt<5> { static constexpr int QB = 16, HQ = 32, HSTR = 36, OFF = 16; };
template <> struct RcFmt<6> { static constexpr int QB = 16, HQ = 64, HSTR = 72, OFF = 32; };
template <> struct RcFmt<8> { static constexpr int QB = 8, HQ = 0, HSTR = 0, OFF = 0; };

constexpr int RC_LSTR = 136;  // main-plane transpose row stride (bytes): 128 + 8 spreads banks

__host__ __device__ constexpr size_t rc_wave_lds(int hstr) { return (size_t)16 * (RC_LSTR + hstr); }
__host__ __device__ constexpr size_t rc_lds_bytes(int hstr, int RB, int W) {
    return (size_t)W * rc_wave_lds(hstr) + (size_t)W * ((RB + 1) / 2) * 4 * 64 * 4;
}

template <int F, int RB, int QW>
struct RcSeg {
    static constexpr int T = (RB + 1) / 2;
    static constexpr int HW = RcFmt<F>::HQ / 32 > 0 ? RcFmt<F>::HQ / 32 : 1;  // high words per lane and block
    u32x4 A[QW][4], XS[QW][4], WV[QW][RB];
    uint32_t HV[QW][RB][HW];
    u32x2 S[QW][T];
};

// ONE: the quads of every wave fit one load segment.
template <int F, int RB, int W, int QW, bool ONE, bool XNAT, bool PART>
__global__ void __launch_bounds__(64 * W)
qgemm_rc_kernel(const int8_t* xq, const float* xs, const uint8_t* w, const uint16_t* ws, uint16_t* y, int K,
                int M, int N, int nb0, int senc, const uint16_t* res, int32_t* __restrict__ part,
                const uint8_t* w1, const uint16_t* ws1, uint16_t* y1) {
    using FM = RcFmt<F>;
    using Seg = RcSeg<F, RB, QW>;
    constexpr int T = Seg::T;
    constexpr int G = F == 8 ? 32 : 64;
    extern __shared__ __align__(16) uint8_t smem[];
    const int tid = (int)threadIdx.x, L = tid & 63, wave = tid >> 6;
    const int n16 = L & 15, kb = L >> 4, qi = ((kb & 1) << 1) | (kb >> 1);
    const int NG = K / G, NQ = NG / 4;
    const int nseg = ONE ? 1 : (NQ + W * QW - 1) / (W * QW);
    int bid = (int)blockIdx.x;
    if (bid >= nb0) {
        bid -= nb0;
        w = w1;
        ws = ws1;
        y = y1;
        res = nullptr;
    }
    const int row0 = bid * 8 * RB;
    const int nrows = min(8 * RB, N - row0);
    const int rbytes = NG * 32;              // main plane: 32 bytes per group
    const int hrb = NG * (FM::HQ / 4);       // high plane: HQ / 4 bytes per group
    const auto wr = buf(w + (size_t)row0 * rbytes, (uint32_t)(nrows * rbytes));
    const auto hr = buf(w + (size_t)N * rbytes + (size_t)row0 * hrb, (uint32_t)(nrows * hrb));
    const auto sr = buf(ws + (size_t)row0 * NG, (uint32_t)(nrows * NG * 2));
    const auto xr = buf(xq, XNAT ? (uint32_t)(M * K) : (uint32_t)NG * 64 * FM::QB);
    const auto xsr = buf(xs, XNAT ? (uint32_t)(M * NG * 4) : (uint32_t)NG * 64);
    const bool m_ok = n16 < M;  // A row of this lane

    auto load = [&](Seg& S, int seg) {
#pragma unroll
        for (int j = 0; j < QW; ++j) {
            const int Q = wave + W * (seg * QW + j);
            const bool ok = Q < NQ;
#pragma unroll
            for (int h = 0; h < 4; ++h) {
                const int g = 4 * Q + h;
                int ao;
                if constexpr (XNAT) ao = (ok && m_ok) ? n16 * K + g * G + FM::QB * qi : OOB;
                else ao = (ok && m_ok) ? (g * 64 + L) * FM::QB : OOB;
                if constexpr (FM::QB == 16) {
                    S.A[j][h] = bload16(xr, ao);
                } else {
                    const u32x2 v = bload8(xr, ao);
                    S.A[j][h] = u32x4{v.x, v.y, 0u, 0u};
                }
                if constexpr (XNAT) {
                    uint32_t v[4];
#pragma unroll
                    for (int r = 0; r < 4; ++r)
                        v[r] = bload4(xsr, (ok && 4 * kb + r < M) ? ((4 * kb + r) * NG + g) * 4 : OOB);
                    S.XS[j][h] = u32x4{v[0], v[1], v[2], v[3]};
                } else {
                    S.XS[j][h] = bload16(xsr, ok ? (g * 16 + 4 * kb) * 4 : OOB);
                }
            }
#pragma unroll
            for (int t = 0; t < T; ++t) S.S[j][t] = bload8(sr, ok ? ((16 * t + n16) * NG + 4 * Q) * 2 : OOB);
        }
        issue_fence();
#pragma unroll
        for (int j = 0; j < QW; ++j) {
            const int Q = wave + W * (seg * QW + j);
            const bool ok = Q < NQ;
#pragma unroll
            for (int b = 0; b < RB; ++b) {
                const int rw = 8 * b + (L >> 3);
                S.WV[j][b] = bload16<AUX_NT>(wr, ok ? rw * rbytes + (8 * Q + (L & 7)) * 16 : OOB);
                if constexpr (FM::HQ == 32) {
                    S.HV[j][b][0] = bload4<AUX_NT>(hr, ok ? rw * hrb + Q * 32 + (L & 7) * 4 : OOB);
                } else if constexpr (FM::HQ == 64) {
                    const u32x2 hh = bload8<AUX_NT>(hr, ok ? rw * hrb + Q * 64 + (L & 7) * 8 : OOB);
                    S.HV[j][b][0] = hh.x;
                    S.HV[j][b][1] = hh.y;
                }
            }
        }
    };

    uint8_t* tb = smem + (size_t)wave * rc_wave_lds(FM::HSTR);
    uint8_t* hb = tb + 16 * RC_LSTR;
    float acc[T][4];
#pragma unroll
    for (int t = 0; t < T; ++t)
#pragma unroll
        for (int r = 0; r < 4; ++r) acc[t][r] = 0.0f;
    constexpr uint32_t BOFF = (uint32_t)(uint8_t)(-FM::OFF) * 0x01010101u;
    auto wave_sync = [] {
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront", "local");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront", "local");
    };
    // high-plane word(s) of the lane's quarter: Q5 shifted so decode_word<5, 0/1>
    // applies, Q6 the word of the quarter's dwords
    const int i0 = 2 * (qi & 1);  // first dword of the quarter within its 16-byte chunk

    auto compute = [&](Seg& S, int seg) {
#pragma unroll
        for (int j = 0; j < QW; ++j) {
            const int Q = wave + W * (seg * QW + j);
            if (Q < NQ) {
                i32x4 Av[4], C0[4];
#pragma unroll
                for (int h = 0; h < 4; ++h) {
                    u32x4 a = S.A[j][h];
                    if constexpr (XNAT && F != 8)
                        a = u32x4{__builtin_amdgcn_perm(a.y, a.x, 0x06040200u), __builtin_amdgcn_perm(a.y, a.x, 0x07050301u),
                                  __builtin_amdgcn_perm(a.w, a.z, 0x06040200u), __builtin_amdgcn_perm(a.w, a.z, 0x07050301u)};
                    Av[h] = i32x4{(int)a.x, (int)a.y, (int)a.z, (int)a.w};
                    C0[h] = i32x4{0, 0, 0, 0};
                    if constexpr (FM::OFF != 0)
                        C0[h] = __builtin_amdgcn_mfma_i32_16x16x64_i8(
                            Av[h], i32x4{(int)BOFF, (int)BOFF, (int)BOFF, (int)BOFF}, C0[h], 0, 0, 0);
                }
#pragma unroll
                for (int t = 0; t < T; ++t) {
                    *(u32x4*)(tb + (L >> 3) * RC_LSTR + (L & 7) * 16) = S.WV[j][2 * t];
                    if (2 * t + 1 < RB) *(u32x4*)(tb + (8 + (L >> 3)) * RC_LSTR + (L & 7) * 16) = S.WV[j][2 * t + 1];
                    if constexpr (FM::HQ == 32) {
                        *(uint32_t*)(hb + (L >> 3) * FM::HSTR + (L & 7) * 4) = S.HV[j][2 * t][0];
                        if (2 * t + 1 < RB) *(uint32_t*)(hb + (8 + (L >> 3)) * FM::HSTR + (L & 7) * 4) = S.HV[j][2 * t + 1][0];
                    } else if constexpr (FM::HQ == 64) {
                        *(u32x2*)(hb + (L >> 3) * FM::HSTR + (L & 7) * 8) = u32x2{S.HV[j][2 * t][0], S.HV[j][2 * t][1]};
                        if (2 * t + 1 < RB)
                            *(u32x2*)(hb + (8 + (L >> 3)) * FM::HSTR + (L & 7) * 8) =
                                u32x2{S.HV[j][2 * t + 1][0], S.HV[j][2 * t + 1][1]};
                    }
                    wave_sync();
                    u32x2 P[4];
                    uint32_t H[4];
#pragma unroll
                    for (int h = 0; h < 4; ++h) {
                        P[h] = *(const u32x2*)(tb + n16 * RC_LSTR + h * 32 + qi * 8);
                        H[h] = 0u;
                        // the quarter's 16-byte chunk within the quad: 2h + (qi >> 1)
                        if constexpr (FM::HQ == 32) {
                            H[h] = *(const uint32_t*)(hb + n16 * FM::HSTR + (2 * h + (qi >> 1)) * 4) >> (2 * i0);
                        } else if constexpr (FM::HQ == 64) {
                            const u32x2 hh = *(const u32x2*)(hb + n16 * FM::HSTR + (2 * h + (qi >> 1)) * 8);
                            H[h] = i0 ? hh.y : hh.x;
                        }
                    }
                    wave_sync();
                    const int n = row0 + 16 * t + n16;
#pragma unroll
                    for (int h = 0; h < 4; ++h) {
                        i32x4 C;
                        if constexpr (F == 8) {
                            C = __builtin_amdgcn_mfma_i32_16x16x32_i8(
                                (long)(((uint64_t)(uint32_t)Av[h].y << 32) | (uint32_t)Av[h].x),
                                (long)(((uint64_t)P[h].y << 32) | P[h].x), C0[h], 0, 0, 0);
                        } else {
                            uint32_t wd[4];
                            decode_word<F, 0>(P[h].x, H[h], H[h], wd);
                            decode_word<F, 1>(P[h].y, H[h], H[h], wd);
                            C = __builtin_amdgcn_mfma_i32_16x16x64_i8(
                                Av[h], i32x4{(int)wd[0], (int)wd[1], (int)wd[2], (int)wd[3]}, C0[h], 0, 0, 0);
                        }
                        const uint32_t sw = (h < 2) ? S.S[j][t].x : S.S[j][t].y;
                        const uint32_t sh = (h & 1) ? (sw >> 16) : (sw & 0xffffu);
                        const float wsf = senc ? bf16f(sh) : f16f(sh);
                        const float xf[4] = {__uint_as_float(S.XS[j][h].x), __uint_as_float(S.XS[j][h].y),
                                             __uint_as_float(S.XS[j][h].z), __uint_as_float(S.XS[j][h].w)};
#pragma unroll
                        for (int r = 0; r < 4; ++r) acc[t][r] = __builtin_fmaf(wsf * xf[r], (float)C[r], acc[t][r]);
                        if constexpr (PART) {
                            if (16 * t + n16 < nrows) {
#pragma unroll
                                for (int r = 0; r < 4; ++r)
                                    if (4 * kb + r < M) part[((size_t)(4 * kb + r) * N + n) * NG + 4 * Q + h] = C[r];
                            }
                        }
                    }
                }
            }
        }
    };

    if constexpr (ONE) {
        Seg S;
        load(S, 0);
        compute(S, 0);
    } else {
        Seg S0, S1;
        load(S0, 0);
        for (int seg = 0; seg < nseg; seg += 2) {
            load(S1, seg + 1);  // past the last segment every load is out of range: no traffic
            compute(S0, seg);
            load(S0, seg + 2);
            compute(S1, seg + 1);
        }
    }

    // cross-wave sum in wave order, residual, bf16 store
    float* red = (float*)(smem + (size_t)W * rc_wave_lds(FM::HSTR));
#pragma unroll
    for (int t = 0; t < T; ++t)
#pragma unroll
        for (int r = 0; r < 4; ++r) red[((wave * T + t) * 4 + r) * 64 + L] = acc[t][r];
    __syncthreads();
    for (int sl = wave; sl < 4 * T; sl += W) {
        const int t = sl >> 2, r = sl & 3;
        float v = 0.0f;
#pragma unroll
        for (int u = 0; u < W; ++u) v += red[((u * T + t) * 4 + r) * 64 + L];
        const int m = 4 * kb + r, nl = 16 * t + n16;
        if (m < M && nl < nrows) {
            const size_t o = (size_t)m * N + row0 + nl;
            if (res != nullptr) v += bf16f(res[o]);
            y[o] = f2bf(v);
        }
    }
}

// ------------------------------------------------------------------ host side

typedef void (*rc_fn)(const int8_t*, const float*, const uint8_t*, const uint16_t*, uint16_t*, int, int, int,
                      int, int, const uint16_t*, int32_t*, const uint8_t*, const uint16_t*, uint16_t*);

// Launch shape: rows per workgroup (8 * rb), waves, quads per wave per
// segment, single segment or double-buffered loop.
struct RcShape {
    int rb, w, qw;
    bool one;
};
// Most 8-row blocks per workgroup that two quads per wave, or the
// double-buffered segment loop, hold in registers without spilling.
__host__ __device__ constexpr int rc_rb_qw2(int F) { return F == 8 ? 6 : F == 6 ? 3 : 4; }
constexpr int RC_RB_LOOP = 2;

template <int F, int RB, int W, int QW, bool ONE>
rc_fn rc_pick4(bool xnat, bool part) {
    if (xnat)
        return part ? qgemm_rc_kernel<F, RB, W, QW, ONE, true, true> : qgemm_rc_kernel<F, RB, W, QW, ONE, true, false>;
    return part ? qgemm_rc_kernel<F, RB, W, QW, ONE, false, true> : qgemm_rc_kernel<F, RB, W, QW, ONE, false, false>;
}
template <int F, int RB>
rc_fn rc_pick3(const RcShape& s, bool xnat, bool part) {
    if (s.one && s.w == 4 && s.qw == 1) return rc_pick4<F, RB, 4, 1, true>(xnat, part);
    if (s.one && s.w == 10 && s.qw == 1) return rc_pick4<F, RB, 10, 1, true>(xnat, part);
    if constexpr (RB <= rc_rb_qw2(F))
        if (s.one && s.w == 10 && s.qw == 2) return rc_pick4<F, RB, 10, 2, true>(xnat, part);
    if constexpr (RB <= RC_RB_LOOP)
        if (!s.one && s.w == 10 && s.qw == 1) return rc_pick4<F, RB, 10, 1, false>(xnat, part);
    return nullptr;
}
template <int F>
rc_fn rc_pick2(const RcShape& s, bool xnat, bool part) {
    switch (s.rb) {
        case 1: return rc_pick3<F, 1>(s, xnat, part);
        case 2: return rc_pick3<F, 2>(s, xnat, part);
        case 3: return rc_pick3<F, 3>(s, xnat, part);
        case 4: return rc_pick3<F, 4>(s, xnat, part);
        case 5: return rc_pick3<F, 5>(s, xnat, part);
        case 6: return rc_pick3<F, 6>(s, xnat, part);
        default: return nullptr;
    }
}

// Kernels of format F (each defined in its own translation unit).
template <int F>
rc_fn rc_pick(const RcShape& s, bool xnat, bool part);

#define VQ_RC_PICK(F) \
    template <>       \
    rc_fn rc_pick<F>(const RcShape& s, bool xnat, bool part) { return rc_pick2<F>(s, xnat, part); }

}  // namespace vq
