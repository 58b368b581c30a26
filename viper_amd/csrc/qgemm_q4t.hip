// M = 2..16, Q4_G64, K a multiple of 256: skinny GEMM on the i8 matrix cores
// with row-contiguous weight loads.
//
// Semantics are those of the reference's multi-row path
// (kernels/ops/linear_multim.cu:64-130): per group, the int32 dot of the
// weight codes with the int8 activations, scaled by ws * xs in fp32 and
// summed over groups.
//
// Why a second matrix-core kernel.  The MFMA operand layout (lane l holds 16
// k-values of column l % 16) makes a direct 16-byte load per lane read 64
// contiguous bytes of each of 16 weight rows per instruction; on MI355X that
// pattern streams 14 MB in 4.2 us where 8 rows x 128 bytes take 3.5 us.  Here
// every weight load instruction reads 8 rows x 128 bytes (lane l: row l / 8,
// 16-byte chunk l % 8), and each wave moves its 16 rows x 128 bytes through a
// wave-private LDS buffer into the operand layout (no workgroup barrier: a
// wave's own LDS accesses are ordered).
//
// Work split.  A workgroup owns 8 * RB weight rows (one workgroup per CU on
// the north-star shape: 40 rows, tiles of 16, 16 and 8 rows) so the activation
// is read once per CU; its W waves split K by quads of 4 groups (128 bytes of
// every row), wave v taking quads v, v + W, ...  A quad's operands are one
// 16-byte activation fragment per group (the fragment order written by
// quantize_act_kernel<64, true>, or gathered from the natural layout), the
// fp32 activation scales of the lane's 4 output rows, the lane's 4 weight
// scales (8 bytes) and the weight rows.  All small operands are requested
// before the weights.
//
// Operands.  v_mfma_i32_16x16x64_i8: lane l supplies k-slot kb = l / 16 of A
// row l % 16 (the activation) and of B column l % 16 (the weight row); the
// fragment of k-slot kb is quarter qi = bit-swap(kb) of the group, octets as
// [even k | odd k], which is the order the low/high nibble split of 8 packed
// bytes produces.  Codes u = w + 8 are multiplied as they are; one extra MFMA
// per group with B = -8 starts the accumulator at -8 * sum(q) (exact int32
// group dot).  Lane l receives C[4 * kb + r][l % 16], r = 0..3.  The W partial
// sums are added in wave order through LDS, so results do not depend on
// timing.  Two matrices of one shape may share a launch (fused pair):
// workgroups [0, nb0) use (w, ws, y), the rest (w1, ws1, y1).

#include "qlinear_host.h"

namespace vq {

constexpr int Q4T_LSTR = 136;  // transpose buffer row stride (bytes): 128 + 8 spreads banks

__host__ __device__ constexpr size_t q4t_lds_bytes(int RB, int W) {
    return (size_t)W * 16 * Q4T_LSTR + (size_t)W * ((RB + 1) / 2) * 4 * 64 * 4;
}

template <int RB, int W, int QW, bool XNAT, bool PART>
__global__ void __launch_bounds__(64 * W)
qgemm_q4t_kernel(const int8_t* xq, const float* xs, const uint8_t* w, const uint16_t* ws, uint16_t* y,
                 int K, int M, int N, int nb0, int senc, const uint16_t* res, int32_t* __restrict__ part,
                 const uint8_t* w1, const uint16_t* ws1, uint16_t* y1) {
    constexpr int T = (RB + 1) / 2;  // tiles of 16 rows (the last may hold 8)
    extern __shared__ __align__(16) uint8_t smem[];
    const int tid = (int)threadIdx.x, L = tid & 63, wave = tid >> 6;
    const int n16 = L & 15, kb = L >> 4, qi = ((kb & 1) << 1) | (kb >> 1);
    const int NG = K / 64, NQ = NG / 4;
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
    const int rbytes = K / 2;
    const auto wr = buf(w + (size_t)row0 * rbytes, (uint32_t)(nrows * rbytes));
    const auto sr = buf(ws + (size_t)row0 * NG, (uint32_t)(nrows * NG * 2));
    const auto xr = buf(xq, XNAT ? (uint32_t)(M * K) : (uint32_t)NG * 1024);
    const auto xsr = buf(xs, XNAT ? (uint32_t)(M * NG * 4) : (uint32_t)NG * 64);
    const bool m_ok = n16 < M;  // A row of this lane

    // 1. small operands of every quad, then the weights
    u32x4 A[QW][4], XS[QW][4], WV[QW][RB];
    u32x2 S[QW][T];
#pragma unroll
    for (int j = 0; j < QW; ++j) {
        const int Q = wave + W * j;
        const bool ok = Q < NQ;
#pragma unroll
        for (int h = 0; h < 4; ++h) {
            const int g = 4 * Q + h;
            if constexpr (XNAT) {
                A[j][h] = bload16(xr, (ok && m_ok) ? n16 * K + g * 64 + 16 * qi : OOB);
                uint32_t v[4];
#pragma unroll
                for (int r = 0; r < 4; ++r) v[r] = bload4(xsr, (ok && 4 * kb + r < M) ? ((4 * kb + r) * NG + g) * 4 : OOB);
                XS[j][h] = u32x4{v[0], v[1], v[2], v[3]};
            } else {
                A[j][h] = bload16(xr, (ok && m_ok) ? (g * 64 + L) * 16 : OOB);
                XS[j][h] = bload16(xsr, ok ? (g * 16 + 4 * kb) * 4 : OOB);
            }
        }
#pragma unroll
        for (int t = 0; t < T; ++t) S[j][t] = bload8(sr, ok ? ((16 * t + n16) * NG + 4 * Q) * 2 : OOB);
    }
    issue_fence();
#pragma unroll
    for (int j = 0; j < QW; ++j) {
        const int Q = wave + W * j;
        const bool ok = Q < NQ;
#pragma unroll
        for (int b = 0; b < RB; ++b)
            WV[j][b] = bload16<AUX_NT>(wr, ok ? (8 * b + (L >> 3)) * rbytes + (8 * Q + (L & 7)) * 16 : OOB);
    }

    // 2. per quad: correction MFMAs, then per tile the LDS transpose, the
    //    nibble split and one MFMA per group, scaled into fp32
    uint8_t* tb = smem + (size_t)wave * 16 * Q4T_LSTR;
    float acc[T][4];
#pragma unroll
    for (int t = 0; t < T; ++t)
#pragma unroll
        for (int r = 0; r < 4; ++r) acc[t][r] = 0.0f;
    const i32x4 BOFF = {(int)0xF8F8F8F8u, (int)0xF8F8F8F8u, (int)0xF8F8F8F8u, (int)0xF8F8F8F8u};
    auto wave_sync = [] {
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront", "local");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront", "local");
    };
#pragma unroll
    for (int j = 0; j < QW; ++j) {
        const int Q = wave + W * j;
        if (Q < NQ) {
            i32x4 Av[4], C0[4];
#pragma unroll
            for (int h = 0; h < 4; ++h) {
                u32x4 a = A[j][h];
                if constexpr (XNAT)
                    a = u32x4{__builtin_amdgcn_perm(a.y, a.x, 0x06040200u), __builtin_amdgcn_perm(a.y, a.x, 0x07050301u),
                              __builtin_amdgcn_perm(a.w, a.z, 0x06040200u), __builtin_amdgcn_perm(a.w, a.z, 0x07050301u)};
                Av[h] = i32x4{(int)a.x, (int)a.y, (int)a.z, (int)a.w};
                C0[h] = __builtin_amdgcn_mfma_i32_16x16x64_i8(Av[h], BOFF, i32x4{0, 0, 0, 0}, 0, 0, 0);
            }
#pragma unroll
            for (int t = 0; t < T; ++t) {
                *(u32x4*)(tb + (L >> 3) * Q4T_LSTR + (L & 7) * 16) = WV[j][2 * t];
                if (2 * t + 1 < RB) *(u32x4*)(tb + (8 + (L >> 3)) * Q4T_LSTR + (L & 7) * 16) = WV[j][2 * t + 1];
                wave_sync();
                u32x2 P[4];
#pragma unroll
                for (int h = 0; h < 4; ++h) P[h] = *(const u32x2*)(tb + n16 * Q4T_LSTR + h * 32 + qi * 8);
                wave_sync();
                const int n = row0 + 16 * t + n16;
#pragma unroll
                for (int h = 0; h < 4; ++h) {
                    const i32x4 B = {(int)(P[h].x & 0x0F0F0F0Fu), (int)((P[h].x >> 4) & 0x0F0F0F0Fu),
                                     (int)(P[h].y & 0x0F0F0F0Fu), (int)((P[h].y >> 4) & 0x0F0F0F0Fu)};
                    const i32x4 C = __builtin_amdgcn_mfma_i32_16x16x64_i8(Av[h], B, C0[h], 0, 0, 0);
                    const uint32_t sw = (h < 2) ? S[j][t].x : S[j][t].y;
                    const uint32_t sh = (h & 1) ? (sw >> 16) : (sw & 0xffffu);
                    const float wsf = senc ? bf16f(sh) : f16f(sh);
                    const float xf[4] = {__uint_as_float(XS[j][h].x), __uint_as_float(XS[j][h].y),
                                         __uint_as_float(XS[j][h].z), __uint_as_float(XS[j][h].w)};
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

    // 3. cross-wave sum in wave order, residual, bf16 store
    float* red = (float*)(smem + (size_t)W * 16 * Q4T_LSTR);
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

typedef void (*q4t_fn)(const int8_t*, const float*, const uint8_t*, const uint16_t*, uint16_t*, int, int, int,
                       int, int, const uint16_t*, int32_t*, const uint8_t*, const uint16_t*, uint16_t*);

// Waves per workgroup and quads per wave (one load segment covers K).
struct Q4tShape {
    int rb, w, qw;
};
constexpr int Q4T_WQ[][2] = {{4, 1}, {10, 1}, {10, 2}};

template <int RB, int W, int QW>
static q4t_fn q4t_pick3(bool xnat, bool part) {
    if (xnat) return part ? qgemm_q4t_kernel<RB, W, QW, true, true> : qgemm_q4t_kernel<RB, W, QW, true, false>;
    return part ? qgemm_q4t_kernel<RB, W, QW, false, true> : qgemm_q4t_kernel<RB, W, QW, false, false>;
}
// Two quads per wave hold RB <= 4 blocks in registers without spilling.
constexpr int Q4T_RB_QW2 = 4;
template <int RB>
static q4t_fn q4t_pick2(int w, int qw, bool xnat, bool part) {
    if (w == 4 && qw == 1) return q4t_pick3<RB, 4, 1>(xnat, part);
    if (w == 10 && qw == 1) return q4t_pick3<RB, 10, 1>(xnat, part);
    if constexpr (RB <= Q4T_RB_QW2)
        if (w == 10 && qw == 2) return q4t_pick3<RB, 10, 2>(xnat, part);
    return nullptr;
}
static q4t_fn q4t_pick(const Q4tShape& s, bool xnat, bool part) {
    switch (s.rb) {
        case 1: return q4t_pick2<1>(s.w, s.qw, xnat, part);
        case 2: return q4t_pick2<2>(s.w, s.qw, xnat, part);
        case 3: return q4t_pick2<3>(s.w, s.qw, xnat, part);
        case 4: return q4t_pick2<4>(s.w, s.qw, xnat, part);
        case 5: return q4t_pick2<5>(s.w, s.qw, xnat, part);
        case 6: return q4t_pick2<6>(s.w, s.qw, xnat, part);
        default: return nullptr;
    }
}

// Rows per workgroup: the multiple of 8 that spreads all rows (both matrices
// of a fused pair) over one workgroup per CU, at most 48; then the fewest
// waves whose quads cover K in one segment.
static Q4tShape q4t_shape(int rows_total, int NQ, int cus) {
    Q4tShape s{0, 0, 0};
    const int rb = (rows_total + 8 * cus - 1) / (8 * cus);
    s.rb = rb < 1 ? 1 : (rb > 6 ? 6 : rb);
    for (const auto& c : Q4T_WQ)
        if (c[0] * c[1] >= NQ) {
            s.w = c[0];
            s.qw = c[1];
            break;
        }
    if (s.qw > 1 && s.rb > Q4T_RB_QW2) s.rb = Q4T_RB_QW2;
    return s;
}

bool q4t_ok(int qtype, int K) {
    if (qtype != VIPER_QTYPE_Q4_G64 || K % 256 != 0) return false;
    return K / 256 <= Q4T_WQ[2][0] * Q4T_WQ[2][1];
}

int launch_q4t(const void* w, const void* s, int senc, int N, int K, const void* xq, const void* xs, bool xnat,
               int M, void* y, const void* res, int32_t* part, const void* w1, const void* s1, void* y1,
               hipStream_t st, hipEvent_t ev0, hipEvent_t ev1) {
    if (!q4t_ok(VIPER_QTYPE_Q4_G64, K) || M < 2 || M > 16) return VIPER_INTERNAL;
    const int NQ = K / 256;
    const Q4tShape sh = q4t_shape(w1 != nullptr ? 2 * N : N, NQ, device_cus());
    if (sh.w == 0) return VIPER_INTERNAL;
    const q4t_fn fn = q4t_pick(sh, xnat, part != nullptr);
    if (fn == nullptr) return VIPER_INTERNAL;
    int nb0 = (N + 8 * sh.rb - 1) / (8 * sh.rb);
    const unsigned grid = (unsigned)(w1 != nullptr ? 2 * nb0 : nb0);
    const size_t lds = q4t_lds_bytes(sh.rb, sh.w);
    const int8_t* a0 = (const int8_t*)xq;
    const float* a1 = (const float*)xs;
    const uint8_t* a2 = (const uint8_t*)w;
    const uint16_t* a3 = (const uint16_t*)s;
    uint16_t* a4 = (uint16_t*)y;
    const uint16_t* a5 = (const uint16_t*)res;
    const uint8_t* b0 = (const uint8_t*)w1;
    const uint16_t* b1 = (const uint16_t*)s1;
    uint16_t* b2 = (uint16_t*)y1;
    void* args[] = {&a0, &a1, &a2, &a3, &a4, &K, &M, &N, &nb0, &senc, &a5, &part, &b0, &b1, &b2};
    launch((const void*)fn, grid, (unsigned)(64 * sh.w), lds, st, args, ev0, ev1);
    return status_of(hipGetLastError());
}

}  // namespace vq
