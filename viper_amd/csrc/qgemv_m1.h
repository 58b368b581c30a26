// M = 1 quantized GEMV kernel (one template, instantiated per format in
// qgemv_m1_q4.hip ... qgemv_m1_w8.hip so the formats compile in parallel).
#pragma once

#include <cstddef>

#include "qlinear_host.h"

namespace vq {

// ------------------------------------------------------- M = 1, fused quantize
//
// Prologues (PRO): the activation row that every workgroup stages into LDS
// arrives as
//   PRO_BF16     bf16 x, quantized here;
//   PRO_INT8     int8 xq (k order) + fp32 group scales xs (the layout of
//                viper_hip_quantize_act), only rearranged;
//   PRO_RMSNORM  bf16 x and gamma: v = bf16((x * rsqrt(sum x^2 / K + eps)) *
//                gamma), then quantized (the reference's rmsnorm_quantize,
//                kernels/ops/rmsnorm_quantize.cu:37-104, folded into the GEMV:
//                every workgroup recomputes the row's sum of squares);
//   PRO_SWIGLU   bf16 gate and up: v = bf16(silu(g) * u) (silu_mul), then
//                quantized (swiglu_quantize.cu:35-78 folded in).
// The two folded prologues need the whole row in one load round
// (K / 8 <= M1_XS * NTT octets).
//
// Up to three matrices with the same K may share a launch (q/k/v, gate/up):
// workgroups [0, e0) work on matrix 0, [e0, e1) on matrix 1, the rest on
// matrix 2.  The residual and the partials belong to matrix 0.
//
// A team of TS lanes streams one output row: in each load instruction lane l
// reads 16-byte chunk c = base + l of the row, so every instruction reads
// whole contiguous row segments.  A chunk is half a quantization group; the
// two halves meet by a DPP lane swap of the int32 partial, and the even lane
// of the pair applies the group's scales.
//
// LDS: xq [K] int8 (octets in the format's dot order), per chunk
// {-OFF * sum(q) over the chunk (int32), xs (fp32)}, 16 floats of cross-wave
// sums and, for exact tilings, the workgroup's block of weight scales.

constexpr int M1_XS = 4;    // activation octets per thread loaded before the weights
constexpr int M1_XS_MR = 8; // the same for MR > 1 rows (all of them: no later rounds)
constexpr int M1_DELAY = 6; // weight-issue delay, s_sleep units (one activation row)
constexpr int M1_DELAY_MR = 8; // the same for MR > 1 bf16 rows (MR rows of activation ahead of the weights)
constexpr int M1_DELAY_ROUND = 4; // the same for MR > 1 int8 rows, per staging round of the rows
// the same for one int8 row on an exact tiling, by workgroup size: 256 threads
// (K = N = 2560: 2.60 -> 2.50 us against 6) and 640 threads (K = 10240,
// N = 2560: 4.41 -> 4.18 us; Q4's two-octet staging 4.09 us at 4); 320
// threads (K = 2560, N = 10240) is best at 6 either way
constexpr int M1_DELAY_INT8_256 = 2;
constexpr int M1_DELAY_INT8_640 = 8;
constexpr int M1_DELAY_PAIR8_640 = 4;
constexpr int M1_DELAY_PAIR = 16; // the same for the gate/up pair (twice the weight stream per workgroup)
constexpr int M1_DELAY_RMS = 3;   // the same for the rmsnorm prologue (q/k/v: 3.31 -> 3.23 us against 6)
constexpr int M1_DELAY_WIDE = 10; // the same for a wide launch with the bf16 prologue (W8, K = 2560: 5.80 -> 5.71 us)

// Row length of an exact tiling (TS lanes x CPL chunks of CK weights): an
// exact launch's K is this constant, so its load rounds and offsets are
// compile-time (the run-time round guards of the general path cost 0.1 us of
// the north-star launch, placed before the weight loads).
template <int F>
__host__ __device__ constexpr int m1_exact_k(int ts, int cpl) { return Fmt<F>::CK * ts * cpl; }
__host__ __device__ constexpr int m1_max(int a, int b) { return a > b ? a : b; }

// Kernel modes: plain, with the int32 group dots (test entry point), or the
// gate/up pair with the swiglu epilogue (M1_SWIGLU): the first NTT/2 threads
// stream P = ROWS/2 rows of the gate matrix (w0), the others the same P rows
// of the up matrix (w1), and the workgroup writes h = bf16(silu(g) * u) from
// the two bf16-rounded outputs.  P must be a whole number of waves' teams so
// every wave reads one matrix.
// M1_TL: M1_PLAIN plus a per-wave timeline (measurement entry point
// viper_hip_qlinear_timeline): the `part` argument then points at
// [workgroup][wave][M1_TL_STAMPS] uint64 s_memrealtime readings (100 MHz).
enum { M1_PLAIN = 0, M1_PART = 1, M1_SWIGLU = 2, M1_TL = 3 };

// A wide launch: an exact tiling whose activation rows fill at most half of
// its threads' octet slots (W8 at K = 2560 on 640 threads, the gate/up pair),
// so half of its waves stage nothing.
template <int F>
__host__ __device__ constexpr bool m1_wide(bool exact, int ts, int ntt, int cpl, int mr) {
    return exact && mr * (m1_exact_k<F>(ts, cpl) / 8) <= ntt / 2;
}

// Launches whose staging threads take two octets each (Q4, exact tilings):
// one int8 row on 320 or 640 threads, one bf16 row on 256, and 2-4 rows of
// either on 640 (on 320 threads 2 rows were equal either way).
template <int F>
__host__ __device__ constexpr bool m1_pairs(bool exact, int ntt, int mr, int pro) {
    return F == 4 && exact &&
           (pro == PRO_INT8   ? (mr == 1 ? (ntt == 320 || ntt == 640) : ntt == 640)
            : pro == PRO_BF16 ? (mr == 1 ? ntt == 256 : ntt == 640)
                              : false);
}

// Weight-issue delay of a launch kind (s_sleep units).  Int8 rows (MR > 1)
// wait in proportion to their staging rounds (one 8-byte load per thread and
// round, or 16 bytes for Q4's two-octet staging; all issued before the
// weights), at least 2: K = 10240, N = 2560 with 2 / 4 rows (4 / 8 rounds)
// 5.9 / 8.2 us at 8 units against 5.1 / 7.6 us at 16 / 32; K = 2560, N = 10240
// with 2 / 4 rows on 320 threads (2 / 4 rounds) best at 8 / 16; Q4's pairs (1,
// 2 or 4 rounds) best at 8, 8 and 16.  The bf16 rows, which quantize what
// they load, are best at 8 in all four cases one octet per thread; Q4's
// two-octet bf16 rows follow the int8 rule (1, 2 or 4 rounds: 8, 8, 16).
template <int F>
__host__ __device__ constexpr int m1_delay(bool exact, int ts, int ntt, int cpl, int mode, int mr, int pro) {
    return mode == M1_SWIGLU                                   ? M1_DELAY_PAIR
           : mr > 1 && pro == PRO_INT8
               ? M1_DELAY_ROUND * (exact ? m1_max(2, (mr * (m1_exact_k<F>(ts, cpl) /
                                                             (m1_pairs<F>(exact, ntt, mr, pro) ? 16 : 8)) + ntt - 1) / ntt)
                                         : M1_XS_MR)
           : mr > 1 && mode == M1_PLAIN && m1_pairs<F>(exact, ntt, mr, pro)
               ? M1_DELAY_ROUND * m1_max(2, (mr * (m1_exact_k<F>(ts, cpl) / 16) + ntt - 1) / ntt)
           : mr > 1                                            ? M1_DELAY_MR
           : pro == PRO_INT8 && exact && ntt == 256            ? M1_DELAY_INT8_256
           : pro == PRO_INT8 && exact && ntt == 640            ? (F == 4 ? M1_DELAY_PAIR8_640 : M1_DELAY_INT8_640)
           : pro == PRO_RMSNORM                                ? M1_DELAY_RMS
           : pro == PRO_BF16 && m1_wide<F>(exact, ts, ntt, cpl, mr) ? M1_DELAY_WIDE
                                                               : M1_DELAY;
}
constexpr int M1_TL_STAMPS = 8;
__host__ __device__ constexpr bool m1_pair_ok(int ts, int ntt) {
    return (ntt / ts) % 2 == 0 && ((ntt / ts) / 2) % (64 / ts) == 0;
}

// Weight-scale block of an exact-tiled workgroup: rows x groups 16-bit scales.
__host__ __device__ constexpr size_t m1_scale_block(int rows, int ngr) {
    return ((size_t)rows * ngr * 2 + 15) / 16 * 16;
}

// LDS bytes of a launch: xq [K], per-chunk records, cross-wave sums, the
// swiglu epilogue's gate values (up to 32), the scale block of `rows` rows
// (exact tilings).
template <int F>
__host__ __device__ constexpr size_t m1_lds_bytes(int K, int rows, int mr = 1) {
    return (size_t)mr * K + (size_t)mr * (K / Fmt<F>::CK) * 8 + 128 + m1_scale_block(rows, K / Fmt<F>::G);
}

// Shapes instantiated for MR > 1 activation rows (the workgroups that stage
// MR rows hold 320 or 640 threads).
__host__ __device__ constexpr bool m1_mr_shape_ok(int ts, int ntt, int cpl) {
    return (ntt == 320 && ts == 16 && cpl == 5) || (ntt == 320 && ts == 8 && cpl == 10) ||
           (ntt == 640 && cpl == 5 && ts >= 16) || (ntt == 640 && cpl == 10 && ts >= 16);
}


// Dot phase for MR > 1 activation rows: per chunk the weights are decoded
// once (Q4: the sign flip for the high-nibble dot; Q5/Q6/W8: the int8 offset
// codes) and dotted with each row's activation from LDS; per row one fp32
// accumulator, one team reduction and one bf16 store (+ residual).
template <int F, int TS, int CPL, int SENC, bool PART, bool EXACT, int MR, typename LoadSeg>
__device__ __forceinline__ void m1_dots_rows(u32x4 (&wv)[CPL], uint32_t (&h0)[CPL], uint32_t (&h1)[CPL],
                                             uint32_t (&sv)[CPL], LoadSeg& load_seg, const int8_t* lxq,
                                             const u32x2* lcs, const uint16_t* lsc, int32_t* part,
                                             const uint16_t* res, uint16_t* y, int M, int N, int K, int CPR,
                                             int NGR, int segw, int nseg, int rr, int l, int row, bool row_ok,
                                             bool lead) {
    using FT = Fmt<F>;
    float acc[MR];
#pragma unroll
    for (int m = 0; m < MR; ++m) acc[m] = 0.0f;
    for (int seg = 0; seg < nseg; ++seg) {
        if (seg) load_seg(seg);
        float WS[CPL];  // weight scale of the chunk's group (0 on the odd lane of a pair)
#pragma unroll
        for (int j = 0; j < CPL; ++j) {
            const int c = seg * segw + j * TS + l;
            uint32_t sraw = sv[j];
            if constexpr (EXACT) sraw = lsc[rr * NGR + (c >> 1)];
            const float wsf = SENC ? bf16f(sraw) : f16f(sraw);
            WS[j] = (EXACT && !lead) ? 0.0f : wsf;
        }
#pragma unroll
        for (int j = 0; j < CPL; ++j) {
            const int c = seg * segw + j * TS + l;
            const bool ok = EXACT || c < CPR;
            const int cc = EXACT ? c : min(c, CPR - 1);
            const u32x4 p = wv[j];
            u32x4 px = p;
            uint32_t wd[8];
            if constexpr (F == 4) px = u32x4{p.x ^ 0x88888888u, p.y ^ 0x88888888u, p.z ^ 0x88888888u, p.w ^ 0x88888888u};
            else decode<F>(p, h0[j], h1[j], wd);
            // every row's operands first (rows >= M read staged but unused LDS:
            // no branch, so the reads overlap), then the dots
            u32x2 cs[MR];
            u32x4 a0[MR], a1[MR];
#pragma unroll
            for (int m = 0; m < MR; ++m) {
                cs[m] = lcs[m * CPR + cc];
                const u32x4* a = (const u32x4*)(lxq + (size_t)m * K + (size_t)cc * FT::CK);
                a0[m] = a[0];
                a1[m] = FT::OFF ? a[1] : a[0];
            }
#pragma unroll
            for (int m = 0; m < MR; ++m) {
                int dot;
                if constexpr (F == 4) {
                    dot = chunk_dot_q4x(p, px, a0[m], a1[m], (int)cs[m].x);
                } else {
                    dot = (int)cs[m].x;
                    dot = sdot4(wd[0], a0[m].x, dot);
                    dot = sdot4(wd[1], a0[m].y, dot);
                    dot = sdot4(wd[2], a0[m].z, dot);
                    dot = sdot4(wd[3], a0[m].w, dot);
                    if constexpr (F != 8) {
                        dot = sdot4(wd[4], a1[m].x, dot);
                        dot = sdot4(wd[5], a1[m].y, dot);
                        dot = sdot4(wd[6], a1[m].z, dot);
                        dot = sdot4(wd[7], a1[m].w, dot);
                    }
                }
                dot += dpp_i<DPP_SWAP1>(dot);
                if constexpr (PART)
                    if (m < M && ok && lead && row_ok) part[((size_t)m * N + row) * NGR + (cc >> 1)] = dot;
                acc[m] = __builtin_fmaf(WS[j] * __uint_as_float(cs[m].y), (float)dot, acc[m]);
            }
        }
    }
#pragma unroll
    for (int m = 0; m < MR; ++m) {
        float v = team_sum<TS>(acc[m]);
        if (m < M && l == 0 && row_ok) {
            const size_t o = (size_t)m * N + row;
            if (__builtin_expect(res != nullptr, 0)) v += bf16f(res[o]);
            y[o] = f2bf(v);
        }
    }
}

// n0's high bits: flags of the launch (the row count of matrix 0 below them,
// at most VIPER_QLINEAR_MAX_N)
constexpr int M1_N_EXTRA = VIPER_QLINEAR_MAX_N + 1;  // optional outputs present (xout; the pair's gate / up)
constexpr int M1_N_MASK = VIPER_QLINEAR_MAX_N;

// qgemv_m1_kernel's parameters in order, as they lie in its kernarg segment
// (each at its natural alignment): the offsets of those past the preloaded
// ones, read with vector loads where a scalar load's cache miss would sit on
// the critical path.
struct M1KernArgs {
    const void* x;
    const uint8_t* w0;
    const uint16_t* s0;
    uint16_t* y0;
    int K, n0, e0, e1;
    const uint16_t* res;
    const void* xa;
    float eps;
    uint16_t* xout;
    int32_t* part;
    const uint8_t* w1;
    const uint16_t* s1;
    uint16_t* y1;
    int n1;
    const uint8_t* w2;
    const uint16_t* s2;
    uint16_t* y2;
    int n2;
};
static_assert(offsetof(M1KernArgs, eps) == 64 && offsetof(M1KernArgs, n2) == 144, "kernarg layout");
// (the segment ends with n2: no tail padding is read)
__device__ __forceinline__ __amdgpu_buffer_rsrc_t m1_kernargs() {
    return buf((const void*)__builtin_amdgcn_kernarg_segment_ptr(), (uint32_t)(offsetof(M1KernArgs, n2) + sizeof(int)));
}
// xout, read only in the branch that stores it: the offset goes through an
// opaque zero, so the compiler cannot hoist the scalar load out of the branch
// (hoisted, its cache miss held every workgroup at its next wait on the scalar
// and LDS counter)
__device__ __forceinline__ uint16_t* m1_xout() {
    int z;
    asm volatile("s_mov_b32 %0, 0" : "=s"(z));
    const auto* ka = (const __attribute__((address_space(4))) uint8_t*)__builtin_amdgcn_kernarg_segment_ptr();
    return *(uint16_t* const __attribute__((address_space(4)))*)(ka + offsetof(M1KernArgs, xout) + z);
}

// EXACT: every lane's chunks lie inside its row (the row has exactly TS * CPL
// chunks) and a row's scales fill whole 16-byte words (groups % 8 == 0), so no
// chunk needs masking and the workgroup's scale block is loaded with one
// 16-byte load per thread into LDS instead of one 2-byte load per chunk (those
// small loads slow the weight issue several-fold).  K is then the constant
// m1_exact_k and its argument carries the number of workgroups of the launch
// (the XCD-aware block order needs it, and every preloaded dword is taken).
// CPL: chunk slots per lane per row segment.
// DELAY: s_sleep units (64 clocks) between issuing the activation loads and
// the weight loads.  The activation is a few KB read by every workgroup; a
// short head start lets its requests through the memory pipeline before the
// weight stream saturates it, which moves every workgroup's barrier earlier.
// xa: PRO_INT8 the group scales, PRO_RMSNORM gamma, PRO_SWIGLU up.
// xout (PRO_RMSNORM): the bf16 normalized row, written by the first
// workgroup when n0 carries M1_N_EXTRA.
// M1_SWIGLU takes the up matrix in the res (weights) and e0 / e1 (scales, low
// and high half) slots and writes the product to y0; with M1_N_EXTRA, y1 and
// y2 (each may be null) receive gate and up.
// MR > 1 (PRO_BF16 / PRO_INT8, one matrix): M = e1 <= MR activation rows
// (x [M][K], y and the residual [M][N]); every workgroup stages all M rows,
// each lane decodes its weight chunk once and dots it with every row.  Small
// verify batches then need no separate quantize launch.
template <int F, int TS, int NTT, int CPL, int SENC, int MODE, bool EXACT, int PRO, int MR, int DELAY, int KC = 0>
__global__ void __launch_bounds__(NTT)
qgemv_m1_kernel(const void* x, const uint8_t* w0, const uint16_t* s0, uint16_t* y0, int K, int n0, int e0,
                int e1, const uint16_t* res, const void* xa, float eps, uint16_t* __restrict__ xout,
                int32_t* __restrict__ part, const uint8_t* w1, const uint16_t* s1, uint16_t* y1, int n1,
                const uint8_t* w2, const uint16_t* s2, uint16_t* y2, int n2) {
    using FT = Fmt<F>;
    constexpr bool PART = MODE == M1_PART;
    constexpr bool SWI = MODE == M1_SWIGLU;
    constexpr bool TLM = MODE == M1_TL;
    // timeline stamps (M1_TL only): wave start, activation and scale loads
    // issued, weight loads issued, activation quantized, barrier passed,
    // first chunk dotted, last chunk dotted, output stored
    uint64_t tstamp[M1_TL_STAMPS];
    auto stamp = [&](int i) {
        if constexpr (TLM) tstamp[i] = __builtin_amdgcn_s_memrealtime();
    };
    stamp(0);
    constexpr bool PRE = PRO == PRO_INT8;
    constexpr bool TWO = PRO == PRO_RMSNORM || PRO == PRO_SWIGLU;  // two bf16 inputs
    // exact tilings: K is the tiling's row length and the argument slot
    // carries the grid size instead (for the XCD-aware block order); the
    // load rounds of one row are then exact
    // KC (masked exact tilings): the row has KC < TS * CPL chunks; K is still
    // the constant, the scale block still staged, and the slots past the row
    // read nothing (out of the buffer's range) and add nothing.
    constexpr int KX = EXACT ? (KC ? Fmt<F>::CK * KC : m1_exact_k<F>(TS, CPL)) : 0;
    constexpr bool MASK = EXACT && KC != 0 && KC != TS * CPL;
    static_assert(!MASK || (MR == 1 && KC < TS * CPL), "masked tilings: one row, fewer chunks than slots");
    constexpr bool FULL = EXACT && !MASK;  // every slot holds a chunk of the row
    const int grid = K;
    if constexpr (EXACT) K = KX;
    // SPARE: the first wave stages no activation and issues its weights at
    // once, without the delay; the other ANT threads stage the row (in one
    // more round where needed).  The weight stream then starts a wave
    // earlier.  Taken where it was measured to pay: exact tilings of 256 or
    // 320 threads and wide ones with the bf16 prologue (north star 3.91 ->
    // 3.75 us, K = N = 2560 2.52 -> 2.43 us, W8 at K = 2560 6.00 -> 5.80 us)
    // and the gate/up pair, whose other waves also wait longer
    // (M1_DELAY_PAIR: 6.33 -> 5.80 us at K = 2560, N = 10240).  The staged
    // LDS row is the same either way; for the rmsnorm prologue the pair keeps
    // one octet per staging thread (K / 8 <= ANT), so each wave's sum of
    // squares covers the same octets as without the spare wave and the row's
    // sum (wave sums in wave order, the spare wave's 0 first) is unchanged
    // bit for bit.
    // Q4 from bf16 rows (PAIRBF): each staging thread loads and quantizes two
    // octets (16 values; the group's amax over its 4 lanes, the same maximum
    // as over 8 lanes of one octet).  One row on 256 threads: 160 threads
    // stage a K = 2560 row and the fourth wave issues its weights at once, no
    // spare wave; K = N = 2560 2.51 -> 2.45 us (one row on 320 and 640
    // threads: equal either way, not used).  2-4 rows on 640 threads: half the
    // rounds; K = 10240, N = 2560 with 2 / 3 / 4 rows 5.8 / 8.2 / 9.7 -> 5.2 /
    // 7.5 / 8.4 us, K = 2560, N = 10240 with 3 / 4 rows 5.85 / 6.1 -> 5.65 /
    // 5.95 us (2 rows on 320 threads: equal, not used).  The same LDS rows bit
    // for bit.
    constexpr bool PAIRBF = PRO == PRO_BF16 && MODE == M1_PLAIN && m1_pairs<F>(EXACT, NTT, MR, PRO);
    constexpr bool SPARE = !PAIRBF && EXACT && MR == 1 &&
                           ((PRO == PRO_BF16 && MODE != M1_SWIGLU &&
                             (NTT == 256 || NTT == 320 || m1_wide<F>(EXACT, TS, NTT, CPL, MR))) ||
                            (MODE == M1_SWIGLU && (PRO == PRO_BF16 || (PRO == PRO_RMSNORM && KX / 8 <= NTT - 64))));
    constexpr int A0 = SPARE ? 64 : 0;  // first staging thread
    constexpr int ANT = NTT - A0;       // staging threads
    // Q4 from int8 rows (PAIR8; one row on 320 or 640 threads, 2-4 rows on
    // 640, m1_pairs): each staging thread
    // takes two octets with one 16-byte load and stores them with one 16-byte
    // LDS write, a chunk's two lanes summing its correction; with one row the
    // waves past its K/16 pairs stage nothing and issue their weights at once.
    // Bit for bit the same LDS rows as one octet per thread.  One row: K =
    // 2560, N = 10240 4.06 -> 3.84 us, K = 10240, N = 2560 4.19 -> 4.09 us; 2 /
    // 3 / 4 rows at K = 10240: 5.17 / 7.3 / 7.6 -> 4.85 / 6.55 / 6.85 us; on 256
    // threads (K = N = 2560, one row) one octet per thread stays faster (2.54
    // against 2.64 us).
    constexpr bool PAIR8 = PRE && !SPARE && m1_pairs<F>(EXACT, NTT, MR, PRO);
    constexpr int XS = (PAIR8 || PAIRBF) ? (MR * (KX / 16) + ANT - 1) / ANT
                       : EXACT ? (MR * (KX / 8) + ANT - 1) / ANT : MR > 1 ? M1_XS_MR : M1_XS;
    constexpr int ROWS = NTT / TS;
    const int M = MR == 1 ? 1 : e1;  // activation rows
    constexpr int HB = FT::HIW * 4;  // high-plane bytes per chunk: Q5 4, Q6 8
    constexpr int OPC = FT::CK / 8;  // octets per chunk (4, or 2 for W8)
    extern __shared__ __align__(16) uint8_t smem[];
    const int CPR = K / FT::CK;      // chunks per row
    const int NGR = K / FT::G;       // groups per row
    const size_t lact = (size_t)MR * K + (size_t)MR * CPR * 8;  // activation rows and their records
    int8_t* lxq = (int8_t*)smem;                                  // [MR][K]
    u32x2* lcs = (u32x2*)(smem + (size_t)MR * K);                // [MR][CPR]
    float* lred = (float*)(smem + lact);
    uint16_t* lepi = (uint16_t*)(smem + lact + 64);
    uint16_t* lsc = (uint16_t*)(smem + lact + 128);

    const int tid = (int)threadIdx.x;
    const int l = tid % TS;
    const int rr = tid / TS;  // row within the workgroup
    // matrix of this workgroup (matrix 0's arguments lead the argument list,
    // so its workgroups need nothing beyond the preloaded arguments).  The
    // rare paths of the kernel (other matrices, the residual, activation
    // rounds past the first XS) are marked unlikely: the compiler then lays
    // the common path out straight and schedules it on its own, which takes
    // 0.05 us off the north-star launch; MR > 1 launches are single-matrix and
    // stage their rows in XS rounds, so those paths are not compiled there
    // (0.5 us of an M = 2 launch).
    int bid = EXACT ? xcd_block((int)blockIdx.x, grid) : (int)blockIdx.x;
    const uint8_t* w = w0;
    const uint16_t* ws = s0;
    uint16_t* y = y0;
    int N = n0 & M1_N_MASK;
    const bool extra_out = (n0 & M1_N_EXTRA) != 0;  // optional outputs (xout; the pair's gate / up)
    if (MR == 1 && !SWI && __builtin_expect(bid >= e0, 0)) {
        res = nullptr;
        if (bid >= e1) {
            bid -= e1;
            w = w2;
            ws = s2;
            y = y2;
            N = n2;
        } else {
            bid -= e0;
            w = w1;
            ws = s1;
            y = y1;
            N = n1;
        }
    }
    // swiglu pair: waves of the second half read the up matrix; rt is the
    // team's row within its matrix's block of P rows
    constexpr int P = SWI ? ROWS / 2 : ROWS;
    int rt = rr;
    bool up = false;
    if constexpr (SWI) {
        // the up matrix comes in preloaded slots the pair does not use
        // otherwise (weights in the residual's, scales in e0 / e1): read
        // from the kernarg segment past them, the pointers would hold every
        // up wave's weight requests back by a scalar-cache miss
        up = __builtin_amdgcn_readfirstlane(tid >> 6) * (64 / TS) >= P;  // wave-uniform
        if (up) {
            w = (const uint8_t*)res;
            ws = (const uint16_t*)(((uint64_t)(uint32_t)e1 << 32) | (uint32_t)e0);
            rt = rr - P;
        }
        res = nullptr;
    }
    const int row0 = bid * P;
    const int row = row0 + rt;
    const int nrows = min(P, N - row0);
    const bool row_ok = rt < nrows;
    const int ltid = up ? tid - P * TS : tid;  // thread index within the matrix's half

    // 1. activation octets, then every weight byte and group scale of the
    //    first row segment, all in flight at once
    const int noct = M * (K / 8);  // octets of all rows (rows follow each other)
    constexpr int OPG = FT::G / 8;   // octets per group
    const auto xr = buf(x, (uint32_t)(M * K) * (PRE ? 1 : 2));
    const auto xsr = buf(xa, PRE ? (uint32_t)(M * (K / FT::G)) * 4 : TWO ? (uint32_t)K * 2 : 0u);
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
    // rounds past the row are not issued (the bound is workgroup-uniform)
    // The first input's octets go out first: the second input (int8 group
    // scales, gamma, up) sits past the 14 preloaded argument dwords, and the
    // wait for its argument load then follows these requests instead of
    // preceding every load of the wave.
    const int at = tid - A0;  // staging thread index (negative on the spare wave)
    const bool stager = (PAIR8 || PAIRBF) && MR == 1 ? (__builtin_amdgcn_readfirstlane(tid) & ~63) < KX / 16
                                         : (!SPARE || __builtin_amdgcn_readfirstlane(tid) >= A0);  // wave-uniform
    // int8 rows (MR > 1): every round is issued, the rounds past the rows
    // reading zeros through the buffers' ranges (M * K bytes, M * K / G
    // scales).  A branch per round (the row count is a run-time value) made
    // the compiler wait for each load at the branch join and spill it to
    // scratch: 20 us instead of 8.2 us at K = 10240 with 4 rows.
    constexpr bool ALL_ROUNDS = PRE && MR > 1;
    u32x4 xv[XS], av[XS];
#pragma unroll
    for (int i = 0; i < XS; ++i) {
        xv[i] = u32x4{0u, 0u, 0u, 0u};
        av[i] = xv[i];
        if (ALL_ROUNDS || ((i == 0 || ANT * i < (PAIRBF ? noct / 2 : noct)) && stager)) {
            if constexpr (PAIRBF) {  // octets 2p, 2p + 1 (bf16)
                xv[i] = bload16(xr, (at + ANT * i) * 32);
                av[i] = bload16(xr, (at + ANT * i) * 32 + 16);
            } else if constexpr (PAIR8) {
                xv[i] = bload16(xr, (at + ANT * i) * 16);  // octets 2p, 2p + 1
            } else if constexpr (PRE) {
                const u32x2 q = bload8(xr, (at + ANT * i) * 8);
                xv[i] = u32x4{q.x, q.y, 0u, 0u};
            } else {
                xv[i] = bload16(xr, (at + ANT * i) * 16);
            }
        }
    }
    issue_fence();
    if constexpr (PRE || TWO) {
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int i = 0; i < XS; ++i) {
            if (ALL_ROUNDS || ((i == 0 || ANT * i < noct) && stager)) {
                const int o = at + ANT * i;
                if constexpr (PAIR8) av[i].x = bload4(xsr, ((2 * o) % OPC == 0) ? ((2 * o) / OPG) * 4 : OOB);
                else if constexpr (PRE) xv[i].z = bload4(xsr, (o % OPC == 0) ? (o / OPG) * 4 : OOB);
                else av[i] = bload16(xsr, o * 16);
            }
        }
        issue_fence();
    }
    // eps sits past the preloaded arguments: a scalar load there misses the
    // scalar cache, and its wait, after the row sum's barrier, held the
    // rmsnorm launches 0.5 us.  A vector load issued here returns with the
    // row.
    float epsv = eps;
    if constexpr (PRO == PRO_RMSNORM) {
        epsv = __uint_as_float(bload4(m1_kernargs(), (int)offsetof(M1KernArgs, eps)));
        issue_fence();
    }
    const auto sr = buf(ws + (size_t)row0 * NGR, (uint32_t)(nrows * NGR) * 2);
    u32x4 sblk = {0u, 0u, 0u, 0u};
    if constexpr (EXACT) sblk = bload16(sr, ltid * 16);
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
            const bool in = FULL || c < CPR;
            wv[j] = bload16<AUX_NT>(wr, in ? rt * (int)rbytes + c * 16 : OOB);
            // odd lanes and chunks past the row read scale 0, which zeroes
            // their term without any select
            sv[j] = 0u;
            if constexpr (!EXACT) sv[j] = bload2(sr, (in && lead) ? (rt * NGR + (c >> 1)) * 2 : OOB);
            h0[j] = 0u;
            h1[j] = 0u;
            if constexpr (FT::HIW == 1) {
                h0[j] = bload4<AUX_NT>(hr, in ? (rt * CPR + c) * HB : OOB);
            } else if constexpr (FT::HIW == 2) {
                const u32x2 hh = bload8<AUX_NT>(hr, in ? (rt * CPR + c) * HB : OOB);
                h0[j] = hh.x;
                h1[j] = hh.y;
            }
        }
    };
    stamp(1);
    if constexpr (DELAY > 0)
        if (stager) __builtin_amdgcn_s_sleep(DELAY);
    load_seg(0);
    stamp(2);

    // 2. quantize the activation into LDS (trip counts are workgroup-uniform,
    //    so every DPP group reduction sees whole groups).  Q4 stores each
    //    octet as (ql nibbles, qh nibbles); Q5/Q6 as [k even | k odd] int8;
    //    W8 in k order.
    const int xiters = (noct + ANT - 1) / ANT;
    // PRO_RMSNORM: the row's sum of squares (per-thread fma chain over its
    // octets in order, DPP within the wave, wave sums in wave order)
    float inv = 0.0f;
    if constexpr (PRO == PRO_RMSNORM) {
        float ss = 0.0f;
#pragma unroll
        for (int i = 0; i < XS; ++i) {
            if (stager && at + ANT * i < noct) {
                const u32x4 v = xv[i];
                const uint32_t wd[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
                for (int j = 0; j < 8; ++j) {
                    const float f = bf16f((wd[j >> 1] >> (16 * (j & 1))) & 0xffffu);
                    ss = __builtin_fmaf(f, f, ss);
                }
            }
        }
        ss = team_sum<64>(ss);
        if ((tid & 63) == 0) lred[tid >> 6] = ss;
        lds_barrier();
        float t = 0.0f;
#pragma unroll
        for (int i = 0; i < NTT / 64; ++i) t += lred[i];
        inv = __builtin_amdgcn_rsqf(t / (float)K + epsv);
    }
    // PRO_RMSNORM / PRO_SWIGLU: the bf16 row element-wise from two inputs
    auto produce = [&](const u32x4& v, const u32x4& a) -> u32x4 {
        const uint32_t vw[4] = {v.x, v.y, v.z, v.w}, aw[4] = {a.x, a.y, a.z, a.w};
        uint32_t o[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            float f0 = bf16f(vw[j] & 0xffffu), f1 = bf16f(vw[j] >> 16);
            const float g0 = bf16f(aw[j] & 0xffffu), g1 = bf16f(aw[j] >> 16);
            if constexpr (PRO == PRO_RMSNORM) {
                f0 = (f0 * inv) * g0;
                f1 = (f1 * inv) * g1;
            } else {
                f0 = silu_mul(f0, g0);
                f1 = silu_mul(f1, g1);
            }
            o[j] = f2bf2(f0, f1);
        }
        return u32x4{o[0], o[1], o[2], o[3]};
    };
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
    const int wave0 = (tid & ~63) - A0;  // waves with no octet skip the quantize
#pragma unroll
    for (int i = 0; i < XS; ++i) {
        if constexpr (PAIRBF) {
            const int p = at + ANT * i;
            const int npair = MR == 1 ? KX / 16 : M * (K / 16);  // pairs of all rows
            if (wave0 + ANT * i < npair && stager) {
                uint32_t d0, d1, d2, d3;
                float sc;
                quantize_octet_pair<FT::G>(xv[i], av[i], d0, d1, d2, d3, sc);
                const uint32_t ql0 = nibbles8(d0, d1), qh0 = nibbles8(d0 >> 4, d1 >> 4);
                const uint32_t ql1 = nibbles8(d2, d3), qh1 = nibbles8(d2 >> 4, d3 >> 4);
                int cs = (int)udot8(ql0, 0x11111111u, 0u) + (int)udot8(ql1, 0x11111111u, 0u);
                cs += dpp_i<DPP_SWAP1>(cs);
                if (p < npair) {
                    *(u32x4*)(lxq + (size_t)p * 16) = u32x4{ql0, qh0, ql1, qh1};
                    if ((p & 1) == 0) lcs[p >> 1] = u32x2{(uint32_t)(-8 * cs), __float_as_uint(sc)};
                }
            }
        } else if constexpr (PAIR8) {
            // pair p = octets 2p, 2p + 1 as (ql, qh) nibble words; the chunk
            // (4 octets) is lanes 2c, 2c + 1, its scale loaded by the even one
            const int p = at + ANT * i;
            const int npair = MR == 1 ? KX / 16 : M * (K / 16);  // pairs of all rows
            if (wave0 + ANT * i < npair && stager) {
                const u32x4 v = xv[i];
                const uint32_t ql0 = nibbles8(v.x, v.y), qh0 = nibbles8(v.x >> 4, v.y >> 4);
                const uint32_t ql1 = nibbles8(v.z, v.w), qh1 = nibbles8(v.z >> 4, v.w >> 4);
                int cs = (int)udot8(ql0, 0x11111111u, 0u) + (int)udot8(ql1, 0x11111111u, 0u);
                cs += dpp_i<DPP_SWAP1>(cs);
                if (p < npair) {
                    *(u32x4*)(lxq + (size_t)p * 16) = u32x4{ql0, qh0, ql1, qh1};
                    if ((p & 1) == 0) lcs[p >> 1] = u32x2{(uint32_t)(-8 * cs), av[i].x};
                }
            }
        } else if (i < xiters && wave0 + ANT * i < noct && stager) {
            if constexpr (TWO) {
                const int o = at + ANT * i;
                const u32x4 v = produce(xv[i], av[i]);
                if (PRO == PRO_RMSNORM && __builtin_expect(extra_out, 0) && blockIdx.x == 0) {
                    // (the flag also marks the pair's gate / up outputs: xout may be null)
                    uint16_t* xo = m1_xout();
                    if (xo != nullptr && o < noct) *(u32x4*)(xo + (size_t)o * 8) = v;
                }
                quant_store(o, v);
            } else {
                quant_store(at + ANT * i, xv[i]);
            }
        }
    }
    if constexpr (!TWO && MR == 1 && !PAIR8 && !PAIRBF) {
        if (__builtin_expect(xiters > XS, 0))
            for (int i = XS; i < xiters; ++i)
                if (stager && wave0 + ANT * i < noct) quant_store(at + ANT * i, load_x(at + ANT * i));
    }

    // the scale block into LDS after the activation: its loads come from HBM
    // and arrive after the activation's, and the quantize (and the rmsnorm
    // prologue's row sum) need not wait for them
    // (the up matrix's block follows the gate block: lsc[rr * NGR + g] for every team)
    if constexpr (EXACT)
        if (ltid * 16 < nrows * NGR * 2) *(u32x4*)((uint8_t*)lsc + (up ? P * NGR * 2 : 0) + ltid * 16) = sblk;
    stamp(3);
    lds_barrier();
    stamp(4);

    // 3. chunk dots, group sums, fp32 combine (MR > 1: the loop after this one).  Every LDS operand of the
    //    segment is read before the first dot: the reads then overlap the
    //    wait for the weights instead of sitting between the dots (0.3 us of
    //    the north-star dispatch).  Each chunk waits only for its own weights.
    if constexpr (MR > 1) {
        m1_dots_rows<F, TS, CPL, SENC, PART, EXACT, MR>(wv, h0, h1, sv, load_seg, lxq, lcs, lsc, part, res, y, M, N,
                                                         K, CPR, NGR, segw, nseg, rr, l, row, row_ok, lead);
        return;
    }
    float acc = 0.0f;
    for (int seg = 0; seg < nseg; ++seg) {
        if (seg) load_seg(seg);
        u32x4 A0[CPL], A1[CPL];
        u32x2 CS[CPL];
        float SC[CPL];  // ws * xs of the chunk's group (0 on the odd lane of a pair)
#pragma unroll
        for (int j = 0; j < CPL; ++j) {
            const int c = seg * segw + j * TS + l;
            const int cc = FULL ? c : min(c, CPR - 1);
            CS[j] = lcs[cc];
            const u32x4* a = (const u32x4*)(lxq + (size_t)cc * FT::CK);
            A0[j] = a[0];
            A1[j] = FT::OFF ? a[1] : a[0];
            if constexpr (EXACT) {
                // read on every lane (in bounds), select after: no branch, no
                // wait between the LDS reads, product formed before the weights
                // (a masked slot's scale is 0: its dot of zero weights with the
                // last chunk's activation adds nothing)
                const uint32_t sraw = lsc[rr * NGR + (cc >> 1)];
                const float wsf = SENC ? bf16f(sraw) : f16f(sraw);
                SC[j] = ((lead && (FULL || c < CPR)) ? wsf : 0.0f) * __uint_as_float(CS[j].y);
            }
        }
#pragma unroll
        for (int j = 0; j < CPL; ++j) {
            const int c = seg * segw + j * TS + l;
            const bool ok = FULL || c < CPR;
            const int cc = FULL ? c : min(c, CPR - 1);
            int dot;
            if constexpr (F == 4) dot = chunk_dot_q4(wv[j], A0[j], A1[j], (int)CS[j].x);
            else dot = chunk_dot<F>(wv[j], h0[j], h1[j], A0[j], A1[j], (int)CS[j].x);
            dot += dpp_i<DPP_SWAP1>(dot);
            const int g = cc >> 1;
            if constexpr (PART)
                if (ok && lead && row_ok) part[(size_t)row * NGR + g] = dot;
            float scj;
            if constexpr (EXACT) scj = SC[j];
            else scj = (SENC ? bf16f(sv[j]) : f16f(sv[j])) * __uint_as_float(CS[j].y);
            acc = __builtin_fmaf(scj, (float)dot, acc);
            if (j == 0) stamp(5);
        }
    }
    stamp(6);
    acc = team_sum<TS>(acc);
    if constexpr (SWI) {
        // gate values through LDS; y0 receives the product, y1 / y2 (with
        // extra_out, each may be null) gate and up
        const uint16_t vb = f2bf(acc);
        if (l == 0 && row_ok) {
            if (!up) {
                lepi[rt] = vb;
                if (__builtin_expect(extra_out, 0) && y1 != nullptr) y1[row] = vb;
            } else if (__builtin_expect(extra_out, 0) && y2 != nullptr) {
                y2[row] = vb;
            }
        }
        lds_barrier();
        if (up && l == 0 && row_ok) y0[row] = f2bf(silu_mul(bf16f(lepi[rt]), bf16f(vb)));
    } else {
        if (l == 0 && row_ok) {
            if (__builtin_expect(res != nullptr, 0)) acc += bf16f(res[row]);
            y[row] = f2bf(acc);
        }
    }
    if constexpr (TLM) {
        stamp(7);
        if ((tid & 63) == 0) {
            uint64_t* o = (uint64_t*)part + ((size_t)blockIdx.x * (NTT / 64) + (tid >> 6)) * M1_TL_STAMPS;
#pragma unroll
            for (int i = 0; i < M1_TL_STAMPS; ++i) o[i] = tstamp[i];
        }
    }
}

typedef void (*m1_fn)(const void*, const uint8_t*, const uint16_t*, uint16_t*, int, int, int, int, const uint16_t*,
                      const void*, float, uint16_t*, int32_t*, const uint8_t*, const uint16_t*, uint16_t*, int,
                      const uint8_t*, const uint16_t*, uint16_t*, int);

// Launch shapes instantiated for every format: (team size, workgroup size,
// chunk slots per lane).
// 5 slots tile K = 2560 (Q4/Q5/Q6: 16 lanes), 5120 and 10240; 6 slots tile
// the reference engine's K = 3072 (16 lanes; W8: 32), 6144 (32; W8: 64) and
// 12288 (64 lanes).
// The 384-thread ones spread the engine's q (N = 6144) and o (N = 3072) over
// exactly one workgroup per CU (24 / 12 rows), where 256 / 320 threads left
// some CUs with twice the rows of others.
constexpr int M1_SHAPES[][3] = {{8, 128, 10}, {8, 192, 10}, {8, 320, 10}, {16, 256, 10}, {16, 640, 10},
                                {32, 320, 10}, {32, 640, 10}, {64, 640, 10}, {16, 256, 5}, {16, 320, 5},
                                {16, 640, 5}, {32, 640, 5}, {64, 640, 5}, {16, 256, 6}, {16, 320, 6},
                                {16, 384, 6}, {32, 320, 6}, {32, 384, 6}, {32, 640, 6}, {64, 640, 6}};
// Masked exact tilings (team size, workgroup size, chunk slots per lane,
// chunks per row): rows with no exact tiling of at most 10 slots per lane
// keep K constant and the staged scale block, and mask the last slots.  336
// chunks: the engine's K = 10752 (Q4/Q5/Q6), 64 lanes x 6 slots; 384 and 768
// threads put the engine's N = 3072 on 512 / 256 workgroups (6 / 12 rows).
// One Q4 / Q5 matrix of 96 chunks per row (K = 3072) whose 384-thread
// workgroups leave the CUs unevenly loaded: an 11-wave workgroup of 44 rows
// (m1_wide96 says when).
constexpr int M1_WIDE96[3] = {16, 704, 6};
constexpr int M1_MASKED[][4] = {{64, 320, 6, 336}, {64, 384, 6, 336}, {64, 640, 6, 336}, {64, 768, 6, 336}};

// Shapes of 5 or 6 chunk slots per lane are only ever exact tilings (m1_shape
// picks those by TS * CPL == chunks per row, or a masked tiling's chunks per
// row; other rows take 10 slots), so their non-exact variants are not built.
template <int F, int SENC, int MODE, bool EXACT, int PRO, int MR>
m1_fn m1_kernel_v(int ts, int ntt, int cpl, int kc) {
#define VQ_M1(TS_, NTT_, CPL_)                                                                      \
    if constexpr ((EXACT || CPL_ == 10) && (MODE != M1_SWIGLU || m1_pair_ok(TS_, NTT_)) &&          \
                  (MR == 1 || m1_mr_shape_ok(TS_, NTT_, CPL_)))                                     \
        if (ts == TS_ && ntt == NTT_ && cpl == CPL_ && kc == 0)                                     \
            return qgemv_m1_kernel<F, TS_, NTT_, CPL_, SENC, MODE, EXACT, PRO, MR,                          \
                                   m1_delay<F>(EXACT, TS_, NTT_, CPL_, MODE, MR, PRO)>;
    VQ_M1(8, 128, 10) VQ_M1(8, 192, 10) VQ_M1(8, 320, 10) VQ_M1(16, 256, 10) VQ_M1(16, 640, 10)
    VQ_M1(32, 320, 10) VQ_M1(32, 640, 10) VQ_M1(64, 640, 10) VQ_M1(16, 256, 5) VQ_M1(16, 320, 5)
    VQ_M1(16, 640, 5) VQ_M1(32, 640, 5) VQ_M1(64, 640, 5) VQ_M1(16, 256, 6) VQ_M1(16, 320, 6)
    VQ_M1(16, 384, 6) VQ_M1(32, 320, 6) VQ_M1(32, 384, 6) VQ_M1(32, 640, 6) VQ_M1(64, 640, 6)
    // the 44-row workgroup of one Q4 / Q5 matrix at K = 3072 (M1_WIDE96), bf16 or int8 row
    if constexpr (F == 4 || F == 5)
        if constexpr (MR == 1 && MODE != M1_SWIGLU && (PRO == PRO_BF16 || PRO == PRO_INT8))
            VQ_M1(M1_WIDE96[0], M1_WIDE96[1], M1_WIDE96[2])
#undef VQ_M1
    // masked exact tilings (KC_ chunks in TS_ * CPL_ slots), one row
#define VQ_M1K(TS_, NTT_, CPL_, KC_)                                                                \
    if constexpr (EXACT && MR == 1 && (MODE != M1_SWIGLU || m1_pair_ok(TS_, NTT_)))                  \
        if (ts == TS_ && ntt == NTT_ && cpl == CPL_ && kc == KC_)                                   \
            return qgemv_m1_kernel<F, TS_, NTT_, CPL_, SENC, MODE, EXACT, PRO, MR,                          \
                                   m1_delay<F>(EXACT, TS_, NTT_, CPL_, MODE, MR, PRO), KC_>;
    VQ_M1K(64, 320, 6, 336) VQ_M1K(64, 384, 6, 336) VQ_M1K(64, 640, 6, 336) VQ_M1K(64, 768, 6, 336)
#undef VQ_M1K
    return nullptr;
}

template <int F, int PRO, int MODE, int MR>
m1_fn m1_pick_mode(int ts, int ntt, int cpl, int kc, int senc, bool exact) {
    if (exact)
        return senc ? m1_kernel_v<F, 1, MODE, true, PRO, MR>(ts, ntt, cpl, kc)
                    : m1_kernel_v<F, 0, MODE, true, PRO, MR>(ts, ntt, cpl, kc);
    if (kc != 0) return nullptr;
    return senc ? m1_kernel_v<F, 1, MODE, false, PRO, MR>(ts, ntt, cpl, 0)
                : m1_kernel_v<F, 0, MODE, false, PRO, MR>(ts, ntt, cpl, 0);
}
// The swiglu pair is built for the BF16 and RMSNORM prologues (the inputs of
// the engine's gate/up projection); MR > 1 rows for BF16 and INT8; the
// partials (test entry point viper_hip_qlinear_partials) for BF16 only, the
// one prologue that entry point takes.
template <int F, int PRO>
m1_fn m1_pick_pro(int ts, int ntt, int cpl, int kc, int senc, int mode, bool exact, int mr) {
    constexpr bool PART_OK = PRO == PRO_BF16;
    if constexpr (PRO == PRO_BF16 || PRO == PRO_INT8) {
        if (mr == 2) {
            if constexpr (PART_OK)
                if (mode == M1_PART) return m1_pick_mode<F, PRO, M1_PART, 2>(ts, ntt, cpl, kc, senc, exact);
            if (mode == M1_PLAIN) return m1_pick_mode<F, PRO, M1_PLAIN, 2>(ts, ntt, cpl, kc, senc, exact);
            return nullptr;
        }
        if (mr == 4) {
            if constexpr (PART_OK)
                if (mode == M1_PART) return m1_pick_mode<F, PRO, M1_PART, 4>(ts, ntt, cpl, kc, senc, exact);
            if (mode == M1_PLAIN) return m1_pick_mode<F, PRO, M1_PLAIN, 4>(ts, ntt, cpl, kc, senc, exact);
            return nullptr;
        }
    }
    if (mr != 1) return nullptr;
    // the timeline: bf16 prologue, exact tilings
    if constexpr (PRO == PRO_BF16)
        if (mode == M1_TL)
            return !exact ? nullptr
                          : senc ? m1_kernel_v<F, 1, M1_TL, true, PRO, 1>(ts, ntt, cpl, kc)
                                 : m1_kernel_v<F, 0, M1_TL, true, PRO, 1>(ts, ntt, cpl, kc);
    if constexpr (PART_OK)
        if (mode == M1_PART) return m1_pick_mode<F, PRO, M1_PART, 1>(ts, ntt, cpl, kc, senc, exact);
    if constexpr (PRO == PRO_BF16 || PRO == PRO_RMSNORM)
        if (mode == M1_SWIGLU) return m1_pick_mode<F, PRO, M1_SWIGLU, 1>(ts, ntt, cpl, kc, senc, exact);
    if (mode == M1_PLAIN) return m1_pick_mode<F, PRO, M1_PLAIN, 1>(ts, ntt, cpl, kc, senc, exact);
    return nullptr;
}

// Kernels of format F with the quantize / int8 prologues and with the folded
// rmsnorm / swiglu prologues (each defined in its own translation unit).
template <int F>
m1_fn m1_pick_plain(int ts, int ntt, int cpl, int kc, int senc, int mode, bool exact, int pro, int mr);
template <int F>
m1_fn m1_pick_folded(int ts, int ntt, int cpl, int kc, int senc, int mode, bool exact, int pro, int mr);

#define VQ_M1_PLAIN(F)                                                                                         \
    template <>                                                                                                \
    m1_fn m1_pick_plain<F>(int ts, int ntt, int cpl, int kc, int senc, int mode, bool exact, int pro, int mr) { \
        return pro == PRO_INT8 ? m1_pick_pro<F, PRO_INT8>(ts, ntt, cpl, kc, senc, mode, exact, mr)               \
                               : m1_pick_pro<F, PRO_BF16>(ts, ntt, cpl, kc, senc, mode, exact, mr);              \
    }
#define VQ_M1_FOLDED(F)                                                                                         \
    template <>                                                                                                 \
    m1_fn m1_pick_folded<F>(int ts, int ntt, int cpl, int kc, int senc, int mode, bool exact, int pro, int mr) { \
        return pro == PRO_SWIGLU ? m1_pick_pro<F, PRO_SWIGLU>(ts, ntt, cpl, kc, senc, mode, exact, mr)             \
                                 : m1_pick_pro<F, PRO_RMSNORM>(ts, ntt, cpl, kc, senc, mode, exact, mr);           \
    }

}  // namespace vq
