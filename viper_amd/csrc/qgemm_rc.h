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
//
// Arguments.  Only the first 14 argument dwords arrive preloaded in SGPRs;
// a later argument is a scalar load from the argument buffer that the wave
// waits for (the weight-scale encoding read after the weight loads cost
// 0.17 us of the M = 16 verify, the residual pointer waited for before the
// first load 0.3 us).  So everything the common path reads before its loads
// fits 14 dwords: N, M - 1 and the encoding share one word (nm: N in bits
// 0..26, M - 1 in 27..30, the encoding in bit 31), K and the K split's part
// count share another (kk), the first matrix's workgroup count is derived
// from N (both matrices of a pair have N rows), and the K split's control
// words (sc, whose block counter is the split's first load) come before the
// residual, which is read only when the outputs are formed.
//
// Activation modes (AM): RC_FRAG reads the fragments and [group][16] scales
// the fragment quantize wrote; RC_NAT gathers them from the natural layout
// ([M][K] int8, [M][K/G] fp32); RC_BF16 takes the bf16 rows themselves: every
// workgroup issues its share of the M rows' octets before the weight stream,
// quantizes them while the weights are in flight into an LDS copy of the
// fragment layout (the fragment quantize's arithmetic: group max over the
// G/8 lanes of a group, the exact RNE quotient) and reads its operands from
// there after one LDS barrier.  That needs no quantize launch and no
// workspace traffic; it pays when few rows leave most of the lanes' quantize
// work useful (every workgroup repeats it).
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
constexpr int RC_SPIN = 4096; // K split: re-reads of a slot that still holds an earlier call's sum
constexpr int RC_XR = 8;      // RC_BF16: octets per thread held in registers (all rows in one pass)

__host__ __device__ constexpr size_t rc_wave_lds(int hstr) { return (size_t)16 * (RC_LSTR + hstr); }
__host__ __device__ constexpr size_t rc_lds_bytes(int hstr, int RB, int W) {
    return (size_t)W * rc_wave_lds(hstr) + (size_t)W * ((RB + 1) / 2) * 4 * 64 * 4;
}
// RC_BF16: the LDS copy of the fragments (64 lanes x QB bytes per group) and
// of the [group][16] activation scales, after the regions above.
__host__ __device__ constexpr size_t rc_act_lds_bytes(int qb, int ng) { return (size_t)ng * 64 * qb + (size_t)ng * 64; }
// Single-segment launches with fragment input stage their scales in LDS
// after the regions above: the weight scales of the workgroup's rows for its
// quads ([row][quad], 8 bytes each, rows of whole 16-row tiles), then the
// activation scales of its quads ([group][16] fp32).
__host__ __device__ constexpr size_t rc_stage_bytes(int RB, int nq) {
    return (size_t)16 * ((RB + 1) / 2) * nq * 8 + (size_t)nq * 256;
}

template <int F, int RB, int QW>
struct RcSeg {
    static constexpr int T = (RB + 1) / 2;
    static constexpr int HW = RcFmt<F>::HQ / 32 > 0 ? RcFmt<F>::HQ / 32 : 1;  // high words per lane and block
    u32x4 A[QW][4], XS[QW][4], WV[QW][RB];
    uint32_t HV[QW][RB][HW];
    u32x2 S[QW][T];
};

// ONE: the quads of every wave fit one load segment.  SE: the weight-scale
// encoding, fp16 (0) or bf16 (1) as a constant for the production variants
// (a run-time choice cost 0.1 us of the M = 16 verify), or read from nm (2)
// for the partials and natural-layout variants.  KS (fragment input only):
// K split into sk equal parts (sk = K's argument word >> 27, 2..RC_SK_MAX),
// one workgroup per (row block, part), blockIdx = sk * block + part; each
// part stores its fp32 sums to its block's record of slots, and the last
// part of a block to count adds the sk sums in part order, so the result
// does not depend on which part finishes last.  Partials (PART) are written
// by each part for its own groups.  PR: the launch may carry a fused pair
// (without it the matrix select is not compiled).
//
// The exchange between the parts of a block needs no launch before it and
// leaves the workspace ready for the next call of any shape.  Each sum
// travels in a 64-bit slot {tag, fp32 bits}, written and read as agent-scope
// relaxed atomics, at a place that depends only on (block, part, row m, row
// of the block): record `block` of RC_REC_SLOTS slots, so only that block
// ever writes it, whatever the shape.  The block's counter sc[RC_CTL_CNT +
// block] holds 64 * epoch + (parts of the running call that have counted):
// every part reads it when it starts (its first load: at most sk - 1 parts
// have counted by then, so every part sees the same epoch), tags its slots
// rc_tag(epoch) and counts once its slot stores are issued; the part that
// counts sk - 1 is the last and adds 64 - sk, which moves the counter to
// the next epoch for the next call.  No other word the library stores in a
// workspace can equal a tag: int8 activations are in [-127, 127] (never the
// byte 0x80) and fp32 activation scales are positive; counters live in their
// own region.  So in a workspace zero-filled before its first use, a slot
// that carries the block's current tag was written by this call (a slot
// written 2^24 epochs earlier and not rewritten since is the only
// exception).  The last part accepts a slot only when it carries the current
// tag and re-reads it otherwise (bounded by RC_SPIN; then the output is NaN
// and sc[RC_CTL_MISS] is incremented, a count the library never clears).  So
// the result depends only on the coherence of the atomic accesses to each
// slot, not on any ordering between the slots and the counter.  (An
// agent-scope release/acquire pair would order them but costs a write-back
// and an invalidate of the XCD's L2 per workgroup: 70 us on the down shape.)
// The last part requests every slot at once, then re-reads any that does not
// yet carry the current tag.
// TLM (measurement, fragment input, one segment): `part` receives per-wave
// s_memrealtime readings (100 MHz) at RC_TL_STAMPS points --
// [workgroup][wave][RC_TL_STAMPS] uint64: wave start, activation and scale
// loads issued, weight loads issued, staged scales in LDS, first group
// scaled, last group scaled, cross-wave barrier passed, sums stored (y, or
// with the K split the part's slots), counted (K split: the block's counter
// returned), outputs stored (K split: y by the block's last part; the other
// parts repeat the previous reading; without the split both repeat it).
constexpr int RC_TL_STAMPS = 10;
template <int F, int RB, int W, int QW, bool ONE, int AM, bool PART, int SE, bool KS = false, bool PR = true,
          bool TLM = false>
__global__ void __launch_bounds__(64 * W)
qgemm_rc_kernel(const int8_t* xq, const float* xs, const uint8_t* w, const uint16_t* ws, uint16_t* y, unsigned kk,
                unsigned nm, unsigned* __restrict__ sc, const uint16_t* res, int32_t* __restrict__ part,
                const uint8_t* w1, const uint16_t* ws1, uint16_t* y1) {
    using FM = RcFmt<F>;
    using Seg = RcSeg<F, RB, QW>;
    constexpr int T = Seg::T;
    constexpr bool XNAT = AM == RC_NAT, XBF = AM == RC_BF16;
    static_assert(!KS || AM == RC_FRAG, "the K split reads fragments");
    static_assert(!TLM || (ONE && !PART && AM == RC_FRAG), "timeline: one fragment-input segment");
    // K in bits 0..26, the K split's part count in 27..31
    const int K = (int)(kk & 0x07FFFFFFu), SK = KS ? (int)(kk >> 27) : 1;
    uint64_t tstamp[RC_TL_STAMPS];
    auto stamp = [&](int i) {
        if constexpr (TLM) tstamp[i] = __builtin_amdgcn_s_memrealtime();
    };
    // lane 0 of every wave writes its readings (points past `upto` repeat it)
    auto flush_stamps = [&](int upto) {
        if constexpr (TLM) {
            if ((threadIdx.x & 63) == 0) {
                uint64_t* o = (uint64_t*)part + ((size_t)blockIdx.x * W + (threadIdx.x >> 6)) * RC_TL_STAMPS;
#pragma unroll
                for (int i = 0; i < RC_TL_STAMPS; ++i) o[i] = tstamp[i <= upto ? i : upto];
            }
        }
    };
    stamp(0);
    constexpr int G = F == 8 ? 32 : 64;
    extern __shared__ __align__(16) uint8_t smem[];
    // the wave index as a scalar: per-quad conditions are then uniform branches
    const int tid = (int)threadIdx.x, L = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int n16 = L & 15, kb = L >> 4, qi = ((kb & 1) << 1) | (kb >> 1);
    const int NG = K / G, NQ = NG / 4 / SK;  // quads of this workgroup's part of K
    const int nseg = ONE ? 1 : (NQ + W * QW - 1) / (W * QW);
    const int N = (int)(nm & ((1u << 27) - 1)), M = (int)((nm >> 27) & 15u) + 1;
    const bool senc = SE == 2 ? (nm >> 31) != 0 : SE == 1;
    const int nb0 = (N + 8 * RB - 1) / (8 * RB);
    int bid = (int)blockIdx.x;
    int q0 = 0;  // first quad of the part
    uint32_t cnt0 = 0;
    if constexpr (KS) {
        q0 = (int)(blockIdx.x % SK) * NQ;
        bid = (int)(blockIdx.x / SK);
        // the block's counter, for its epoch: the first vector load of the
        // kernel, so it returns ahead of the weights (loads retire in issue
        // order), with sc among the preloaded arguments (a scalar load of the
        // counter through an sc read from the argument buffer measured
        // 0.25-0.45 us slower at the down shape)
        cnt0 = bload4(buf(sc + RC_CTL_CNT + bid, 4u), 0);
        issue_fence();
    }
    // the second matrix of a fused pair and the residual are the rare paths:
    // marked unlikely, the common path is laid out and scheduled straight
    if (PR && __builtin_expect(bid >= nb0, 0)) {
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
    // (with a K split the resources start at the part's first quad: the
    // offsets below stay those of an unsplit launch with NQ quads)
    const uint8_t* wp = w + (size_t)row0 * rbytes + q0 * 128;
    const uint8_t* hp = w + (size_t)N * rbytes + (size_t)row0 * hrb + q0 * FM::HQ;
    const uint16_t* sp0 = ws + (size_t)row0 * NG + 4 * q0;
    const int8_t* xp = xq + (size_t)q0 * 4 * 64 * FM::QB;
    const float* xsp = xs + (size_t)q0 * 4 * 16;
    const uint32_t wn = (uint32_t)(nrows * rbytes - q0 * 128), hn = (uint32_t)(nrows * hrb - q0 * FM::HQ);
    const uint32_t sn = (uint32_t)(nrows * NG - 4 * q0) * 2;
    const uint32_t xn = XNAT ? (uint32_t)(M * K) : XBF ? (uint32_t)(M * K) * 2 : (uint32_t)(NG - 4 * q0) * 64 * FM::QB;
    const uint32_t xsn = XNAT ? (uint32_t)(M * NG * 4) : XBF ? 0u : (uint32_t)(NG - 4 * q0) * 64;
    const auto xr = buf(xp, xn);
    const auto xsr = buf(xsp, xsn);
    const bool m_ok = n16 < M;  // A row of this lane
    // RC_BF16: the LDS fragments and scales (after the transpose buffers and
    // the cross-wave sums)
    int8_t* lxq = (int8_t*)(smem + rc_lds_bytes(FM::HSTR, RB, W));
    float* lxs = (float*)(lxq + (size_t)NQ * 4 * 64 * FM::QB);
    constexpr int NTT = 64 * W;
    const int KO = K / 8, noct = M * KO;  // RC_BF16: octets of all rows
    u32x4 xv[XBF ? RC_XR : 1];
    if constexpr (XBF) {
        // every octet this thread quantizes, before any weight request: two
        // consecutive octets of a group per round (pair p = octets 2p, 2p + 1;
        // with 64-groups, 16-byte fragment slots, they share one slot, with
        // 32-groups, W8's 8-byte slots, they go to two)
#pragma unroll
        for (int i = 0; i < RC_XR; ++i) {
            xv[i] = u32x4{0u, 0u, 0u, 0u};
            const int r = i >> 1;  // pair round; octet 2p + (i & 1) of pair p
            if (r == 0 || NTT * r < noct / 2) xv[i] = bload16(xr, ((tid + NTT * r) * 2 + (i & 1)) * 16);
        }
        issue_fence();
    }
    // Staged scales (single segment, fragment input): the block's weight
    // scales for this part's NQ quads in 8-byte pieces (piece c = row c % 8RB
    // of quad c / 8RB) and the part's activation scales in 16-byte pieces,
    // one or two loads per thread instead of a load per lane, tile and quad
    // (those small loads, queued ahead of every wave's weights: down shape
    // M = 4 9.4 -> 9.1 us, M = 16 10.0 -> 9.7 us).  Rows past the block read
    // as zero.  RC_BF16 stages the weight scales only (its activation scales
    // are the quantize's), stored after the rows' quantize so that it does not
    // wait for them from HBM.  Not for Q5/Q6, whose high-plane loads follow (8
    // rows: 8.5 / 8.7 -> 9.1 / 9.3 us).  (Forming the products ws * xs here, before the weights
    // arrive, took 32-48 more VGPRs: the K split lost its second workgroup
    // per CU.)
    constexpr bool STG = ONE && (AM == RC_FRAG || XBF) && FM::HQ == 0;
    constexpr int R8 = 8 * RB;
    constexpr int SI = (R8 * QW + 63) / 64;  // pieces per thread: 8RB * NQ <= 8RB * W * QW
    uint8_t* wsl = smem + rc_lds_bytes(FM::HSTR, RB, W) + (XBF ? rc_act_lds_bytes(FM::QB, 4 * NQ) : 0);
    uint8_t* xsl = wsl + (size_t)16 * T * NQ * 8;
    u32x2 stw[STG ? SI : 1];
    u32x4 stx = {0u, 0u, 0u, 0u};
    if constexpr (STG) {
        const auto wst = buf(ws + (size_t)row0 * NG, (uint32_t)(nrows * NG) * 2);
#pragma unroll
        for (int i = 0; i < SI; ++i) {
            const int c = tid + NTT * i, q = c / R8, r = c - q * R8;
            stw[i] = bload8(wst, q < NQ ? (r * NG + 4 * (q0 + q)) * 2 : OOB);
        }
        if constexpr (!XBF) stx = bload16(xsr, tid < NQ * 16 ? tid * 16 : OOB);
    }

    auto load = [&](Seg& S, int seg) {
#pragma unroll
        for (int j = 0; j < QW; ++j) {
            // a wave past the part's last quad loads nothing: its resources
            // are empty (sizes chosen by a uniform condition), which needs no
            // per-lane select or branch around the loads
            const int Q = wave + W * (seg * QW + j);
            const bool ok = Q < NQ;
            const auto xrj = buf(xp, ok ? xn : 0u), xsrj = buf(xsp, ok ? xsn : 0u), srj = buf(sp0, ok ? sn : 0u);
#pragma unroll
            for (int h = 0; h < 4 && !XBF; ++h) {
                const int g = 4 * Q + h;
                int ao;
                if constexpr (XNAT) ao = m_ok ? n16 * K + g * G + FM::QB * qi : OOB;
                else ao = m_ok ? (g * 64 + L) * FM::QB : OOB;
                if constexpr (FM::QB == 16) {
                    S.A[j][h] = bload16(xrj, ao);
                } else {
                    const u32x2 v = bload8(xrj, ao);
                    S.A[j][h] = u32x4{v.x, v.y, 0u, 0u};
                }
                if constexpr (XNAT) {
                    uint32_t v[4];
#pragma unroll
                    for (int r = 0; r < 4; ++r) v[r] = bload4(xsrj, 4 * kb + r < M ? ((4 * kb + r) * NG + g) * 4 : OOB);
                    S.XS[j][h] = u32x4{v[0], v[1], v[2], v[3]};
                } else if constexpr (!STG) {
                    S.XS[j][h] = bload16(xsrj, (g * 16 + 4 * kb) * 4);
                }
            }
            if constexpr (!STG)
#pragma unroll
                for (int t = 0; t < T; ++t) S.S[j][t] = bload8(srj, ((16 * t + n16) * NG + 4 * Q) * 2);
        }
        issue_fence();
        if (seg == 0) stamp(1);
#pragma unroll
        for (int j = 0; j < QW; ++j) {
            const int Q = wave + W * (seg * QW + j);
            const bool ok = Q < NQ;
            const auto wrj = buf(wp, ok ? wn : 0u), hrj = buf(hp, ok ? hn : 0u);
#pragma unroll
            for (int b = 0; b < RB; ++b) {
                const int rw = 8 * b + (L >> 3);
                S.WV[j][b] = bload16<AUX_NT>(wrj, rw * rbytes + (8 * Q + (L & 7)) * 16);
                if constexpr (FM::HQ == 32) {
                    S.HV[j][b][0] = bload4<AUX_NT>(hrj, rw * hrb + Q * 32 + (L & 7) * 4);
                } else if constexpr (FM::HQ == 64) {
                    const u32x2 hh = bload8<AUX_NT>(hrj, rw * hrb + Q * 64 + (L & 7) * 8);
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
                // weight scales of the quad's groups for each tile, decoded
                // once per quad under one uniform branch (a select per group
                // inside the MFMA loop became a branch pair per group and
                // tile, 0.4 us of the M = 16 verify)
                float WSV[T][4];
                if (senc) {
#pragma unroll
                    for (int t = 0; t < T; ++t) {
                        WSV[t][0] = bf16f(S.S[j][t].x & 0xffffu);
                        WSV[t][1] = bf16f(S.S[j][t].x >> 16);
                        WSV[t][2] = bf16f(S.S[j][t].y & 0xffffu);
                        WSV[t][3] = bf16f(S.S[j][t].y >> 16);
                    }
                } else {
#pragma unroll
                    for (int t = 0; t < T; ++t) {
                        WSV[t][0] = f16f(S.S[j][t].x & 0xffffu);
                        WSV[t][1] = f16f(S.S[j][t].x >> 16);
                        WSV[t][2] = f16f(S.S[j][t].y & 0xffffu);
                        WSV[t][3] = f16f(S.S[j][t].y >> 16);
                    }
                }
#pragma unroll
                for (int h = 0; h < 4; ++h) {
                    u32x4 a;
                    if constexpr (XBF) {
                        const int8_t* fa = lxq + ((size_t)(4 * Q + h) * 64 + L) * FM::QB;
                        if constexpr (FM::QB == 16) {
                            a = *(const u32x4*)fa;
                        } else {
                            const u32x2 v = *(const u32x2*)fa;
                            a = u32x4{v.x, v.y, 0u, 0u};
                        }
                        S.XS[j][h] = *(const u32x4*)(lxs + (4 * Q + h) * 16 + 4 * kb);
                    } else {
                        a = S.A[j][h];
                    }
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
                        const float wsf = WSV[t][h];
                        const float xf[4] = {__uint_as_float(S.XS[j][h].x), __uint_as_float(S.XS[j][h].y),
                                             __uint_as_float(S.XS[j][h].z), __uint_as_float(S.XS[j][h].w)};
#pragma unroll
                        for (int r = 0; r < 4; ++r) acc[t][r] = __builtin_fmaf(wsf * xf[r], (float)C[r], acc[t][r]);
                        if constexpr (TLM)
                            if (j == 0 && t == 0 && h == 0) stamp(4);
                        if constexpr (PART) {
                            if (16 * t + n16 < nrows) {
#pragma unroll
                                for (int r = 0; r < 4; ++r)
                                    if (4 * kb + r < M) part[((size_t)(4 * kb + r) * N + n) * NG + 4 * (q0 + Q) + h] = C[r];
                            }
                        }
                    }
                }
            }
        }
    };

    // RC_BF16: quantize the staged octets into the LDS fragments while the
    // first segment's weights are in flight.  Octet o of row m = o / KO sits
    // in group g = k8 / (G/8) at octet j = k8 % (G/8); the lane that supplies
    // it to the MFMA is 16 * bitswap(quarter) + m (quarter = j / 2 for 64-groups,
    // = j for 32-groups).  Trip counts are wave-uniform, so every DPP group
    // reduction sees whole groups.
    auto quantize = [&] {
        const int wave0 = tid & ~63;
        // pair p = octets 2p, 2p + 1 (j, j + 1 of a group, j even): the
        // group's amax over its G / 16 lanes, the same bytes as one octet per
        // thread (quantize_octet_pair)
#pragma unroll
        for (int r = 0; r < RC_XR / 2; ++r) {
            if (wave0 + NTT * r < noct / 2) {
                const int p = tid + NTT * r;
                uint32_t d0, d1, d2, d3;
                float sc;
                quantize_octet_pair<G, (F != 8)>(xv[2 * r], xv[2 * r + 1], d0, d1, d2, d3, sc);
                if (p < noct / 2) {
                    const int o = 2 * p, m = o / KO, k8 = o - m * KO;
                    if constexpr (G == 64) {  // one 16-byte slot
                        const int g = k8 / 8, q = (k8 % 8) >> 1;
                        const int slot = ((q & 1) << 1) | (q >> 1);
                        *(u32x4*)(lxq + ((size_t)g * 64 + 16 * slot + m) * 16) = u32x4{d0, d1, d2, d3};
                        if (k8 % 8 == 0) lxs[g * 16 + m] = sc;
                    } else {  // two 8-byte slots
                        const int g = k8 / 4, q0 = k8 % 4, q1 = q0 + 1;
                        const int s0 = ((q0 & 1) << 1) | (q0 >> 1), s1 = ((q1 & 1) << 1) | (q1 >> 1);
                        *(u32x2*)(lxq + ((size_t)g * 64 + 16 * s0 + m) * 8) = u32x2{d0, d1};
                        *(u32x2*)(lxq + ((size_t)g * 64 + 16 * s1 + m) * 8) = u32x2{d2, d3};
                        if (q0 == 0) lxs[g * 16 + m] = sc;
                    }
                }
            }
        }
    };

    if constexpr (ONE) {
        Seg S;
        load(S, 0);
        stamp(2);
        // RC_BF16: the rows' quantize first (its octets arrive ahead of the
        // weight scales, which come from HBM), then the staging stores, one
        // barrier for both
        if constexpr (XBF) {
            issue_fence();
            quantize();
        }
        if constexpr (STG) {
            issue_fence();  // the weight requests stay ahead of the staging stores
#pragma unroll
            for (int i = 0; i < SI; ++i) {
                const int c = tid + NTT * i, q = c / R8, r = c - q * R8;
                if (q < NQ) *(u32x2*)(wsl + (r * NQ + q) * 8) = stw[i];
            }
            if constexpr (!XBF)
                if (tid < NQ * 16) *(u32x4*)(xsl + tid * 16) = stx;
        }
        if constexpr (STG || XBF) lds_barrier();
        if constexpr (STG) {
#pragma unroll
            for (int j = 0; j < QW; ++j) {
                const int Q = wave + W * j;
                if (Q < NQ) {
#pragma unroll
                    for (int t = 0; t < T; ++t) S.S[j][t] = *(const u32x2*)(wsl + ((16 * t + n16) * NQ + Q) * 8);
                    if constexpr (!XBF)
#pragma unroll
                        for (int h = 0; h < 4; ++h) S.XS[j][h] = *(const u32x4*)(xsl + ((4 * Q + h) * 16 + 4 * kb) * 4);
                }
            }
        }
        stamp(3);
        if (wave >= NQ) stamp(4);  // a wave with no quad scales no group
        compute(S, 0);
        stamp(5);
    } else {
        Seg S0, S1;
        load(S0, 0);
        if constexpr (XBF) {
            quantize();
            lds_barrier();
        }
        for (int seg = 0; seg < nseg; seg += 2) {
            load(S1, seg + 1);  // past the last segment every load is out of range: no traffic
            compute(S0, seg);
            load(S0, seg + 2);
            compute(S1, seg + 1);
        }
    }

    // cross-wave sum in wave order, residual, bf16 store (K split: the part's
    // sums to its slots, kept in registers too: at most MINE per thread)
    float* red = (float*)(smem + (size_t)W * rc_wave_lds(FM::HSTR));
#pragma unroll
    for (int t = 0; t < T; ++t)
#pragma unroll
        for (int r = 0; r < 4; ++r) red[((wave * T + t) * 4 + r) * 64 + L] = acc[t][r];
    __syncthreads();
    stamp(6);
    constexpr int MINE = (4 * T + W - 1) / W;
    float mine[MINE] = {};
    const int kpart = KS ? (int)(blockIdx.x % SK) : 0;
    // K split: the block's record of slots and this call's tag
    uint64_t* rec = KS ? (uint64_t*)((uint8_t*)sc + RC_CTL_BYTES) + (size_t)bid * RC_REC_SLOTS : nullptr;
    const unsigned tag = rc_tag((unsigned)__builtin_amdgcn_readfirstlane((int)cnt0) >> 6);
#pragma unroll
    for (int i = 0; i < MINE; ++i) {
        const int sl = wave + i * W;
        if (sl >= 4 * T) break;
        const int t = sl >> 2, r = sl & 3;
        float v = 0.0f;
#pragma unroll
        for (int u = 0; u < W; ++u) v += red[((u * T + t) * 4 + r) * 64 + L];
        mine[i] = v;
        const int m = 4 * kb + r, nl = 16 * t + n16;
        if (m < M && nl < nrows) {
            const size_t o = (size_t)m * N + row0 + nl;
            if constexpr (KS) {
                __hip_atomic_store(rec + (kpart * 16 + m) * RC_REC_ROWS + nl, ((uint64_t)tag << 32) | __float_as_uint(v),
                                   __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            } else {
                if (__builtin_expect(res != nullptr, 0)) v += bf16f(res[o]);
                y[o] = f2bf(v);
            }
        }
    }
    stamp(7);
    if constexpr (!KS) flush_stamps(7);
    if constexpr (KS) {
        // count once every wave's slot stores are issued; a slot whose store
        // is still in flight when the last part reads it is re-read (waiting
        // for the stores to complete before counting measured 0.4 us slower).
        // The last part moves the counter to the next epoch (64 * (epoch + 1)).
        // (A fixed part that adds the sums without counting, the last one
        // dispatched, saves the counter's round trip but waits as long for
        // the other parts' slots, 7.8 against 7.7 us at the down shape, and a
        // part delayed by other work on the GPU would leave it spinning.)
        lds_barrier();
        int* last = (int*)red;
        if (tid == 0) {
            unsigned* cnt = sc + RC_CTL_CNT + bid;
            const unsigned old = __hip_atomic_fetch_add(cnt, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            const int is_last = (int)(old & 63u) == SK - 1;
            if (is_last) __hip_atomic_fetch_add(cnt, (unsigned)(64 - SK), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            last[0] = is_last;
        }
        lds_barrier();
        stamp(8);
        if (!last[0]) {
            flush_stamps(8);
            return;
        }
        // every slot of the other parts is requested at once (a load that
        // waited for the previous one's tag would serialise the round trips:
        // 0.4 us of the down-shape launch), then the tags are checked and a
        // slot that does not carry this call's tag yet is re-read
        uint64_t u[MINE][RC_SK_MAX];
#pragma unroll
        for (int i = 0; i < MINE; ++i) {
            const int sl = wave + i * W;
            const int t = sl >> 2, r = sl & 3;
            const int m = 4 * kb + r, nl = 16 * t + n16;
            const bool ok = sl < 4 * T && m < M && nl < nrows;
#pragma unroll
            for (int p = 0; p < RC_SK_MAX; ++p) {
                u[i][p] = ((uint64_t)tag << 32) | __float_as_uint(mine[i]);
                if (ok && p < SK && p != kpart)
                    u[i][p] = __hip_atomic_load(rec + (p * 16 + m) * RC_REC_ROWS + nl, __ATOMIC_RELAXED,
                                                __HIP_MEMORY_SCOPE_AGENT);
            }
        }
        unsigned missed = 0;  // sums that never arrived (NaN in y), counted in the workspace
#pragma unroll
        for (int i = 0; i < MINE; ++i) {
            const int sl = wave + i * W;
            if (sl >= 4 * T) break;
            const int t = sl >> 2, r = sl & 3;
            const int m = 4 * kb + r, nl = 16 * t + n16;
            if (m < M && nl < nrows) {
                const size_t o = (size_t)m * N + row0 + nl;
                float v = 0.0f;
#pragma unroll
                for (int p = 0; p < RC_SK_MAX; ++p) {
                    if (p >= SK) break;
                    uint64_t w = u[i][p];
                    if (__builtin_expect((unsigned)(w >> 32) != tag, 0)) {
                        uint64_t* a = rec + (p * 16 + m) * RC_REC_ROWS + nl;
                        for (int it = 0; (unsigned)(w >> 32) != tag && it < RC_SPIN; ++it)
                            w = __hip_atomic_load(a, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                    }
                    const bool ok = (unsigned)(w >> 32) == tag;
                    missed += !ok;
                    v += ok ? __uint_as_float((unsigned)w) : __builtin_nanf("");
                }
                if (__builtin_expect(res != nullptr, 0)) v += bf16f(res[o]);
                y[o] = f2bf(v);
            }
        }
        if (__builtin_expect(missed != 0, 0))
            __hip_atomic_fetch_add(sc + RC_CTL_MISS, missed, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        stamp(9);
        flush_stamps(9);
    }
}

// ------------------------------------------------------------------ host side

typedef void (*rc_fn)(const int8_t*, const float*, const uint8_t*, const uint16_t*, uint16_t*, unsigned, unsigned,
                      unsigned*, const uint16_t*, int32_t*, const uint8_t*, const uint16_t*, uint16_t*);

// Launch shape: rows per workgroup (8 * rb), waves, quads per wave per
// segment, single segment or double-buffered loop.
struct RcShape {
    int rb, w, qw;
    bool one;
    int sk = 1;  // parts of K (1: no split, else 2..RC_SK_MAX)
};
// Most 8-row blocks per workgroup that two quads per wave, or the
// double-buffered segment loop, hold in registers without spilling.
__host__ __device__ constexpr int rc_rb_qw2(int F) { return F == 8 ? 6 : F == 6 ? 3 : 4; }
constexpr int RC_RB_LOOP = 2;

template <int F, int RB, int W, int QW, bool ONE, int AM, int SE>
rc_fn rc_pick5(bool pair) {
    return pair ? qgemm_rc_kernel<F, RB, W, QW, ONE, AM, false, SE, false, true>
                : qgemm_rc_kernel<F, RB, W, QW, ONE, AM, false, SE, false, false>;
}
template <int F, int RB, int W, int QW, bool ONE>
rc_fn rc_pick4(int am, bool part, int senc, bool pair) {
    if (am == RC_NAT)  // the prequantized entry points, which write no partials
        return part ? nullptr : qgemm_rc_kernel<F, RB, W, QW, ONE, RC_NAT, false, 2>;
    if (part)
        return am == RC_BF16 ? qgemm_rc_kernel<F, RB, W, QW, ONE, RC_BF16, true, 2>
                             : qgemm_rc_kernel<F, RB, W, QW, ONE, RC_FRAG, true, 2>;
    if (am == RC_BF16)
        return senc ? rc_pick5<F, RB, W, QW, ONE, RC_BF16, 1>(pair) : rc_pick5<F, RB, W, QW, ONE, RC_BF16, 0>(pair);
    return senc ? rc_pick5<F, RB, W, QW, ONE, RC_FRAG, 1>(pair) : rc_pick5<F, RB, W, QW, ONE, RC_FRAG, 0>(pair);
}
template <int F, int RB, int QW>
rc_fn rc_pick_split(int senc, bool part) {
    if (part) return qgemm_rc_kernel<F, RB, 10, QW, true, RC_FRAG, true, 2, true, false>;
    return senc ? qgemm_rc_kernel<F, RB, 10, QW, true, RC_FRAG, false, 1, true, false>
                : qgemm_rc_kernel<F, RB, 10, QW, true, RC_FRAG, false, 0, true, false>;
}
template <int F, int RB>
rc_fn rc_pick3(const RcShape& s, int am, bool part, int senc, bool pair) {
    if (s.sk != 1) {  // K split: fragment input, one segment of 10 waves
        if (s.sk < 2 || s.sk > RC_SK_MAX || am != RC_FRAG || !s.one || s.w != 10 || pair) return nullptr;
        if (s.qw == 1) return rc_pick_split<F, RB, 1>(senc, part);
        if constexpr (RB <= rc_rb_qw2(F))
            if (s.qw == 2) return rc_pick_split<F, RB, 2>(senc, part);
        return nullptr;
    }
    if (s.one && s.w == 4 && s.qw == 1) return rc_pick4<F, RB, 4, 1, true>(am, part, senc, pair);
    if (s.one && s.w == 10 && s.qw == 1) return rc_pick4<F, RB, 10, 1, true>(am, part, senc, pair);
    if (s.one && s.w == 12 && s.qw == 1) return rc_pick4<F, RB, 12, 1, true>(am, part, senc, pair);
    if constexpr (RB <= rc_rb_qw2(F))
        if (s.one && s.w == 10 && s.qw == 2) return rc_pick4<F, RB, 10, 2, true>(am, part, senc, pair);
    if constexpr (RB <= RC_RB_LOOP)
        if (!s.one && s.w == 10 && s.qw == 1) return rc_pick4<F, RB, 10, 1, false>(am, part, senc, pair);
    return nullptr;
}
template <int F>
rc_fn rc_pick2(const RcShape& s, int am, bool part, int senc, bool pair) {
    switch (s.rb) {
        case 1: return rc_pick3<F, 1>(s, am, part, senc, pair);
        case 2: return rc_pick3<F, 2>(s, am, part, senc, pair);
        case 3: return rc_pick3<F, 3>(s, am, part, senc, pair);
        case 4: return rc_pick3<F, 4>(s, am, part, senc, pair);
        case 5: return rc_pick3<F, 5>(s, am, part, senc, pair);
        case 6: return rc_pick3<F, 6>(s, am, part, senc, pair);
        default: return nullptr;
    }
}

// Timeline kernels (fragment input, one segment; Q4 only, qgemm_rc_q4.hip).
template <int F, int RB>
rc_fn rc_pick_tl3(const RcShape& s, int senc) {
#define VQ_RC_TL(W_, QW_, KS_)                                                                         \
    if (s.w == W_ && s.qw == QW_ && (s.sk > 1) == KS_)                                                 \
        return senc ? qgemm_rc_kernel<F, RB, W_, QW_, true, RC_FRAG, false, 1, KS_, false, true>       \
                    : qgemm_rc_kernel<F, RB, W_, QW_, true, RC_FRAG, false, 0, KS_, false, true>;
    VQ_RC_TL(4, 1, false)
    VQ_RC_TL(10, 1, false)
    VQ_RC_TL(12, 1, false)
    VQ_RC_TL(10, 1, true)
    if constexpr (RB <= rc_rb_qw2(F)) {
        VQ_RC_TL(10, 2, false)
        VQ_RC_TL(10, 2, true)
    }
#undef VQ_RC_TL
    return nullptr;
}
template <int F>
rc_fn rc_pick_tl(const RcShape& s, int senc) {
    if (!s.one) return nullptr;
    switch (s.rb) {
        case 1: return rc_pick_tl3<F, 1>(s, senc);
        case 2: return rc_pick_tl3<F, 2>(s, senc);
        case 3: return rc_pick_tl3<F, 3>(s, senc);
        case 4: return rc_pick_tl3<F, 4>(s, senc);
        case 5: return rc_pick_tl3<F, 5>(s, senc);
        case 6: return rc_pick_tl3<F, 6>(s, senc);
        default: return nullptr;
    }
}
rc_fn rc_pick_tl4(const RcShape& s, int senc);
rc_fn rc_pick_tl8(const RcShape& s, int senc);

// Kernels of format F (each defined in its own translation unit).
template <int F>
rc_fn rc_pick(const RcShape& s, int am, bool part, int senc, bool pair);

#define VQ_RC_PICK(F) \
    template <>       \
    rc_fn rc_pick<F>(const RcShape& s, int am, bool part, int senc, bool pair) { return rc_pick2<F>(s, am, part, senc, pair); }

}  // namespace vq
