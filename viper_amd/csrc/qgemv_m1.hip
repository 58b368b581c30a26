#include "qlinear_host.h"

namespace vq {

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

size_t lds_m1(int qtype, int K) {
    switch (qtype) {
        case VIPER_QTYPE_Q4_G64: return m1_lds_bytes<4>(K);
        case VIPER_QTYPE_Q5_G64: return m1_lds_bytes<5>(K);
        case VIPER_QTYPE_Q6_G64: return m1_lds_bytes<6>(K);
        default: return m1_lds_bytes<8>(K);
    }
}

int launch_m1(int qtype, const void* w, const void* s, int senc, int N, int K,
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

}  // namespace vq
