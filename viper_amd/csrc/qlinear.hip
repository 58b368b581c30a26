// Quantized linear for MI355X (gfx950): y = bf16( sum_g ws*xs*D_g [+ res] ).
//
// Semantics follow the reference's int8 decode path (itzrnvr/viper):
// activation quantize as kernels/ops/rmsnorm_quantize.cu:71-104 and
// linear_multim.cu:21-61 (per-row, per-group amax/127 floored at 1e-8,
// round-to-nearest-even of x/scale), group dot + fp32 combine as
// kernels/ops/dp4a_smem_kernel.cu:25-74 and linear_multim.cu:64-130, weight
// layout as tools/convert/convert.cpp:91-127.  The design is gfx950's own.
//
// M = 1 (qgemv_m1_kernel in qgemv_m1.h, the decode GEMV): teams of 16-64
// lanes stream output rows with 16-byte non-temporal loads; each workgroup
// quantizes the bf16 activation into LDS while its weights are in flight,
// the int32 group dots are exact (v_dot8 on split activation nibbles for Q4,
// v_dot4 on offset codes for Q5/Q6/W8) and the fp32 combine is reduced with
// DPP in a fixed order (deterministic).
//
// M = 2..16 (qgemm_rc.h, qgemm_mfma.hip, qgemm_pre.hip): activations are
// quantized once into a caller workspace (quantize_frag64_kernel in the
// matrix-core fragment order, else quantize_act_kernel) or supplied by the
// caller, and every weight byte is read once for all M rows.
//
// The activation quantizer never divides per element: with s the group scale
// (an IEEE divide amax/127, once per group) and r = rcp(s) (the hardware
// reciprocal, within 1 ulp), q0 = x*r and q1 = fma(fma(-q0, s, x), r, q0);
// adding 1.5*2^23 rounds q1 to the nearest even integer and leaves it, two's
// complement, in the low byte.  For every finite bf16 pair (amax, x) the byte
// equals RNE(x/s): check_quantizer_kernel verifies that exhaustively on the
// device (and the CPU oracle the same steps with an IEEE 1/s).

#include "qlinear_host.h"

#include <mutex>

namespace vq {

// ------------------------------------------------ allocation-free entry point

// The workspace of viper_hip_qlinear_static: a file-scope device array, one
// copy on every device the library runs on, held until the process ends.  In
// host code `scratch` names a host-side stand-in, never device memory: the
// device address comes from hipGetSymbolAddress, taken once per device with
// that device current and kept in scratch_dev.
constexpr size_t STATIC_SCRATCH_BYTES = VIPER_QLINEAR_STATIC_SCRATCH_BYTES;
static __device__ __align__(256) uint8_t scratch[STATIC_SCRATCH_BYTES];

constexpr int MAX_DEVICES = 64;
static std::mutex scratch_mu;
static void* scratch_dev[MAX_DEVICES];

// Device address of the current device's scratch (looked up on its first use).
static int scratch_address(void** out) {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) return VIPER_DEVICE_ERROR;
    if (dev < 0 || dev >= MAX_DEVICES) return VIPER_INTERNAL;
    std::lock_guard<std::mutex> lock(scratch_mu);
    if (scratch_dev[dev] == nullptr) {
        void* p = nullptr;
        const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess || p == nullptr) return VIPER_DEVICE_ERROR;
        scratch_dev[dev] = p;
    }
    *out = scratch_dev[dev];
    return VIPER_OK;
}

// ------------------------------------------------ standalone activation quantize

// MF: the fragment order the matrix-core kernels read (xs transposed to
// [K/G][16]; 64-groups use quantize_frag64_kernel); else xq [M][K] in k order
// and xs [M][K/G].
template <int G, bool MF>
__global__ void __launch_bounds__(NT)
quantize_act_kernel(const uint16_t* x, int8_t* __restrict__ xq,
                    float* __restrict__ xs, int oct_total, int K) {
    const int o = (int)blockIdx.x * NT + (int)threadIdx.x;
    const bool ok = o < oct_total;
    u32x4 v = {0u, 0u, 0u, 0u};
    if (ok) v = *(const u32x4*)(x + (size_t)o * 8);
    uint32_t d0, d1;
    float s;
    quantize_octet<G, MF && G == 64>(v, d0, d1, s);
    if (ok) {
        if constexpr (MF) {
            // group g, k-slot kb of the octet's quarter, row m (matrix-core
            // fragment order: quarter qi of a group sits in k-slot
            // kb = bit-swap(qi), Q bytes per fragment); written through like
            // quantize_frag64_kernel's stores
            constexpr int Q = G == 64 ? 16 : 8;
            const int opr = K / 8;
            const int m = o / opr, og = o % opr;
            const int g = og / (G / 8), k0 = (og % (G / 8)) * 8;
            const int qi = k0 / Q;
            const int kb = ((qi & 1) << 1) | (qi >> 1);
            const auto xw = buf(xq, (uint32_t)(K / G) * 64u * (uint32_t)Q);
            const auto sw = buf(xs, (uint32_t)(K / G) * 64u);
            bstore8<AUX_SC1>(xw, ((g * 4 + kb) * 16 + m) * Q + k0 % Q, u32x2{d0, d1});
            if ((o & (G / 8 - 1)) == 0) bstore4<AUX_SC1>(sw, (g * 16 + m) * 4, __float_as_uint(s));
        } else {
            *(u32x2*)(xq + (size_t)o * 8) = u32x2{d0, d1};
            if ((o & (G / 8 - 1)) == 0) xs[(size_t)o * 8 / G] = s;
        }
    }
}

// Fragment order of 64-groups, one wave per group: lane l = 16 * kb + m
// quantizes row m's quarter bit-swap(kb) of the group (16 values) and stores
// its 16-byte fragment, so a wave writes the group's 1 KB contiguously.  The
// group amax is the max over the 4 lanes of row m (lanes m, m + 16, m + 32,
// m + 48).  Rows m >= M are neither read nor written.
__global__ void __launch_bounds__(64)
quantize_frag64_kernel(const uint16_t* x, int M, int K, int8_t* __restrict__ xq, float* __restrict__ xs) {
    const int L = (int)threadIdx.x, g = (int)blockIdx.x;
    const int m = L & 15, kb = L >> 4, qi = ((kb & 1) << 1) | (kb >> 1);
    const bool ok = m < M;
    const auto xr = buf(x, (uint32_t)M * (uint32_t)K * 2u);
    const int off = ok ? (m * K + g * 64 + 16 * qi) * 2 : OOB;
    const u32x4 v0 = bload16(xr, off), v1 = bload16(xr, off + 16);
    const uint32_t wd[8] = {v0.x, v0.y, v0.z, v0.w, v1.x, v1.y, v1.z, v1.w};
    float f[16];
    float a = 0.0f;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
        f[i] = bf16f((wd[i >> 1] >> (16 * (i & 1))) & 0xffffu);
        a = fmaxf(a, fabsf(f[i]));
    }
    a = fmaxf(a, __shfl_xor(a, 16, 64));
    a = fmaxf(a, __shfl_xor(a, 32, 64));
    float s, r;
    group_scale(a, s, r);
    uint32_t t[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) t[i] = qbits(f[i], s, r);
    const u32x4 o = {bytes4(t[0], t[2], t[4], t[6]), bytes4(t[1], t[3], t[5], t[7]), bytes4(t[8], t[10], t[12], t[14]),
                     bytes4(t[9], t[11], t[13], t[15])};
    // written through (the matrix-core kernel reads them right after this
    // launch; 0.2 us of the M = 16 verify)
    const auto xw = buf(xq, (uint32_t)(K / 64) * 1024u);
    const auto sw = buf(xs, (uint32_t)(K / 64) * 64u);
    bstore16<AUX_SC1>(xw, ok ? (g * 64 + L) * 16 : OOB, o);
    bstore4<AUX_SC1>(sw, (ok && kb == 0) ? (g * 16 + m) * 4 : OOB, __float_as_uint(s));
}

// ----------------------------------------------- bf16 rounding self-check

// Every fp32 bit pattern through the kernels' conversion (f2bf2, the
// hardware v_cvt_pk_bf16_f32) and its arithmetic statement f2bf_sw; *count
// receives the number of disagreements (each thread covers a contiguous
// range of patterns, two per conversion).
constexpr int BFC_GRID = 4096, BFC_NT = 256;
__global__ void __launch_bounds__(BFC_NT) check_bf16_kernel(unsigned long long* __restrict__ count) {
    constexpr unsigned long long per = (1ull << 32) / ((unsigned long long)BFC_GRID * BFC_NT);
    const unsigned long long base = ((unsigned long long)blockIdx.x * BFC_NT + threadIdx.x) * per;
    unsigned bad = 0;
    for (unsigned long long k = 0; k < per; k += 2) {
        const float a = __uint_as_float((uint32_t)(base + k)), b = __uint_as_float((uint32_t)(base + k + 1));
        const uint32_t hw = f2bf2(a, b);
        bad += (hw & 0xffffu) != f2bf_sw(a);
        bad += (hw >> 16) != f2bf_sw(b);
    }
    if (bad) atomicAdd(count, (unsigned long long)bad);
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

static int launch_quantize(int group, const void* x, int M, int K, void* xq, void* xs, bool mf, hipStream_t st) {
    const int oct_total = M * K / 8;
    const unsigned grid = (unsigned)((oct_total + NT - 1) / NT);
    const uint16_t* a0 = (const uint16_t*)x;
    int8_t* a1 = (int8_t*)xq;
    float* a2 = (float*)xs;
    if (mf && group == 64) {
        void* fargs[] = {&a0, &M, &K, &a1, &a2};
        launch((const void*)quantize_frag64_kernel, (unsigned)(K / 64), 64, 0, st, fargs);
        return status_of(hipGetLastError());
    }
    void* args[] = {&a0, &a1, &a2, (void*)&oct_total, &K};
    const void* fn;
    if (group == 64) fn = (const void*)quantize_act_kernel<64, false>;
    else fn = mf ? (const void*)quantize_act_kernel<32, true> : (const void*)quantize_act_kernel<32, false>;
    launch(fn, grid, NT, 0, st, args);
    return status_of(hipGetLastError());
}

// M = 1 is fused when the quantized activation and its per-chunk records fit
// the LDS budget.
static bool fused_ok(int qtype, int M, int K) {
    return M == 1 && lds_m1(qtype, K) <= (size_t)LDS_MAX;
}

// Workspace of a call with M > 1 (zero-filled before its first use): the
// K split's control words and block counters at offset 0 for every shape
// (RC_CTL_BYTES: the missed-sum count, then RC_CNT_MAX counters from byte
// 256), then (long K on the matrix cores) the K split's records of part sums,
// one per row block at the same offset for every shape, then xq ([M][K], or
// fragment order with room for 16 rows) and xs ([M][K/G], or [K/G][16])
// fp32.  Offsets in bytes.
struct WsLayout {
    size_t cnt, sp, xq, xs, total;
    int blocks;  // row blocks of the K split (0: no split)
};
static size_t workspace_xq(int K) { return align16((size_t)16 * K); }
static size_t workspace_xs(int qtype, int K) { return align16((size_t)(K / group_of(qtype)) * 16 * 4); }
static size_t split_record_bytes(int blocks) { return (size_t)blocks * RC_REC_SLOTS * 8; }

static WsLayout workspace_layout(int qtype, int N, int K, int M) {
    WsLayout l{0, 0, 0, 0, 0, 0};
    const int G = group_of(qtype);
    if (G == 0 || M <= 0 || K <= 0 || N <= 0 || K % G != 0) return l;
    if (fused_ok(qtype, M, K)) return l;
    l.blocks = M >= 2 && M <= 16 ? rc_split_blocks(qtype, N, K) : 0;
    l.cnt = (size_t)RC_CTL_CNT * 4;
    l.sp = RC_CTL_BYTES;
    l.xq = l.sp + split_record_bytes(l.blocks);
    l.xs = l.xq + workspace_xq(K);
    l.total = l.xs + workspace_xs(qtype, K);
    return l;
}

// Workspace of the fragment-input entry points: the control words and, for
// long K, the K split's records (0: the launch needs none).
static size_t frag_workspace_need(int qtype, int N, int K, int M) {
    const int G = group_of(qtype);
    if (G == 0 || M < 2 || M > 16 || N <= 0 || K <= 0 || K % G != 0) return 0;
    const int blocks = rc_split_blocks(qtype, N, K);
    return blocks > 0 ? RC_CTL_BYTES + split_record_bytes(blocks) : 0;
}

static size_t workspace_need(int qtype, int N, int K, int M) { return workspace_layout(qtype, N, K, M).total; }

// Optional second matrix of the same shape applied to the same activation in
// the same launch (the reference's fused2: k and v, gate and up).
struct Second {
    const void* w = nullptr;
    const void* s = nullptr;
    void* y = nullptr;
};

static int validate_second(const Second& b, int qtype, int senc, int group, int N, int K, int M,
                           const void* res, const int32_t* part) {
    if (b.w == nullptr && b.s == nullptr && b.y == nullptr) return VIPER_OK;
    if (b.y == nullptr || res != nullptr || part != nullptr) return VIPER_INVALID_ARGUMENT;
    if (misaligned(b.y, 2)) return VIPER_INVALID_ARGUMENT;
    return validate_weights(qtype, b.w, b.s, senc, group, N, K, M);
}

static int qlinear_common(int qtype, const void* w, const void* s, int senc, int group, int N,
                          int K, const void* x, int M, void* y, const void* res, void* wsp,
                          size_t wsp_bytes, int32_t* part, void* stream, Second b = Second()) {
    int rc = validate_weights(qtype, w, s, senc, group, N, K, M);
    if (rc != VIPER_OK) return rc;
    if (x == nullptr || y == nullptr) return VIPER_INVALID_ARGUMENT;
    if (misaligned(x, 16) || misaligned(y, 2) || misaligned(res, 2) || misaligned(part, 4))
        return VIPER_INVALID_ARGUMENT;
    rc = validate_second(b, qtype, senc, group, N, K, M, res, part);
    if (rc != VIPER_OK) return rc;
    hipStream_t st = (hipStream_t)stream;
    if (fused_ok(qtype, M, K)) {
        const M1Out outs[2] = {{w, s, y, N}, {b.w, b.s, b.y, N}};
        return launch_m1(qtype, senc, K, PRO_BF16, x, nullptr, 0.0f, nullptr, outs, b.w ? 2 : 1, res, part, st);
    }
    const size_t need = workspace_need(qtype, N, K, M);
    if (wsp == nullptr || wsp_bytes < need || misaligned(wsp, 16)) return VIPER_INVALID_ARGUMENT;
    // Few rows: every workgroup quantizes the rows itself, one launch (the
    // workspace stays required for M > 1 whichever kernel runs).  Two to four
    // rows of one matrix on the M = 1 kernel's dot path; 5..8 rows (and fused
    // pairs of 3..8) on the matrix cores with the quantize into LDS
    // (north-star shape: M = 5 6.63 us, 8 7.49 us against 8.21 / 8.25 us for
    // the next-best path; at M >= 10 the rows' quantize in every workgroup
    // costs more than the quantize launch).
    const bool mf = mfma_ok(qtype, K, M, s) && (b.w == nullptr || mfma_ok(qtype, K, M, b.s));
    if (b.w == nullptr && M == 2 && m1_rows_ok(qtype, K, M)) {
        const M1Out outs[1] = {{w, s, y, N}};
        return launch_m1(qtype, senc, K, PRO_BF16, x, nullptr, 0.0f, nullptr, outs, 1, res, part, st, M);
    }
    // Long K splits over workgroups in the two-launch path (down shape
    // K = 10240, 4 rows 9.5 us against 10.3 us without the split).  (Every
    // workgroup quantizing the bf16 rows of its own part of K, in one launch,
    // measured slower at every row count: down shape 3 / 8 / 16 rows 10.4 /
    // 12.6 / 15.9 us against 8.4 / 9.4 / 9.8 us.)
    const bool split_ok = mf && b.w == nullptr && rc_split_blocks(qtype, N, K) > 0;
    // Q5/Q6/W8 (K = 2560, N = 10240, 5% outlier channels): 3 or 4 rows of one
    // matrix run faster on the multi-row dot kernel below (Q5 4 rows 7.86
    // against 8.10 us; W8 3 / 4 rows 7.47 / 7.77 against 8.9 / 9.17 us); 5-8
    // rows of every format stay on the one-launch path.
    // (Q4 rows staged two octets per thread also past that size: down shape
    // K = 10240, 4 rows 8.4 us against 9.0-9.1 us for two launches with the K
    // split)
    const bool rows_ok = b.w == nullptr && m1_rows_ok(qtype, K, M) &&
                         ((long)M * K <= 32768 || m1_rows_pair(qtype, K, M));
    // With the rows staged two octets per thread (64-groups), the one-launch
    // path also wins for Q4 at 3-4 rows (5.45 / 5.74 against 5.6 / 5.9 us on the
    // dot kernel) and 9-10 rows (6.76 / 7.00 against 7.27 us in two launches;
    // 12 and 16 rows stay two launches: 7.5 / 8.2 against 7.3 us), and for
    // Q5 / Q6 at 8 rows (7.90 / 8.22 against 8.37 / 8.58 us).  W8 keeps 3-4
    // rows on the dot kernel and 5-8 here.
    const bool q4 = qtype == VIPER_QTYPE_Q4_G64;
    const int bf_max = q4 && b.w == nullptr ? 10 : 8;
    const bool bf_ok = mf && M >= 3 && M <= bf_max && !split_ok && rc_bf16_ok(qtype, N, K, M, b.w != nullptr);
    if (bf_ok && (M > 4 || !rows_ok || q4))
        return launch_rc(qtype, w, s, senc, N, K, x, nullptr, RC_BF16, M, y, res, part, b.w, b.s, b.y, st);
    // (3 or 4 rows here also where the LDS copy does not fit: while every
    // workgroup's share of the rows' quantize stays small; down shape
    // K = 10240: 3 rows 8.8 us against about 9.5 us for two launches with the K
    // split)
    if (rows_ok) {
        const M1Out outs[1] = {{w, s, y, N}};
        return launch_m1(qtype, senc, K, PRO_BF16, x, nullptr, 0.0f, nullptr, outs, 1, res, part, st, M);
    }
    const bool staged = mf && mfma_staged(qtype, N, K);
    if (!mf && lds_pre(qtype, M, K) > (size_t)LDS_MAX) return VIPER_INVALID_ARGUMENT;
    const WsLayout lay = workspace_layout(qtype, N, K, M);
    if (split_ok && lay.blocks == 0) return VIPER_INTERNAL;
    uint8_t* xq = (uint8_t*)wsp + lay.xq;
    float* xs = (float*)((uint8_t*)wsp + lay.xs);
    // long K on the matrix cores: the K split (control words and counters at
    // the workspace's start, then the records of part sums)
    const bool split = split_ok;
    uint64_t* sp = split ? (uint64_t*)((uint8_t*)wsp + lay.sp) : nullptr;
    unsigned* sc = split ? (unsigned*)wsp : nullptr;
    rc = launch_quantize(group, x, M, K, xq, xs, staged, st);
    if (rc != VIPER_OK) return rc;
    if (mf)
        return launch_mfma(qtype, w, s, senc, N, K, xq, xs, !staged, M, y, res, part, b.w, b.s, b.y,
                           st, sp, sc);
    rc = launch_pre(qtype, w, s, senc, N, K, xq, xs, M, y, res, part, st);
    if (rc == VIPER_OK && b.w != nullptr)
        rc = launch_pre(qtype, b.w, b.s, senc, N, K, xq, xs, M, b.y, nullptr, nullptr, st);
    return rc;
}

static int prequant_common(int qtype, const void* w, const void* s, int senc, int group, int N,
                           int K, const void* xq, const void* xs, int M, void* y, const void* res,
                           void* stream, Second b = Second()) {
    int rc = validate_weights(qtype, w, s, senc, group, N, K, M);
    if (rc != VIPER_OK) return rc;
    if (xq == nullptr || xs == nullptr || y == nullptr) return VIPER_INVALID_ARGUMENT;
    if (misaligned(xq, 8) || misaligned(xs, 4) || misaligned(y, 2) || misaligned(res, 2))
        return VIPER_INVALID_ARGUMENT;
    rc = validate_second(b, qtype, senc, group, N, K, M, res, nullptr);
    if (rc != VIPER_OK) return rc;
    hipStream_t st = (hipStream_t)stream;
    if (fused_ok(qtype, M, K)) {
        const M1Out outs[2] = {{w, s, y, N}, {b.w, b.s, b.y, N}};
        return launch_m1(qtype, senc, K, PRO_INT8, xq, xs, 0.0f, nullptr, outs, b.w ? 2 : 1, res, nullptr, st);
    }
    if (b.w == nullptr && m1_rows_ok(qtype, K, M)) {
        const M1Out outs[1] = {{w, s, y, N}};
        return launch_m1(qtype, senc, K, PRO_INT8, xq, xs, 0.0f, nullptr, outs, 1, res, nullptr, st, M);
    }
    if (mfma_ok(qtype, K, M, s) && (b.w == nullptr || mfma_ok(qtype, K, M, b.s)))
        return launch_mfma(qtype, w, s, senc, N, K, xq, xs, true, M, y, res, nullptr, b.w, b.s, b.y, st);
    rc = launch_pre(qtype, w, s, senc, N, K, xq, xs, M, y, res, nullptr, st);
    if (rc == VIPER_OK && b.w != nullptr)
        rc = launch_pre(qtype, b.w, b.s, senc, N, K, xq, xs, M, b.y, nullptr, nullptr, st);
    return rc;
}

// 2..16 int8 rows already in the matrix-core fragment order (a producer's
// fragment output): one launch of the row-contiguous matrix-core kernel.  Long
// K splits over workgroups when a workspace of frag_workspace_need bytes is
// given (no launch before it: the split keeps its own counters), else runs
// the segment loop.
static int prequant_frag(int qtype, const void* w, const void* s, int senc, int group, int N, int K,
                         const void* xf, const void* xsf, int M, void* y, const void* res, void* wsp,
                         size_t wsp_bytes, void* stream, Second b = Second()) {
    int rc = validate_weights(qtype, w, s, senc, group, N, K, M);
    if (rc != VIPER_OK) return rc;
    if (xf == nullptr || xsf == nullptr || y == nullptr || M < 2 || !rc_ok(qtype, K)) return VIPER_INVALID_ARGUMENT;
    if (misaligned(xf, 16) || misaligned(xsf, 16) || misaligned(y, 2) || misaligned(res, 2))
        return VIPER_INVALID_ARGUMENT;
    rc = validate_second(b, qtype, senc, group, N, K, M, res, nullptr);
    if (rc != VIPER_OK) return rc;
    if (wsp != nullptr && misaligned(wsp, 16)) return VIPER_INVALID_ARGUMENT;
    const size_t need = b.w == nullptr ? frag_workspace_need(qtype, N, K, M) : 0;
    if (wsp != nullptr && need > 0 && wsp_bytes < need) return VIPER_INVALID_ARGUMENT;
    const bool split = wsp != nullptr && need > 0;
    uint64_t* sp = split ? (uint64_t*)((uint8_t*)wsp + RC_CTL_BYTES) : nullptr;
    unsigned* sc = split ? (unsigned*)wsp : nullptr;
    return launch_rc(qtype, w, s, senc, N, K, xf, xsf, RC_FRAG, M, y, res, nullptr, b.w, b.s, b.y,
                     (hipStream_t)stream, sp, sc);
}

}  // namespace vq

// ------------------------------------------------------------------- C ABI

extern "C" int viper_hip_abi_version(void) { return VIPER_QLINEAR_ABI_VERSION; }

extern "C" int viper_hip_group_size(int qtype) { return vq::group_of(qtype); }

extern "C" size_t viper_hip_qlinear_workspace_bytes(int qtype, int N, int K, int M) {
    return vq::workspace_need(qtype, N, K, M);
}

extern "C" size_t viper_hip_qlinear_workspace_layout(int qtype, int N, int K, int M, size_t* offsets) {
    const vq::WsLayout l = vq::workspace_layout(qtype, N, K, M);
    if (offsets != nullptr) {
        offsets[0] = l.total ? (size_t)vq::RC_CTL_MISS * 4 : SIZE_MAX;
        offsets[1] = l.total ? l.cnt : SIZE_MAX;
        offsets[2] = l.blocks ? l.sp : SIZE_MAX;
        offsets[3] = l.total ? l.xq : SIZE_MAX;
        offsets[4] = l.total ? l.xs : SIZE_MAX;
        offsets[5] = (size_t)l.blocks;
    }
    return l.total;
}

extern "C" size_t viper_hip_qlinear_frag_workspace_bytes(int qtype, int N, int K, int M) {
    return vq::frag_workspace_need(qtype, N, K, M);
}

extern "C" int viper_hip_qlinear(int qtype, const void* w_packed, const void* w_scales,
                                 int scale_enc, int group, int N, int K, const void* x_bf16, int M,
                                 void* y_bf16, const void* residual_bf16, void* workspace,
                                 size_t workspace_bytes, void* stream) {
    return vq::qlinear_common(qtype, w_packed, w_scales, scale_enc, group, N, K, x_bf16, M, y_bf16,
                              residual_bf16, workspace, workspace_bytes, nullptr, stream);
}

extern "C" int viper_hip_qlinear_static(int qtype, const void* w_packed, const void* w_scales, int scale_enc,
                                        int group, int N, int K, const void* x_bf16, int M, void* y_bf16,
                                        const void* residual_bf16, void* stream) {
    const size_t need = vq::workspace_need(qtype, N, K, M);
    if (need > vq::STATIC_SCRATCH_BYTES) return VIPER_INVALID_ARGUMENT;
    void* wsp = nullptr;
    if (need > 0) {
        const int rc = vq::scratch_address(&wsp);
        if (rc != VIPER_OK) return rc;
    }
    return vq::qlinear_common(qtype, w_packed, w_scales, scale_enc, group, N, K, x_bf16, M, y_bf16, residual_bf16,
                              wsp, need > 0 ? vq::STATIC_SCRATCH_BYTES : 0, nullptr, stream);
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
    return vq::launch_quantize(group, x_bf16, M, K, xq, xs, false, (hipStream_t)stream);
}

extern "C" int viper_hip_qlinear_prequantized(int qtype, const void* w_packed,
                                              const void* w_scales, int scale_enc, int group,
                                              int N, int K, const void* xq, const void* xs, int M,
                                              void* y_bf16, const void* residual_bf16,
                                              void* stream) {
    return vq::prequant_common(qtype, w_packed, w_scales, scale_enc, group, N, K, xq, xs, M, y_bf16,
                               residual_bf16, stream);
}

extern "C" int viper_hip_qlinear_fused2(int qtype, const void* w0_packed, const void* w0_scales,
                                        const void* w1_packed, const void* w1_scales, int scale_enc,
                                        int group, int N, int K, const void* x_bf16, int M,
                                        void* y0_bf16, void* y1_bf16, void* workspace,
                                        size_t workspace_bytes, void* stream) {
    if (w1_packed == nullptr || w1_scales == nullptr || y1_bf16 == nullptr) return VIPER_INVALID_ARGUMENT;
    return vq::qlinear_common(qtype, w0_packed, w0_scales, scale_enc, group, N, K, x_bf16, M, y0_bf16,
                              nullptr, workspace, workspace_bytes, nullptr, stream,
                              vq::Second{w1_packed, w1_scales, y1_bf16});
}

extern "C" int viper_hip_qlinear_fused2_prequantized(int qtype, const void* w0_packed,
                                                     const void* w0_scales, const void* w1_packed,
                                                     const void* w1_scales, int scale_enc, int group,
                                                     int N, int K, const void* xq, const void* xs,
                                                     int M, void* y0_bf16, void* y1_bf16,
                                                     void* stream) {
    if (w1_packed == nullptr || w1_scales == nullptr || y1_bf16 == nullptr) return VIPER_INVALID_ARGUMENT;
    return vq::prequant_common(qtype, w0_packed, w0_scales, scale_enc, group, N, K, xq, xs, M, y0_bf16,
                               nullptr, stream, vq::Second{w1_packed, w1_scales, y1_bf16});
}

extern "C" int viper_hip_qlinear_prequantized_frag(int qtype, const void* w_packed, const void* w_scales,
                                                   int scale_enc, int group, int N, int K, const void* xfrag,
                                                   const void* xsfrag, int M, void* y_bf16,
                                                   const void* residual_bf16, void* workspace, size_t workspace_bytes,
                                                   void* stream) {
    return vq::prequant_frag(qtype, w_packed, w_scales, scale_enc, group, N, K, xfrag, xsfrag, M, y_bf16,
                             residual_bf16, workspace, workspace_bytes, stream);
}

extern "C" int viper_hip_qlinear_fused2_prequantized_frag(int qtype, const void* w0_packed,
                                                          const void* w0_scales, const void* w1_packed,
                                                          const void* w1_scales, int scale_enc, int group,
                                                          int N, int K, const void* xfrag, const void* xsfrag,
                                                          int M, void* y0_bf16, void* y1_bf16, void* stream) {
    if (w1_packed == nullptr || w1_scales == nullptr || y1_bf16 == nullptr) return VIPER_INVALID_ARGUMENT;
    return vq::prequant_frag(qtype, w0_packed, w0_scales, scale_enc, group, N, K, xfrag, xsfrag, M, y0_bf16,
                             nullptr, nullptr, 0, stream, vq::Second{w1_packed, w1_scales, y1_bf16});
}

extern "C" int viper_hip_qlinear_frag_timeline(int qtype, const void* w_packed, const void* w_scales, int scale_enc,
                                               int group, int N, int K, const void* xfrag, const void* xsfrag, int M,
                                               void* y_bf16, uint64_t* stamps, size_t stamp_bytes, int* workgroups,
                                               int* waves_per_workgroup, void* workspace, size_t workspace_bytes,
                                               void* stream) {
    int rc = vq::validate_weights(qtype, w_packed, w_scales, scale_enc, group, N, K, M);
    if (rc != VIPER_OK) return rc;
    if (xfrag == nullptr || xsfrag == nullptr || y_bf16 == nullptr || vq::misaligned(xfrag, 16) ||
        vq::misaligned(xsfrag, 16) || vq::misaligned(y_bf16, 2) || vq::misaligned(stamps, 8) ||
        vq::misaligned(workspace, 16))
        return VIPER_INVALID_ARGUMENT;
    const size_t need = vq::frag_workspace_need(qtype, N, K, M);
    if (workspace != nullptr && (need == 0 || workspace_bytes < need)) return VIPER_INVALID_ARGUMENT;
    return vq::launch_rc_timeline(qtype, w_packed, w_scales, scale_enc, N, K, xfrag, xsfrag, M, y_bf16, stamps,
                                  stamp_bytes, workgroups, waves_per_workgroup, (unsigned*)workspace,
                                  (hipStream_t)stream);
}

extern "C" int viper_hip_qlinear_m1(int qtype, int scale_enc, int group, int K, int prologue, const void* a,
                                    const void* b, float eps, void* norm_out, int n_out,
                                    const void* const* w_packed, const void* const* w_scales, const int* N,
                                    void* const* y_bf16, const void* residual_bf16, void* stream) {
    if (n_out < 1 || n_out > 3 || w_packed == nullptr || w_scales == nullptr || N == nullptr || y_bf16 == nullptr)
        return VIPER_INVALID_ARGUMENT;
    if (prologue < VIPER_PROLOGUE_BF16 || prologue > VIPER_PROLOGUE_SWIGLU) return VIPER_INVALID_ARGUMENT;
    vq::M1Out outs[3];
    for (int i = 0; i < n_out; ++i) {
        const int rc = vq::validate_weights(qtype, w_packed[i], w_scales[i], scale_enc, group, N[i], K, 1);
        if (rc != VIPER_OK) return rc;
        if (y_bf16[i] == nullptr || vq::misaligned(y_bf16[i], 2)) return VIPER_INVALID_ARGUMENT;
        outs[i] = vq::M1Out{w_packed[i], w_scales[i], y_bf16[i], N[i]};
    }
    if (a == nullptr || (prologue != VIPER_PROLOGUE_BF16 && b == nullptr)) return VIPER_INVALID_ARGUMENT;
    const size_t align_a = prologue == VIPER_PROLOGUE_INT8 ? 8 : 16;
    const size_t align_b = prologue == VIPER_PROLOGUE_INT8 ? 4 : 16;
    if (vq::misaligned(a, align_a) || vq::misaligned(b, align_b) || vq::misaligned(norm_out, 16) ||
        vq::misaligned(residual_bf16, 2))
        return VIPER_INVALID_ARGUMENT;
    if (norm_out != nullptr && prologue != VIPER_PROLOGUE_RMSNORM) return VIPER_INVALID_ARGUMENT;
    if (vq::lds_m1(qtype, K) > (size_t)vq::LDS_MAX) return VIPER_INVALID_ARGUMENT;
    if ((prologue == VIPER_PROLOGUE_RMSNORM || prologue == VIPER_PROLOGUE_SWIGLU) && !vq::m1_folded_ok(qtype, K, N[0]))
        return VIPER_INVALID_ARGUMENT;
    return vq::launch_m1(qtype, scale_enc, K, prologue, a, b, eps, norm_out, outs, n_out, residual_bf16, nullptr,
                         (hipStream_t)stream);
}

extern "C" int viper_hip_qlinear_m1_swiglu(int qtype, int scale_enc, int group, int K, int prologue, const void* a,
                                           const void* b, float eps, void* norm_out, const void* w_gate,
                                           const void* s_gate, const void* w_up, const void* s_up, int N,
                                           void* h_bf16, void* gate_bf16, void* up_bf16, void* stream) {
    if (prologue != VIPER_PROLOGUE_BF16 && prologue != VIPER_PROLOGUE_RMSNORM) return VIPER_INVALID_ARGUMENT;
    int rc = vq::validate_weights(qtype, w_gate, s_gate, scale_enc, group, N, K, 1);
    if (rc != VIPER_OK) return rc;
    rc = vq::validate_weights(qtype, w_up, s_up, scale_enc, group, N, K, 1);
    if (rc != VIPER_OK) return rc;
    if (h_bf16 == nullptr || vq::misaligned(h_bf16, 2) || vq::misaligned(gate_bf16, 2) || vq::misaligned(up_bf16, 2))
        return VIPER_INVALID_ARGUMENT;
    if (a == nullptr || (prologue == VIPER_PROLOGUE_RMSNORM && b == nullptr)) return VIPER_INVALID_ARGUMENT;
    if (vq::misaligned(a, 16) || vq::misaligned(b, 16) || vq::misaligned(norm_out, 16)) return VIPER_INVALID_ARGUMENT;
    if (norm_out != nullptr && prologue != VIPER_PROLOGUE_RMSNORM) return VIPER_INVALID_ARGUMENT;
    if (vq::lds_m1(qtype, K) > (size_t)vq::LDS_MAX) return VIPER_INVALID_ARGUMENT;
    if (prologue == VIPER_PROLOGUE_RMSNORM && !vq::m1_folded_ok(qtype, K, N)) return VIPER_INVALID_ARGUMENT;
    return vq::launch_m1_swiglu(qtype, scale_enc, K, prologue, a, b, eps, norm_out, w_gate, s_gate, w_up, s_up, N,
                                h_bf16, gate_bf16, up_bf16, (hipStream_t)stream);
}

extern "C" int viper_hip_qlinear_timeline(int qtype, const void* w_packed, const void* w_scales, int scale_enc,
                                          int group, int N, int K, const void* x_bf16, void* y_bf16, uint64_t* stamps,
                                          size_t stamp_bytes, int* workgroups, int* waves_per_workgroup,
                                          void* stream) {
    const int rc = vq::validate_weights(qtype, w_packed, w_scales, scale_enc, group, N, K, 1);
    if (rc != VIPER_OK) return rc;
    if (x_bf16 == nullptr || y_bf16 == nullptr || vq::misaligned(x_bf16, 16) || vq::misaligned(y_bf16, 2) ||
        vq::misaligned(stamps, 8))
        return VIPER_INVALID_ARGUMENT;
    return vq::launch_m1_timeline(qtype, scale_enc, K, x_bf16, w_packed, w_scales, y_bf16, N, stamps, stamp_bytes,
                                  workgroups, waves_per_workgroup, (hipStream_t)stream);
}

extern "C" int viper_hip_check_bf16_rounding(unsigned long long* count, void* stream) {
    if (count == nullptr || vq::misaligned(count, 8)) return VIPER_INVALID_ARGUMENT;
    void* args[] = {&count};
    vq::launch((const void*)vq::check_bf16_kernel, vq::BFC_GRID, vq::BFC_NT, 0, (hipStream_t)stream, args);
    return vq::status_of(hipGetLastError());
}

extern "C" int viper_hip_check_quantizer(int exp_lo, int exp_hi, int32_t* counts, void* stream) {
    if (counts == nullptr || exp_lo < 0 || exp_hi > 254 || exp_lo > exp_hi)
        return VIPER_INVALID_ARGUMENT;
    if (vq::misaligned(counts, 4)) return VIPER_INVALID_ARGUMENT;
    int ab0 = exp_lo << 7;
    int32_t* c = counts;
    void* args[] = {&ab0, &c};
    const unsigned grid = (unsigned)((exp_hi - exp_lo + 1) << 7);
    vq::launch((const void*)vq::check_quantizer_kernel, grid, vq::NT, 0, (hipStream_t)stream, args);
    return vq::status_of(hipGetLastError());
}
