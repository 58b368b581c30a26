// Host side of the row-contiguous matrix-core kernels (M = 2..16): launch
// shape and dispatch.  The kernel template is in qgemm_rc.h.
#include "qgemm_rc.h"

#include <map>
#include <mutex>

namespace vq {

// Waves per workgroup and quads per wave of the single-segment shapes, in
// order of preference; longer K loops over segments of one quad per wave.
// (12 waves of one quad: the reference engine's K = 3072, whose 12 quads on
// 10 waves of two left two waves with twice the work and, at N = 10752, the
// two-quad kernel's registers one workgroup per CU for 336 workgroups.)
constexpr int RC_WQ[][2] = {{4, 1}, {10, 1}, {12, 1}, {10, 2}};

// Rows per workgroup: the multiple of 8 that spreads all rows (both matrices
// of a fused pair) over one workgroup per CU, at most 48 (fewer with two
// quads per wave or the segment loop, whose registers hold fewer blocks);
// then the fewest waves whose quads cover K in one segment, else the loop.
static RcShape rc_shape(int F, int rows_total, int NQ, int cus) {
    RcShape s{0, 0, 0, true};
    const int rb = (rows_total + 8 * cus - 1) / (8 * cus);
    s.rb = rb < 1 ? 1 : (rb > 6 ? 6 : rb);
    for (const auto& c : RC_WQ)
        if (c[0] * c[1] >= NQ) {
            s.w = c[0];
            s.qw = c[1];
            break;
        }
    if (s.w == 0) {
        s.w = 10;
        s.qw = 1;
        s.one = false;
    }
    if (s.qw > 1 && s.rb > rc_rb_qw2(F)) s.rb = rc_rb_qw2(F);
    if (!s.one && s.rb > RC_RB_LOOP) s.rb = RC_RB_LOOP;
    return s;
}

// K split (fragment input): K whose unsplit shape is the segment loop, in
// sk parts that each fit one segment of 10 waves: the fewest parts of at most
// 10 quads (one per wave; K = 10240: 4 parts, K = 6144: 3 parts of 8 quads,
// 6.7 us at M = 16 and N = 3072 against 7.3 us for 4 parts of 6), else of at
// most 20 (two per wave).  Rows per workgroup spread the sk * N (row, part)
// pairs over two workgroups per CU where the kernel fits two (down shape
// K = 10240, N = 2560: 107 blocks of 24 rows x 4 parts instead of 160 blocks
// of 16 rows that each read all of K's activation, M = 4 / 8 / 16: 9.47 /
// 9.45 / 9.87 us; 40 rows, one workgroup per CU: 9.9 / 9.8 / 10.0 us; 16 rows
// 11.3 / 11.6 / 11.9 us).
static int rc_split_parts(int NQ) {
    if (NQ <= 20) return 0;
    for (int lim : {10, 20})
        for (int sk = 2; sk <= RC_SK_MAX; ++sk)
            if (NQ % sk == 0 && NQ / sk <= lim) return sk;
    return 0;
}

// Registers a kernel takes per lane (0 where the device cannot be asked),
// cached per kernel.
static int rc_regs(rc_fn fn) {
    static std::mutex mu;
    static std::map<const void*, int> cache;
    std::lock_guard<std::mutex> lock(mu);
    const auto it = cache.find((const void*)fn);
    if (it != cache.end()) return it->second;
    hipFuncAttributes a{};
    if (hipFuncGetAttributes(&a, (const void*)fn) != hipSuccess) {
        (void)hipGetLastError();
        return 0;
    }
    cache[(const void*)fn] = a.numRegs;
    return a.numRegs;
}

// A split pays only where two workgroups of ten waves sit on a CU with room
// to spare: at most 80 registers, six waves per SIMD (forced shapes, M = 16,
// fragment input, one box: Q4 24-row blocks, 72 registers: K = 10240 7.6
// against 8.5 us on the segment loop, K = 6144 6.7 against 7.4; W8 40-row
// blocks, 68: K = 10240 11.1 against 13.6; Q4 32- and 40-row blocks, 84 and
// 96 registers: K = 8960 10.6 against 7.9, K = 12288 11.9 against 10.3,
// K = 10752 13.5 against 10.1; Q5 24-row blocks, 84: K = 10240 11.7 against
// 10.1).  Without a device to ask, the split is assumed to fit.
constexpr int RC_SPLIT_MAX_REGS = 80;

static bool rc_split_shape(int qtype, int rows, int K, int cus, RcShape& s) {
    const int F = qtype == VIPER_QTYPE_W8_G32 ? 8 : qtype, NQ = K / group_of(qtype) / 4;
    const int sk = rc_split_parts(NQ);
    if (sk == 0) return false;
    s.w = 10;
    s.one = true;
    s.qw = NQ / sk <= 10 ? 1 : 2;
    s.sk = sk;
    const int rb = (sk * rows + 16 * cus - 1) / (16 * cus), rbmax = s.qw == 2 ? rc_rb_qw2(F) : 6;
    s.rb = rb < 1 ? 1 : (rb > rbmax ? rbmax : rb);
    if ((rows + 8 * s.rb - 1) / (8 * s.rb) > RC_CNT_MAX) return false;
    rc_fn fn;
    switch (F) {
        case 4: fn = rc_pick<4>(s, RC_FRAG, false, 0, false); break;
        case 5: fn = rc_pick<5>(s, RC_FRAG, false, 0, false); break;
        case 6: fn = rc_pick<6>(s, RC_FRAG, false, 0, false); break;
        default: fn = rc_pick<8>(s, RC_FRAG, false, 0, false); break;
    }
    return fn != nullptr && rc_regs(fn) <= RC_SPLIT_MAX_REGS;
}

int rc_split_blocks(int qtype, int N, int K) {
    const int G = group_of(qtype);
    if (G == 0 || K % (4 * G) != 0 || K >= (1 << 27)) return 0;
    RcShape s{0, 0, 0, true};
    if (!rc_split_shape(qtype, N, K, device_cus(), s)) return 0;
    return (N + 8 * s.rb - 1) / (8 * s.rb);
}

bool rc_ok(int qtype, int K) {
    const int G = group_of(qtype);
    return G != 0 && K % (4 * G) == 0;
}

static int rc_hstr(int qtype) {
    switch (qtype) {
        case VIPER_QTYPE_Q5_G64: return RcFmt<5>::HSTR;
        case VIPER_QTYPE_Q6_G64: return RcFmt<6>::HSTR;
        default: return 0;
    }
}

// LDS bytes of a launch (RC_BF16 adds the workgroup's copy of the fragments).
static size_t rc_launch_lds(int qtype, const RcShape& sh, int K, int am) {
    const int qb = qtype == VIPER_QTYPE_W8_G32 ? RcFmt<8>::QB : RcFmt<4>::QB;
    const bool staged = sh.one && (am == RC_FRAG || am == RC_BF16) && rc_hstr(qtype) == 0;  // the kernel's staged scales
    const int ngp = K / group_of(qtype) / sh.sk;  // groups of the workgroup's part
    return rc_lds_bytes(rc_hstr(qtype), sh.rb, sh.w) + (am == RC_BF16 ? rc_act_lds_bytes(qb, ngp) : 0) +
           (staged ? rc_stage_bytes(sh.rb, ngp / 4) : 0);
}

static RcShape rc_launch_shape(int qtype, int rows_total, int K) {
    const int F = qtype == VIPER_QTYPE_W8_G32 ? 8 : qtype;
    return rc_shape(F, rows_total, K / group_of(qtype) / 4, device_cus());
}

// RC_BF16: every row's octets in RC_XR rounds of the workgroup, and the
// fragments fit LDS beside the kernel's own buffers.
bool rc_bf16_ok(int qtype, int N, int K, int M, bool pair) {
    if (!rc_ok(qtype, K) || M < 2 || M > 16) return false;
    const RcShape sh = rc_launch_shape(qtype, pair ? 2 * N : N, K);
    if ((long)M * (K / 8) > (long)RC_XR * 64 * sh.w) return false;
    return rc_launch_lds(qtype, sh, K, RC_BF16) <= (size_t)device_lds_max();
}

int launch_rc(int qtype, const void* w, const void* s, int senc, int N, int K, const void* xq, const void* xs,
              int am, int M, void* y, const void* res, int32_t* part, const void* w1, const void* s1, void* y1,
              hipStream_t st, uint64_t* sp, unsigned* sc) {
    if (!rc_ok(qtype, K) || M < 2 || M > 16) return VIPER_INTERNAL;
    if (N >= (1 << 27)) return VIPER_INVALID_ARGUMENT;  // N shares a word with M and the encoding
    if (am == RC_BF16 && !rc_bf16_ok(qtype, N, K, M, w1 != nullptr)) return VIPER_INTERNAL;
    RcShape sh = rc_launch_shape(qtype, w1 != nullptr ? 2 * N : N, K);
    if (sp != nullptr) {
        if (am != RC_FRAG || w1 != nullptr || sc == nullptr || K >= (1 << 27) ||
            !rc_split_shape(qtype, N, K, device_cus(), sh))
            return VIPER_INTERNAL;
    }
    rc_fn fn;
    switch (qtype) {
        case VIPER_QTYPE_Q4_G64: fn = rc_pick<4>(sh, am, part != nullptr, senc, w1 != nullptr); break;
        case VIPER_QTYPE_Q5_G64: fn = rc_pick<5>(sh, am, part != nullptr, senc, w1 != nullptr); break;
        case VIPER_QTYPE_Q6_G64: fn = rc_pick<6>(sh, am, part != nullptr, senc, w1 != nullptr); break;
        default: fn = rc_pick<8>(sh, am, part != nullptr, senc, w1 != nullptr); break;
    }
    if (fn == nullptr) return VIPER_INTERNAL;
    int nb0 = (N + 8 * sh.rb - 1) / (8 * sh.rb);
    const unsigned grid = (unsigned)(w1 != nullptr ? 2 * nb0 : nb0 * sh.sk);
    if (sh.sk > 1 && nb0 > RC_CNT_MAX) return VIPER_INTERNAL;
    const size_t lds = rc_launch_lds(qtype, sh, K, am);
    const int8_t* a0 = (const int8_t*)xq;
    const float* a1 = (const float*)xs;
    const uint8_t* a2 = (const uint8_t*)w;
    const uint16_t* a3 = (const uint16_t*)s;
    uint16_t* a4 = (uint16_t*)y;
    const uint16_t* a5 = (const uint16_t*)res;
    const uint8_t* b0 = (const uint8_t*)w1;
    const uint16_t* b1 = (const uint16_t*)s1;
    uint16_t* b2 = (uint16_t*)y1;
    unsigned nm = (unsigned)N | ((unsigned)(M - 1) << 27) | (senc ? 1u << 31 : 0u);  // see the kernel's arguments note
    unsigned kk = (unsigned)K | (sh.sk > 1 ? (unsigned)sh.sk << 27 : 0u);
    void* args[] = {&a0, &a1, &a2, &a3, &a4, &kk, &nm, &sc, &a5, &part, &b0, &b1, &b2};
    launch((const void*)fn, grid, (unsigned)(64 * sh.w), lds, st, args);
    return status_of(hipGetLastError());
}

// The timeline variant of launch_rc (Q4 or W8, fragment input, one segment, or the
// K split when sc is given): see viper_hip_qlinear_frag_timeline.
int launch_rc_timeline(int qtype, const void* w, const void* s, int senc, int N, int K, const void* xq,
                       const void* xs, int M, void* y, uint64_t* stamps, size_t stamp_bytes, int* workgroups,
                       int* waves, unsigned* sc, hipStream_t st) {
    if ((qtype != VIPER_QTYPE_Q4_G64 && qtype != VIPER_QTYPE_W8_G32) || !rc_ok(qtype, K) || M < 2 || M > 16 ||
        N >= (1 << 27))
        return VIPER_INVALID_ARGUMENT;
    RcShape sh = rc_launch_shape(qtype, N, K);
    if (sc != nullptr && (K >= (1 << 27) || !rc_split_shape(qtype, N, K, device_cus(), sh))) return VIPER_INVALID_ARGUMENT;
    const rc_fn fn = qtype == VIPER_QTYPE_W8_G32 ? rc_pick_tl8(sh, senc) : rc_pick_tl4(sh, senc);
    if (fn == nullptr) return VIPER_INVALID_ARGUMENT;
    const int nb0 = (N + 8 * sh.rb - 1) / (8 * sh.rb), grid = nb0 * sh.sk;
    if (sh.sk > 1 && nb0 > RC_CNT_MAX) return VIPER_INVALID_ARGUMENT;
    if (stamps == nullptr || stamp_bytes < (size_t)grid * sh.w * RC_TL_STAMPS * sizeof(uint64_t)) return VIPER_INVALID_ARGUMENT;
    if (workgroups != nullptr) *workgroups = grid;
    if (waves != nullptr) *waves = sh.w;
    const size_t lds = rc_launch_lds(qtype, sh, K, RC_FRAG);
    const int8_t* a0 = (const int8_t*)xq;
    const float* a1 = (const float*)xs;
    const uint8_t* a2 = (const uint8_t*)w;
    const uint16_t* a3 = (const uint16_t*)s;
    uint16_t* a4 = (uint16_t*)y;
    const uint16_t* a5 = nullptr;
    int32_t* part = (int32_t*)stamps;
    const uint8_t* b0 = nullptr;
    const uint16_t* b1 = nullptr;
    uint16_t* b2 = nullptr;
    unsigned nm = (unsigned)N | ((unsigned)(M - 1) << 27) | (senc ? 1u << 31 : 0u);
    unsigned kk = (unsigned)K | (sh.sk > 1 ? (unsigned)sh.sk << 27 : 0u);
    void* args[] = {&a0, &a1, &a2, &a3, &a4, &kk, &nm, &sc, &a5, &part, &b0, &b1, &b2};
    launch((const void*)fn, (unsigned)grid, (unsigned)(64 * sh.w), lds, st, args);
    return status_of(hipGetLastError());
}

}  // namespace vq
