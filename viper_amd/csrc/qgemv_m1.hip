// Host side of the M = 1 GEMV: launch shape and dispatch.
#include "qgemv_m1.h"

namespace vq {

// kc: chunks per row of a masked exact tiling (M1_MASKED), else 0.
struct M1Shape {
    int ts, ntt, cpl;
    int kc = 0;
};

static m1_fn m1_kernel(int qtype, const M1Shape& sh, int senc, int mode, bool exact, int pro, int mr = 1) {
    const bool folded = pro == PRO_RMSNORM || pro == PRO_SWIGLU;
    const int ts = sh.ts, ntt = sh.ntt, cpl = sh.cpl, kc = sh.kc;
    switch (qtype) {
        case VIPER_QTYPE_Q4_G64:
            return folded ? m1_pick_folded<4>(ts, ntt, cpl, kc, senc, mode, exact, pro, mr)
                          : m1_pick_plain<4>(ts, ntt, cpl, kc, senc, mode, exact, pro, mr);
        case VIPER_QTYPE_Q5_G64:
            return folded ? m1_pick_folded<5>(ts, ntt, cpl, kc, senc, mode, exact, pro, mr)
                          : m1_pick_plain<5>(ts, ntt, cpl, kc, senc, mode, exact, pro, mr);
        case VIPER_QTYPE_Q6_G64:
            return folded ? m1_pick_folded<6>(ts, ntt, cpl, kc, senc, mode, exact, pro, mr)
                          : m1_pick_plain<6>(ts, ntt, cpl, kc, senc, mode, exact, pro, mr);
        default:
            return folded ? m1_pick_folded<8>(ts, ntt, cpl, kc, senc, mode, exact, pro, mr)
                          : m1_pick_plain<8>(ts, ntt, cpl, kc, senc, mode, exact, pro, mr);
    }
}

// A launch shape takes the exact-tiling kernels: TS * CPL chunks per row, or
// a masked tiling's chunks per row, and a row's scales in whole 16-byte words.
static bool m1_exact(const M1Shape& sh, int cpr, int ngr) {
    return (cpr == sh.ts * sh.cpl || (sh.kc != 0 && cpr == sh.kc)) && ngr % 8 == 0;
}

// Per-CU row load of a shape: ceil(ceil(N / rows) / CUs) * rows (rows per
// workgroup are halved for the swiglu pair, whose workgroups also read the
// same rows of the second matrix).
static long m1_load(const M1Shape& sh, int N, int cus, bool pair = false) {
    const long rows = pair ? sh.ntt / sh.ts / 2 : sh.ntt / sh.ts;
    const long groups = (N + rows - 1) / rows;
    return ((groups + cus - 1) / cus) * rows;
}

// Launch shape.  Exact tilings (TS * CPL == chunks per row) come first: their
// lanes need no masking and their scales arrive in one block.  Among them the
// smallest per-CU row load wins, then a workgroup that stages the activation
// row in one round (noct <= NTT: one octet per thread, a single quantize
// pass), then fewer chunk slots per lane (more lanes per row, so each lane's
// dot chain after the weights arrive is shorter), then the smaller workgroup
// (two 320-thread workgroups per CU beat one of 640 on the north-star shape:
// each quantizes and passes its barrier on its own).  With no exact tiling:
// the smallest team covering a row in 10 slots per lane (longer rows loop over
// segments of 64 lanes), workgroup size by row load, ties to more rows per
// workgroup (fewer redundant activation quantizations).
// MR > 1 rows: only the shapes m1_mr_shape_ok instantiates, with every row
// staged in M1_XS_MR rounds; there a workgroup that stages the rows in at
// most two rounds is taken first (the rows' quantize is repeated by every
// workgroup, so fewer, larger workgroups do less of it: 4 rows at K = 2560,
// 6.7 us with 640 threads against 7.4 us with 320), and the one-round
// preference does not apply (2 rows: 5.04 us with 320 threads, 5.03 us with
// 640).
static M1Shape m1_shape(int cpr, int N, int cus, int min_ntt, int noct, bool pair = false, int mr = 1) {
    M1Shape best{0, 0, 0};
    long best_load = -1;
    auto extra = [&](const M1Shape& c) { const int r = (noct + c.ntt - 1) / c.ntt; return r > 2 ? r - 2 : 0; };
    auto consider = [&](const M1Shape& c) {
        const long load = m1_load(c, N, cus, pair);
        const bool one = mr == 1 && c.ntt >= noct, best_one = mr == 1 && best.ntt >= noct;
        const int xr = extra(c), bxr = best.ntt ? extra(best) : 0;
        const bool take = best_load < 0 || load < best_load ||
                          (load == best_load &&
                           (xr < bxr ||
                            (xr == bxr &&
                             (one > best_one ||
                              (one == best_one && (c.cpl < best.cpl || (c.cpl == best.cpl && c.ntt < best.ntt)))))));
        if (take) {
            best = c;
            best_load = load;
        }
    };
    for (const auto& s : M1_SHAPES) {
        const M1Shape c{s[0], s[1], s[2]};
        if (c.ntt < min_ntt || c.ts * c.cpl != cpr || (pair && !m1_pair_ok(c.ts, c.ntt))) continue;
        if (mr > 1 && !m1_mr_shape_ok(c.ts, c.ntt, c.cpl)) continue;
        consider(c);
    }
    if (best.ntt != 0) return best;
    // masked exact tilings (one row: not the multi-row shapes), in the same order
    for (const auto& s : M1_MASKED) {
        const M1Shape c{s[0], s[1], s[2], s[3]};
        if (mr > 1 || c.kc != cpr || c.ntt < min_ntt || (pair && !m1_pair_ok(c.ts, c.ntt))) continue;
        consider(c);
    }
    if (best.ntt != 0) return best;
    int ts = 8;
    while (ts < 64 && ts * 10 < cpr) ts *= 2;
    for (const auto& s : M1_SHAPES) {
        const M1Shape c{s[0], s[1], s[2]};
        if (c.ts != ts || c.cpl != 10 || c.ntt < min_ntt || (pair && !m1_pair_ok(c.ts, c.ntt))) continue;
        if (mr > 1 && !m1_mr_shape_ok(c.ts, c.ntt, c.cpl)) continue;
        const long load = m1_load(c, N, cus, pair);
        if (best_load < 0 || load < best_load || (load == best_load && c.ntt > best.ntt)) {
            best = c;
            best_load = load;
        }
    }
    return best;
}

// The reference engine's gate / up matrices (K = 3072, N = 10752) on the
// 384-thread tiling (24 rows, 448 workgroups) load some CUs with 48 rows
// against a 42-row mean.  One Q4 / Q5 matrix there takes the 44-row
// workgroup (M1_WIDE96, 245 workgroups) when its grid still covers 95 % of
// the CUs and it lowers the per-CU rows: N = 10752 Q4 5.06-5.16 -> 4.63-4.68
// us (int8 row 4.90-4.93 -> 4.72-4.73), Q5 6.04-6.09 -> 5.87-5.90 us,
// N = 11000 Q4 5.10-5.17 -> 4.69-4.70 us.  Not for Q6 (6.41-6.49 -> 7.03-7.14
// us) nor a grid that leaves CUs idle (Q4 N = 9000, 205 workgroups:
// 4.19-4.21 -> 4.25-4.38 us).
static M1Shape m1_wide96(int qtype, int cpr, int N, int cus, const M1Shape& sh) {
    if ((qtype != VIPER_QTYPE_Q4_G64 && qtype != VIPER_QTYPE_Q5_G64) || cpr != 96 || sh.ntt == 0) return sh;
    const M1Shape c{M1_WIDE96[0], M1_WIDE96[1], M1_WIDE96[2]};
    const long rows = c.ntt / c.ts, groups = (N + rows - 1) / rows;
    if (groups * 20 < (long)cus * 19) return sh;
    return m1_load(c, N, cus) < m1_load(sh, N, cus) ? c : sh;
}

// Q5 from a bf16 row on the 16-lane tiling of K = 2560: where one 40-row
// workgroup per CU carries as many rows as two of 20, it is faster (the
// north-star shape, config 4: 4.92-4.99 -> 4.79-4.80 us); Q4 keeps two
// workgroups of 20 (their quantize and barrier run independently: 3.8
// against 3.97 us), and so do Q5 from an int8 row (4.86-4.88 against
// 5.04-5.09 us) and Q6 (equal).
static M1Shape m1_q5_bf16(int qtype, int pro, int N, int cus, const M1Shape& sh) {
    if (qtype != VIPER_QTYPE_Q5_G64 || pro != PRO_BF16 || sh.ts != 16 || sh.ntt != 320 || sh.cpl != 5) return sh;
    const M1Shape c{16, 640, 5};
    return m1_load(c, N, cus) == m1_load(sh, N, cus) ? c : sh;
}

// Upper bound over the launch shapes (an exact tiling's scale block holds at
// most NTT * CPL bytes).
size_t lds_m1(int qtype, int K) {
    constexpr int kBlockMax = 640 * 10;
    switch (qtype) {
        case VIPER_QTYPE_Q4_G64: return m1_lds_bytes<4>(K, 0) + kBlockMax;
        case VIPER_QTYPE_Q5_G64: return m1_lds_bytes<5>(K, 0) + kBlockMax;
        case VIPER_QTYPE_Q6_G64: return m1_lds_bytes<6>(K, 0) + kBlockMax;
        default: return m1_lds_bytes<8>(K, 0) + kBlockMax;
    }
}

static size_t lds_m1_launch(int qtype, int K, int rows, bool exact, int mr = 1) {
    const int r = exact ? rows : 0;
    switch (qtype) {
        case VIPER_QTYPE_Q4_G64: return m1_lds_bytes<4>(K, r, mr);
        case VIPER_QTYPE_Q5_G64: return m1_lds_bytes<5>(K, r, mr);
        case VIPER_QTYPE_Q6_G64: return m1_lds_bytes<6>(K, r, mr);
        default: return m1_lds_bytes<8>(K, r, mr);
    }
}

static int m1_mr(int M) { return M <= 1 ? 1 : (M == 2 ? 2 : 4); }

bool m1_rows_ok(int qtype, int K, int M) {
    // every row is staged in the first M1_XS_MR rounds of the workgroup, and
    // some multi-row shape tiles the row (the shape does not depend on N)
    if (M < 2 || M > 4 || (long)M * (K / 8) > (long)M1_XS_MR * 640) return false;
    const int ck = qtype == VIPER_QTYPE_W8_G32 ? 16 : 32, noct = M * (K / 8);
    const M1Shape sh = m1_shape(K / ck, 1 << 14, device_cus(), (noct + M1_XS_MR - 1) / M1_XS_MR, noct, false, m1_mr(M));
    constexpr int kBlockMax = 640 * 10;
    return sh.ntt != 0 && lds_m1_launch(qtype, K, 0, false, m1_mr(M)) + kBlockMax <= (size_t)LDS_MAX;
}

bool m1_rows_pair(int qtype, int K, int M) {
    // the multi-row shape stages its rows two octets per thread (m1_pairs)
    if (qtype != VIPER_QTYPE_Q4_G64 || !m1_rows_ok(qtype, K, M)) return false;
    const int noct = M * (K / 8);
    const M1Shape sh = m1_shape(K / 32, 1 << 14, device_cus(), (noct + M1_XS_MR - 1) / M1_XS_MR, noct, false, m1_mr(M));
    return m1_pairs<4>(m1_exact(sh, K / 32, K / 64), sh.ntt, m1_mr(M), PRO_BF16);
}

bool m1_folded_ok(int qtype, int K, int N) {
    const int ck = qtype == VIPER_QTYPE_W8_G32 ? 16 : 32;
    const int noct = K / 8;
    const M1Shape sh = m1_shape(K / ck, N, device_cus(), (noct + M1_XS - 1) / M1_XS, noct);
    return sh.ntt != 0 && lds_m1(qtype, K) <= (size_t)LDS_MAX;
}

int launch_m1(int qtype, int senc, int K, int pro, const void* x, const void* xa, float eps, void* xout,
              const M1Out* outs, int nouts, const void* res, int32_t* part, hipStream_t st, int M) {
    if (nouts < 1 || nouts > 3) return VIPER_INVALID_ARGUMENT;
    const int mr = m1_mr(M);
    if (mr > 1 && (nouts != 1 || (pro != PRO_BF16 && pro != PRO_INT8) || !m1_rows_ok(qtype, K, M)))
        return VIPER_INVALID_ARGUMENT;
    const int ck = qtype == VIPER_QTYPE_W8_G32 ? 16 : 32;
    const bool folded = pro == PRO_RMSNORM || pro == PRO_SWIGLU;
    int ntot = 0;
    for (int i = 0; i < nouts; ++i) {
        // n0's high bits carry flags
        if (outs[i].n >= M1_N_EXTRA || ntot > INT32_MAX - outs[i].n) return VIPER_INVALID_ARGUMENT;
        ntot += outs[i].n;
    }
    // The folded prologues hold the whole row after one load round, and run
    // fastest with one octet per thread (rmsnorm's row sum and swiglu's
    // element work are then a single pass): take such a workgroup when an
    // exact tiling allows it, even at a higher row load.
    const int noct = M * (K / 8);
    const int cus = device_cus();
    M1Shape sh{0, 0, 0};
    if (folded) sh = m1_shape(K / ck, ntot, cus, noct < 640 ? noct : 640, noct);
    if (sh.ntt == 0) {
        const int min_ntt = mr > 1 ? (noct + M1_XS_MR - 1) / M1_XS_MR : folded ? (noct + M1_XS - 1) / M1_XS : 0;
        sh = m1_shape(K / ck, ntot, cus, min_ntt, noct, false, mr);
    }
    if (sh.ntt == 0) return VIPER_INVALID_ARGUMENT;
    if (!folded && nouts == 1 && mr == 1) sh = m1_q5_bf16(qtype, pro, ntot, cus, m1_wide96(qtype, K / ck, ntot, cus, sh));
    const int group = qtype == VIPER_QTYPE_W8_G32 ? 32 : 64;
    const bool exact = m1_exact(sh, K / ck, K / group);
    const m1_fn fn = m1_kernel(qtype, sh, senc, part != nullptr ? M1_PART : M1_PLAIN, exact, pro, mr);
    if (fn == nullptr) return VIPER_INTERNAL;
    const int rows = sh.ntt / sh.ts;
    const size_t lds = lds_m1_launch(qtype, K, rows, exact, mr);
    if (lds > (size_t)LDS_MAX) return VIPER_INVALID_ARGUMENT;
    int nb[3] = {0, 0, 0};
    for (int i = 0; i < nouts; ++i) nb[i] = (outs[i].n + rows - 1) / rows;
    const M1Out o0 = outs[0], o1 = nouts > 1 ? outs[1] : outs[0], o2 = nouts > 2 ? outs[2] : outs[0];
    const uint8_t *w0 = (const uint8_t*)o0.w, *w1 = (const uint8_t*)o1.w, *w2 = (const uint8_t*)o2.w;
    const uint16_t *s0 = (const uint16_t*)o0.s, *s1 = (const uint16_t*)o1.s, *s2 = (const uint16_t*)o2.s;
    uint16_t *y0 = (uint16_t*)o0.y, *y1 = (uint16_t*)o1.y, *y2 = (uint16_t*)o2.y;
    int n0 = o0.n | (pro == PRO_RMSNORM && xout != nullptr ? M1_N_EXTRA : 0), n1 = o1.n, n2 = o2.n;
    int e0 = nb[0], e1 = nb[0] + nb[1];
    if (mr > 1) e1 = M;  // one matrix: e1 carries the activation rows
    const unsigned grid = (unsigned)(nb[0] + nb[1] + nb[2]);
    const uint16_t* r = (const uint16_t*)res;
    // an exact tiling's K is a kernel constant: the slot carries the grid size
    int kg = exact ? (int)grid : K;
    void* args[] = {&x, &w0, &s0, &y0, &kg, &n0, &e0, &e1, &r, &xa, &eps, &xout, &part,
                    &w1, &s1, &y1, &n1, &w2, &s2, &y2, &n2};
    launch((const void*)fn, grid, (unsigned)sh.ntt, lds, st, args);
    return status_of(hipGetLastError());
}

int launch_m1_timeline(int qtype, int senc, int K, const void* x, const void* w, const void* s, void* y, int N,
                       uint64_t* stamps, size_t stamp_bytes, int* workgroups, int* waves, hipStream_t st) {
    const int ck = qtype == VIPER_QTYPE_W8_G32 ? 16 : 32, group = qtype == VIPER_QTYPE_W8_G32 ? 32 : 64;
    const int noct = K / 8;
    const int cus = device_cus();
    const M1Shape sh = m1_q5_bf16(qtype, PRO_BF16, N, cus, m1_wide96(qtype, K / ck, N, cus, m1_shape(K / ck, N, cus, 0, noct)));  // as launch_m1
    if (sh.ntt == 0 || !m1_exact(sh, K / ck, K / group)) return VIPER_INVALID_ARGUMENT;
    const m1_fn fn = m1_kernel(qtype, sh, senc, M1_TL, true, PRO_BF16);
    if (fn == nullptr) return VIPER_INTERNAL;
    const int rows = sh.ntt / sh.ts;
    const int grid = (N + rows - 1) / rows;
    const size_t need = (size_t)grid * (sh.ntt / 64) * M1_TL_STAMPS * sizeof(uint64_t);
    if (stamps == nullptr || stamp_bytes < need) return VIPER_INVALID_ARGUMENT;
    if (workgroups != nullptr) *workgroups = grid;
    if (waves != nullptr) *waves = sh.ntt / 64;
    const size_t lds = lds_m1_launch(qtype, K, rows, true);
    const uint8_t* w0 = (const uint8_t*)w;
    const uint16_t* s0 = (const uint16_t*)s;
    uint16_t* y0 = (uint16_t*)y;
    int kg = grid, n0 = N, e0 = grid, e1 = grid, nz = 0;
    const uint16_t* r = nullptr;
    const void* xa = nullptr;
    float eps = 0.0f;
    uint16_t* xout = nullptr;
    int32_t* part = (int32_t*)stamps;
    const void* nul = nullptr;
    void* args[] = {&x, &w0, &s0, &y0, &kg, &n0, &e0, &e1, &r, &xa, &eps, &xout, &part,
                    &nul, &nul, &nul, &nz, &nul, &nul, &nul, &nz};
    launch((const void*)fn, (unsigned)grid, (unsigned)sh.ntt, lds, st, args);
    return status_of(hipGetLastError());
}

int launch_m1_swiglu(int qtype, int senc, int K, int pro, const void* x, const void* xa, float eps, void* xout,
                     const void* wg, const void* sg, const void* wu, const void* su, int N, void* h, void* g_out,
                     void* u_out, hipStream_t st) {
    if (pro != PRO_BF16 && pro != PRO_RMSNORM) return VIPER_INVALID_ARGUMENT;
    if (N >= M1_N_EXTRA) return VIPER_INVALID_ARGUMENT;  // n0's high bits carry flags
    const int ck = qtype == VIPER_QTYPE_W8_G32 ? 16 : 32;
    const int noct = K / 8;
    const int cus = device_cus();
    M1Shape sh{0, 0, 0};
    if (pro == PRO_RMSNORM) sh = m1_shape(K / ck, N, cus, noct < 640 ? noct : 640, noct, true);
    if (sh.ntt == 0) sh = m1_shape(K / ck, N, cus, pro == PRO_RMSNORM ? (noct + M1_XS - 1) / M1_XS : 0, noct, true);
    if (sh.ntt == 0) return VIPER_INVALID_ARGUMENT;
    const int group = qtype == VIPER_QTYPE_W8_G32 ? 32 : 64;
    const bool exact = m1_exact(sh, K / ck, K / group);
    const m1_fn fn = m1_kernel(qtype, sh, senc, M1_SWIGLU, exact, pro);
    if (fn == nullptr) return VIPER_INTERNAL;
    const int rows = sh.ntt / sh.ts;
    const size_t lds = lds_m1_launch(qtype, K, rows, exact);
    if (lds > (size_t)LDS_MAX) return VIPER_INVALID_ARGUMENT;
    // every workgroup is a pair of gate and up rows; the up matrix goes in the
    // residual's slot (weights) and e0 / e1 (scales), the product to y0, the
    // optional gate / up outputs to y1 / y2 (flagged in n0)
    const bool extra = g_out != nullptr || u_out != nullptr || (pro == PRO_RMSNORM && xout != nullptr);
    int n0 = N | (extra ? M1_N_EXTRA : 0), n1 = N, n2 = N;
    const unsigned grid = (unsigned)((N + rows / 2 - 1) / (rows / 2));
    const uint64_t su_bits = (uint64_t)(uintptr_t)su;
    int e0 = (int)(uint32_t)su_bits, e1 = (int)(uint32_t)(su_bits >> 32);
    const uint8_t *w0 = (const uint8_t*)wg, *w1 = nullptr, *w2 = nullptr;
    const uint16_t *s0 = (const uint16_t*)sg, *s1 = nullptr, *s2 = nullptr;
    uint16_t *y0 = (uint16_t*)h, *y1 = (uint16_t*)g_out, *y2 = (uint16_t*)u_out;
    const uint16_t* r = (const uint16_t*)wu;
    int32_t* part = nullptr;
    int kg = exact ? (int)grid : K;  // as in launch_m1
    void* args[] = {&x, &w0, &s0, &y0, &kg, &n0, &e0, &e1, &r, &xa, &eps, &xout, &part,
                    &w1, &s1, &y1, &n1, &w2, &s2, &y2, &n2};
    launch((const void*)fn, grid, (unsigned)sh.ntt, lds, st, args);
    return status_of(hipGetLastError());
}

}  // namespace vq
