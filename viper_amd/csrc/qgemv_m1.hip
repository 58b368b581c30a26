// Host side of the M = 1 GEMV: launch shape and dispatch.
#include "qgemv_m1.h"

namespace vq {

struct M1Shape {
    int ts, ntt;
};

static bool m1_instantiated(int ts, int ntt) {
    for (const auto& s : M1_SHAPES)
        if (s[0] == ts && s[1] == ntt) return true;
    return false;
}

static m1_fn m1_kernel(int qtype, int ts, int ntt, int senc, bool part, bool exact, int pro) {
    const bool folded = pro == PRO_RMSNORM || pro == PRO_SWIGLU;
    switch (qtype) {
        case VIPER_QTYPE_Q4_G64:
            return folded ? m1_pick_folded<4>(ts, ntt, senc, part, exact, pro) : m1_pick_plain<4>(ts, ntt, senc, part, exact, pro);
        case VIPER_QTYPE_Q5_G64:
            return folded ? m1_pick_folded<5>(ts, ntt, senc, part, exact, pro) : m1_pick_plain<5>(ts, ntt, senc, part, exact, pro);
        case VIPER_QTYPE_Q6_G64:
            return folded ? m1_pick_folded<6>(ts, ntt, senc, part, exact, pro) : m1_pick_plain<6>(ts, ntt, senc, part, exact, pro);
        default:
            return folded ? m1_pick_folded<8>(ts, ntt, senc, part, exact, pro) : m1_pick_plain<8>(ts, ntt, senc, part, exact, pro);
    }
}

// Team size: the smallest of 8..64 lanes covering a row in at most M1_CPL
// chunks per lane (longer rows loop over segments of 64 lanes).  Workgroup
// size: among the instantiated ones for that team, the one whose per-CU row
// load ceil(ceil(N/rows)/CUs)*rows is smallest (ties: more rows per group,
// i.e. fewer redundant activation quantizations).
static M1Shape m1_shape(int cpr, int N, int cus, int min_ntt) {
    int ts = 8;
    while (ts < 64 && ts * M1_CPL < cpr) ts *= 2;
    static const int cand[] = {128, 192, 256, 320, 640};
    M1Shape best{ts, 0};
    long best_load = -1;
    for (int ntt : cand) {
        if (!m1_instantiated(ts, ntt) || ntt < min_ntt) continue;
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

bool m1_folded_ok(int qtype, int K, int N) {
    const int ck = qtype == VIPER_QTYPE_W8_G32 ? 16 : 32;
    const int noct = K / 8;
    const M1Shape sh = m1_shape(K / ck, N, device_cus(), (noct + M1_XS - 1) / M1_XS);
    return sh.ntt != 0 && lds_m1(qtype, K) <= (size_t)LDS_MAX;
}

int launch_m1(int qtype, int senc, int K, int pro, const void* x, const void* xa, float eps, void* xout,
              const M1Out* outs, int nouts, const void* res, int32_t* part, hipStream_t st,
              hipEvent_t ev0, hipEvent_t ev1) {
    if (nouts < 1 || nouts > 3) return VIPER_INVALID_ARGUMENT;
    const int ck = qtype == VIPER_QTYPE_W8_G32 ? 16 : 32;
    const bool folded = pro == PRO_RMSNORM || pro == PRO_SWIGLU;
    int ntot = 0;
    for (int i = 0; i < nouts; ++i) ntot += outs[i].n;
    // the folded prologues hold the whole row after one load round
    const int min_ntt = folded ? (K / 8 + M1_XS - 1) / M1_XS : 0;
    const M1Shape sh = m1_shape(K / ck, ntot, device_cus(), min_ntt);
    if (sh.ntt == 0) return VIPER_INVALID_ARGUMENT;
    const bool exact = (K / ck) == sh.ts * M1_CPL;
    const m1_fn fn = m1_kernel(qtype, sh.ts, sh.ntt, senc, part != nullptr, exact, pro);
    if (fn == nullptr) return VIPER_INTERNAL;
    const int rows = sh.ntt / sh.ts;
    const size_t lds = lds_m1(qtype, K);
    if (lds > (size_t)LDS_MAX) return VIPER_INVALID_ARGUMENT;
    int nb[3] = {0, 0, 0};
    for (int i = 0; i < nouts; ++i) nb[i] = (outs[i].n + rows - 1) / rows;
    const M1Out o0 = outs[0], o1 = nouts > 1 ? outs[1] : outs[0], o2 = nouts > 2 ? outs[2] : outs[0];
    const uint8_t *w0 = (const uint8_t*)o0.w, *w1 = (const uint8_t*)o1.w, *w2 = (const uint8_t*)o2.w;
    const uint16_t *s0 = (const uint16_t*)o0.s, *s1 = (const uint16_t*)o1.s, *s2 = (const uint16_t*)o2.s;
    uint16_t *y0 = (uint16_t*)o0.y, *y1 = (uint16_t*)o1.y, *y2 = (uint16_t*)o2.y;
    int n0 = o0.n, n1 = o1.n, n2 = o2.n;
    int e0 = nb[0], e1 = nb[0] + nb[1];
    const unsigned grid = (unsigned)(nb[0] + nb[1] + nb[2]);
    const uint16_t* r = (const uint16_t*)res;
    void* args[] = {&x, &xa, &K, &e0, &e1, &w0, &s0, &y0, &n0, &eps, &xout, &r, &part,
                    &w1, &s1, &y1, &n1, &w2, &s2, &y2, &n2};
    launch((const void*)fn, grid, (unsigned)sh.ntt, lds, st, args, ev0, ev1);
    return status_of(hipGetLastError());
}

}  // namespace vq
