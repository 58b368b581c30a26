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

static m1_fn m1_kernel(int qtype, int ts, int ntt, int senc, bool part, bool exact, bool pre) {
    switch (qtype) {
        case VIPER_QTYPE_Q4_G64: return m1_pick<4>(ts, ntt, senc, part, exact, pre);
        case VIPER_QTYPE_Q5_G64: return m1_pick<5>(ts, ntt, senc, part, exact, pre);
        case VIPER_QTYPE_Q6_G64: return m1_pick<6>(ts, ntt, senc, part, exact, pre);
        default: return m1_pick<8>(ts, ntt, senc, part, exact, pre);
    }
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
        if (!m1_instantiated(ts, ntt)) continue;
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

int launch_m1(int qtype, const void* w, const void* s, int senc, int N, int K, const void* x,
              const float* xs, void* y, const void* res, int32_t* part, const void* w1,
              const void* s1, void* y1, hipStream_t st, hipEvent_t ev0, hipEvent_t ev1) {
    const int ck = qtype == VIPER_QTYPE_W8_G32 ? 16 : 32;
    const M1Shape sh = m1_shape(K / ck, N, device_cus());
    const bool exact = (K / ck) == sh.ts * M1_CPL;
    const m1_fn fn = m1_kernel(qtype, sh.ts, sh.ntt, senc, part != nullptr, exact, xs != nullptr);
    if (fn == nullptr) return VIPER_INTERNAL;
    const int rows = sh.ntt / sh.ts;
    const size_t lds = lds_m1(qtype, K);
    if (lds > (size_t)LDS_MAX) return VIPER_INVALID_ARGUMENT;
    int nb0 = (N + rows - 1) / rows;
    const unsigned grid = (unsigned)(w1 != nullptr ? 2 * nb0 : nb0);
    const uint8_t* a0 = (const uint8_t*)w;
    const uint16_t* a1 = (const uint16_t*)s;
    uint16_t* a4 = (uint16_t*)y;
    const uint16_t* a5 = (const uint16_t*)res;
    const uint8_t* b0 = (const uint8_t*)w1;
    const uint16_t* b1 = (const uint16_t*)s1;
    uint16_t* b2 = (uint16_t*)y1;
    void* args[] = {&a0, &a1, &x, &xs, &a4, &a5, &part, &N, &K, &b0, &b1, &b2, &nb0};
    launch((const void*)fn, grid, (unsigned)sh.ntt, lds, st, args, ev0, ev1);
    return status_of(hipGetLastError());
}

}  // namespace vq
