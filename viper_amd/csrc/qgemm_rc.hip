// Host side of the row-contiguous matrix-core kernels (M = 2..16): launch
// shape and dispatch.  The kernel template is in qgemm_rc.h.
#include "qgemm_rc.h"

namespace vq {

// Waves per workgroup and quads per wave of the single-segment shapes, in
// order of preference; longer K loops over segments of one quad per wave.
constexpr int RC_WQ[][2] = {{4, 1}, {10, 1}, {10, 2}};

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

bool rc_ok(int qtype, int K) {
    const int G = group_of(qtype);
    return G != 0 && K % (4 * G) == 0;
}

int launch_rc(int qtype, const void* w, const void* s, int senc, int N, int K, const void* xq, const void* xs,
              bool xnat, int M, void* y, const void* res, int32_t* part, const void* w1, const void* s1, void* y1,
              hipStream_t st, hipEvent_t ev0, hipEvent_t ev1) {
    if (!rc_ok(qtype, K) || M < 2 || M > 16) return VIPER_INTERNAL;
    const int NQ = K / group_of(qtype) / 4;
    const int F = qtype == VIPER_QTYPE_W8_G32 ? 8 : qtype;
    const RcShape sh = rc_shape(F, w1 != nullptr ? 2 * N : N, NQ, device_cus());
    rc_fn fn;
    int hstr;
    switch (qtype) {
        case VIPER_QTYPE_Q4_G64: fn = rc_pick<4>(sh, xnat, part != nullptr); hstr = RcFmt<4>::HSTR; break;
        case VIPER_QTYPE_Q5_G64: fn = rc_pick<5>(sh, xnat, part != nullptr); hstr = RcFmt<5>::HSTR; break;
        case VIPER_QTYPE_Q6_G64: fn = rc_pick<6>(sh, xnat, part != nullptr); hstr = RcFmt<6>::HSTR; break;
        default: fn = rc_pick<8>(sh, xnat, part != nullptr); hstr = RcFmt<8>::HSTR; break;
    }
    if (fn == nullptr) return VIPER_INTERNAL;
    int nb0 = (N + 8 * sh.rb - 1) / (8 * sh.rb);
    const unsigned grid = (unsigned)(w1 != nullptr ? 2 * nb0 : nb0);
    const size_t lds = rc_lds_bytes(hstr, sh.rb, sh.w);
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
