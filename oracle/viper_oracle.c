/*
 * CPU oracle for Viper's quantized linear path.  TEST INFRASTRUCTURE ONLY:
 * the checker for the HIP kernels, never part of the product path.  The
 * header (viper_oracle.h) lists which reference file:line each function
 * restates and the frozen bit layouts.
 *
 * Built with -ffp-contract=off so every fp32 product and sum below is
 * rounded exactly where the source says.
 */
#include "viper_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

/* ------------------------------------------------------------------ */
/* scalar conversions                                                 */
/* ------------------------------------------------------------------ */

float vo_bf16_to_f32(uint16_t h) {
    uint32_t u = (uint32_t)h << 16;
    float f;
    memcpy(&f, &u, 4);
    return f;
}

uint16_t vo_f32_to_bf16(float f) {
    uint32_t u;
    memcpy(&u, &f, 4);
    if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x0040u);
    u += 0x7fffu + ((u >> 16) & 1u);
    return (uint16_t)(u >> 16);
}

float vo_f16_to_f32(uint16_t h) {
    uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    uint32_t e = (h >> 10) & 0x1fu;
    uint32_t m = h & 0x3ffu;
    uint32_t u;
    if (e == 0) {
        if (m == 0) {
            u = sign;
        } else { /* subnormal: m * 2^-24, exact in fp32 */
            float f = (float)m * 0x1p-24f;
            memcpy(&u, &f, 4);
            u |= sign;
        }
    } else if (e == 31) {
        u = sign | 0x7f800000u | (m << 13);
    } else {
        u = sign | ((e + 112u) << 23) | (m << 13);
    }
    float f;
    memcpy(&f, &u, 4);
    return f;
}

uint16_t vo_f32_to_f16(float f) {
    uint32_t u;
    memcpy(&u, &f, 4);
    uint16_t sign = (uint16_t)((u >> 16) & 0x8000u);
    uint32_t a = u & 0x7fffffffu;
    if (a > 0x7f800000u) return (uint16_t)(sign | 0x7e00u);
    if (a >= 0x477ff000u) return (uint16_t)(sign | 0x7c00u); /* rounds to >= 65520 -> inf */
    if (a < 0x38800000u) {                                    /* below 2^-14: subnormal */
        float af;
        memcpy(&af, &a, 4);
        /* value / 2^-24, rounded to nearest even integer: exact in double */
        double q = (double)af * 16777216.0;
        double r = nearbyint(q);
        return (uint16_t)(sign | (uint16_t)r);
    }
    uint32_t e = (a >> 23) - 112u;
    uint32_t m = a & 0x7fffffu;
    uint32_t h = (e << 10) | (m >> 13);
    uint32_t rem = m & 0x1fffu;
    if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) h += 1u;
    return (uint16_t)(sign | h);
}

float vo_scale_to_f32(uint16_t s, int scale_enc) {
    return scale_enc == VO_SCALE_BF16 ? vo_bf16_to_f32(s) : vo_f16_to_f32(s);
}

static uint16_t encode_scale(float s, int scale_enc) {
    return scale_enc == VO_SCALE_BF16 ? vo_f32_to_bf16(s) : vo_f32_to_f16(s);
}

/* ------------------------------------------------------------------ */
/* format facts                                                        */
/* ------------------------------------------------------------------ */

int vo_group_size(int qtype) {
    switch (qtype) {
        case VO_Q4_G64:
        case VO_Q5_G64:
        case VO_Q6_G64: return 64;
        case VO_W8_G32: return 32;
        default: return 0;
    }
}

int vo_wmin(int qtype) {
    switch (qtype) {
        case VO_Q4_G64: return -8;
        case VO_Q5_G64: return -16;
        case VO_Q6_G64: return -32;
        case VO_W8_G32: return -127;
        default: return 0;
    }
}

int vo_wmax(int qtype) {
    switch (qtype) {
        case VO_Q4_G64: return 7;
        case VO_Q5_G64: return 15;
        case VO_Q6_G64: return 31;
        case VO_W8_G32: return 127;
        default: return 0;
    }
}

size_t vo_packed_bytes(int qtype, int64_t N, int64_t K) {
    switch (qtype) {
        case VO_Q4_G64: return (size_t)(N * K / 2);
        case VO_Q5_G64: return (size_t)(N * K / 2 + N * K / 8);
        case VO_Q6_G64: return (size_t)(N * K / 2 + N * K / 4);
        case VO_W8_G32: return (size_t)(N * K);
        default: return 0;
    }
}

static int shape_ok(int qtype, int N, int K) {
    int G = vo_group_size(qtype);
    return G > 0 && N > 0 && K > 0 && K % G == 0 && (qtype == VO_W8_G32 || K % 32 == 0);
}

/* ------------------------------------------------------------------ */
/* pack / unpack                                                       */
/* ------------------------------------------------------------------ */

/* offset-binary code of w for the nibble formats */
static int code_offset(int qtype) { return -vo_wmin(qtype); }

int vo_pack(int qtype, const int8_t* w, int N, int K, uint8_t* packed) {
    if (!shape_ok(qtype, N, K)) return -1;
    if (qtype == VO_W8_G32) {
        memcpy(packed, w, (size_t)N * (size_t)K);
        return 0;
    }
    const int off = code_offset(qtype);
    const size_t lo_bytes = (size_t)N * (size_t)K / 2;
    uint8_t* hi = packed + lo_bytes;
    for (int n = 0; n < N; ++n) {
        const int8_t* wr = w + (size_t)n * K;
        uint8_t* lo = packed + (size_t)n * (K / 2);
        for (int k = 0; k < K; k += 2) {
            unsigned u0 = (unsigned)(wr[k] + off);
            unsigned u1 = (unsigned)(wr[k + 1] + off);
            lo[k / 2] = (uint8_t)((u0 & 15u) | ((u1 & 15u) << 4));
        }
        if (qtype == VO_Q4_G64) continue;
        for (int c = 0; c < K / 32; ++c) {
            uint32_t W[2] = {0u, 0u};
            for (int i = 0; i < 4; ++i)
                for (int b = 0; b < 4; ++b)
                    for (int p = 0; p < 2; ++p) {
                        unsigned u = (unsigned)(wr[32 * c + 8 * i + 2 * b + p] + off);
                        if (qtype == VO_Q5_G64)
                            W[0] |= ((u >> 4) & 1u) << (8 * b + 2 * i + p);
                        else
                            W[i >> 1] |= ((u >> 4) & 3u) << (8 * b + 4 * (i & 1) + 2 * p);
                    }
            int nw = qtype == VO_Q5_G64 ? 1 : 2;
            uint8_t* dst = hi + ((size_t)n * (K / 32) + c) * 4 * nw;
            for (int j = 0; j < nw; ++j)
                for (int by = 0; by < 4; ++by) dst[4 * j + by] = (uint8_t)(W[j] >> (8 * by));
        }
    }
    return 0;
}

/* decode one weight (row n, column k) straight from the packed buffer */
static inline int decode_one(int qtype, const uint8_t* packed, int N, int K, int n, int k) {
    if (qtype == VO_W8_G32) return (int8_t)packed[(size_t)n * K + k];
    uint8_t byte = packed[(size_t)n * (K / 2) + k / 2];
    unsigned u = (k & 1) ? (byte >> 4) : (byte & 15u);
    if (qtype != VO_Q4_G64) {
        const uint8_t* hi = packed + (size_t)N * (K / 2);
        int c = k / 32, r = k % 32;
        int i = r / 8, b = (r % 8) / 2, p = r % 2;
        if (qtype == VO_Q5_G64) {
            const uint8_t* src = hi + ((size_t)n * (K / 32) + c) * 4;
            uint32_t W = (uint32_t)src[0] | ((uint32_t)src[1] << 8) | ((uint32_t)src[2] << 16) |
                         ((uint32_t)src[3] << 24);
            u |= ((W >> (8 * b + 2 * i + p)) & 1u) << 4;
        } else {
            const uint8_t* src = hi + ((size_t)n * (K / 32) + c) * 8 + 4 * (i >> 1);
            uint32_t W = (uint32_t)src[0] | ((uint32_t)src[1] << 8) | ((uint32_t)src[2] << 16) |
                         ((uint32_t)src[3] << 24);
            u |= ((W >> (8 * b + 4 * (i & 1) + 2 * p)) & 3u) << 4;
        }
    }
    return (int)u - code_offset(qtype);
}

int vo_unpack(int qtype, const uint8_t* packed, int N, int K, int8_t* w) {
    if (!shape_ok(qtype, N, K)) return -1;
    for (int n = 0; n < N; ++n)
        for (int k = 0; k < K; ++k) w[(size_t)n * K + k] = (int8_t)decode_one(qtype, packed, N, K, n, k);
    return 0;
}

/* ------------------------------------------------------------------ */
/* seeded generator                                                    */
/* ------------------------------------------------------------------ */

uint64_t vo_splitmix64(uint64_t* state) {
    uint64_t z = (*state += 0x9e3779b97f4a7c15ull);
    z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
    z = (z ^ (z >> 27)) * 0x94d049bb133111ebull;
    return z ^ (z >> 31);
}

uint64_t vo_substream(uint64_t seed, uint64_t stream_id) {
    uint64_t s = seed ^ (stream_id * 0xd1b54a32d192ed03ull);
    return vo_splitmix64(&s);
}

static inline double u01(uint64_t r) { return (double)(r >> 11) * 0x1p-53; }

int vo_gen_weights(int qtype, int N, int K, uint64_t seed, int scale_enc, uint8_t* packed,
                   uint16_t* scales) {
    if (!shape_ok(qtype, N, K)) return -1;
    const int G = vo_group_size(qtype);
    const int lo = vo_wmin(qtype), hi = vo_wmax(qtype);
    const uint64_t range = (uint64_t)(hi - lo + 1);
    int8_t* row = (int8_t*)malloc((size_t)K);
    if (!row) return -2;
    /* pack row by row through a one-row staging buffer (vo_pack needs the
     * full matrix for the plane formats, so pack a 1 x K matrix and place it) */
    uint8_t* rowpk = (uint8_t*)malloc(vo_packed_bytes(qtype, 1, K));
    if (!rowpk) {
        free(row);
        return -2;
    }
    uint64_t st = vo_substream(seed, 1);
    const size_t lo_row = (size_t)K / 2;
    const size_t hi_row = qtype == VO_Q5_G64 ? (size_t)K / 8 : qtype == VO_Q6_G64 ? (size_t)K / 4 : 0;
    for (int n = 0; n < N; ++n) {
        for (int k = 0; k < K; ++k) {
            uint64_t r = vo_splitmix64(&st);
            row[k] = (int8_t)(lo + (int)(((r >> 32) * range) >> 32));
        }
        vo_pack(qtype, row, 1, K, rowpk);
        if (qtype == VO_W8_G32) {
            memcpy(packed + (size_t)n * K, rowpk, (size_t)K);
        } else {
            memcpy(packed + (size_t)n * lo_row, rowpk, lo_row);
            if (hi_row)
                memcpy(packed + (size_t)N * lo_row + (size_t)n * hi_row, rowpk + lo_row, hi_row);
        }
    }
    free(rowpk);
    free(row);
    uint64_t ss = vo_substream(seed, 2);
    const double l0 = log(1e-3), span = log(10.0);
    for (size_t i = 0; i < (size_t)N * (K / G); ++i) {
        double u = u01(vo_splitmix64(&ss));
        scales[i] = encode_scale((float)exp(l0 + u * span), scale_enc);
    }
    return 0;
}

void vo_gen_act(int M, int K, uint64_t seed, double outlier_frac, float outlier_mul,
                uint16_t* x) {
    uint64_t st = vo_substream(seed, 3);
    const size_t total = (size_t)M * (size_t)K;
    const double two_pi = 6.283185307179586476925286766559;
    for (size_t i = 0; i < total; i += 2) {
        double u1 = ((double)(vo_splitmix64(&st) >> 11) + 1.0) * 0x1p-53; /* (0, 1] */
        double u2 = u01(vo_splitmix64(&st));
        double rad = sqrt(-2.0 * log(u1));
        float z0 = (float)(rad * cos(two_pi * u2));
        float z1 = (float)(rad * sin(two_pi * u2));
        for (int j = 0; j < 2 && i + j < total; ++j) {
            float z = j ? z1 : z0;
            int k = (int)((i + j) % (size_t)K);
            if (outlier_frac > 0.0 && u01(vo_substream(seed ^ 0x071e5ull, (uint64_t)k)) < outlier_frac)
                z *= outlier_mul;
            x[i + j] = vo_f32_to_bf16(z);
        }
    }
}

/* ------------------------------------------------------------------ */
/* offline weight quantizer                                            */
/* ------------------------------------------------------------------ */

int vo_quantize_weights(int qtype, const uint16_t* w_bf16, int N, int K, int scale_enc,
                        uint8_t* packed, uint16_t* scales) {
    if (!shape_ok(qtype, N, K)) return -1;
    const int G = vo_group_size(qtype);
    const int wmin = vo_wmin(qtype), wmax = vo_wmax(qtype);
    /* divisor: the positive end of the code range (7 for Q4, as the converter) */
    const float qdiv = (float)wmax;
    int8_t* w = (int8_t*)malloc((size_t)N * (size_t)K);
    if (!w) return -2;
    for (int n = 0; n < N; ++n) {
        for (int g = 0; g < K / G; ++g) {
            const uint16_t* src = w_bf16 + (size_t)n * K + (size_t)g * G;
            float max_abs = 0.0f;
            for (int j = 0; j < G; ++j) {
                float v = fabsf(vo_bf16_to_f32(src[j]));
                if (v > max_abs) max_abs = v;
            }
            float scale = max_abs / qdiv;
            if (scale < 1e-8f) scale = 1e-8f;
            if (scale_enc == VO_SCALE_BF16) {
                uint32_t su;
                memcpy(&su, &scale, 4);
                scales[(size_t)n * (K / G) + g] = (uint16_t)(su >> 16); /* truncation */
            } else {
                scales[(size_t)n * (K / G) + g] = vo_f32_to_f16(scale);
            }
            for (int j = 0; j < G; ++j) {
                float v = vo_bf16_to_f32(src[j]);
                int q = (int)roundf(v / scale);
                if (q < wmin) q = wmin;
                if (q > wmax) q = wmax;
                w[(size_t)n * K + (size_t)g * G + j] = (int8_t)q;
            }
        }
    }
    int rc = vo_pack(qtype, w, N, K, packed);
    free(w);
    return rc;
}

/* ------------------------------------------------------------------ */
/* activation quantize                                                 */
/* ------------------------------------------------------------------ */

int vo_quantize_act(const uint16_t* x, int M, int K, int group, int8_t* xq, float* xs) {
    if (M <= 0 || K <= 0 || group <= 0 || K % group) return -1;
    const int ng = K / group;
    for (int m = 0; m < M; ++m) {
        for (int g = 0; g < ng; ++g) {
            const uint16_t* src = x + (size_t)m * K + (size_t)g * group;
            float amax = 0.0f;
            for (int j = 0; j < group; ++j) amax = fmaxf(amax, fabsf(vo_bf16_to_f32(src[j])));
            float scale = fmaxf(amax / 127.0f, 1e-8f);
            xs[(size_t)m * ng + g] = scale;
            for (int j = 0; j < group; ++j) {
                float q = rintf(vo_bf16_to_f32(src[j]) / scale);
                if (!(q == q)) q = 0.0f;
                if (q > 127.0f) q = 127.0f;
                if (q < -127.0f) q = -127.0f;
                xq[(size_t)m * K + (size_t)g * group + j] = (int8_t)q;
            }
        }
    }
    return 0;
}

/* ------------------------------------------------------------------ */
/* producers of the activation: rmsnorm and swiglu (before the quantize) */
/* ------------------------------------------------------------------ */

int vo_rmsnorm_bf16(const uint16_t* x, const uint16_t* gamma, float eps, int M, int H, uint16_t* out) {
    if (M <= 0 || H <= 0) return -1;
    for (int m = 0; m < M; ++m) {
        const uint16_t* xr = x + (size_t)m * H;
        double ss = 0.0;
        for (int i = 0; i < H; ++i) {
            const double v = vo_bf16_to_f32(xr[i]);
            ss += v * v;
        }
        const float t = (float)ss / (float)H + eps;
        const float inv = (float)(1.0 / sqrt((double)t));
        for (int i = 0; i < H; ++i) {
            const float v = (vo_bf16_to_f32(xr[i]) * inv) * vo_bf16_to_f32(gamma[i]);
            out[(size_t)m * H + i] = vo_f32_to_bf16(v);
        }
    }
    return 0;
}

int vo_swiglu_bf16(const uint16_t* gate, const uint16_t* up, int M, int I, uint16_t* out) {
    if (M <= 0 || I <= 0) return -1;
    for (size_t i = 0; i < (size_t)M * I; ++i) {
        const float g = vo_bf16_to_f32(gate[i]), u = vo_bf16_to_f32(up[i]);
        const float v = g / (1.0f + expf(-g)) * u;
        out[i] = vo_f32_to_bf16(v);
    }
    return 0;
}

/* ------------------------------------------------------------------ */
/* bf16 GEMV (LM head) and greedy argmax                               */
/* ------------------------------------------------------------------ */

int vo_linear_bf16(const uint16_t* w, const uint16_t* x, int M, int N, int K, uint16_t* y,
                   float* y_f32, double* absterm) {
    if (M <= 0 || N <= 0 || K <= 0) return -1;
#ifdef _OPENMP
#pragma omp parallel for schedule(static)
#endif
    for (int n = 0; n < N; ++n) {
        const uint16_t* wr = w + (size_t)n * K;
        for (int m = 0; m < M; ++m) {
            const uint16_t* xr = x + (size_t)m * K;
            double s = 0.0, a = 0.0;
            for (int k = 0; k < K; ++k) {
                const double p = (double)vo_bf16_to_f32(wr[k]) * (double)vo_bf16_to_f32(xr[k]);
                s += p;
                a += fabs(p);
            }
            const size_t o = (size_t)m * N + n;
            y[o] = vo_f32_to_bf16((float)s);
            if (y_f32) y_f32[o] = (float)s;
            if (absterm) absterm[o] = a;
        }
    }
    return 0;
}

int vo_argmax_bf16(const uint16_t* logits, int B, int V, int32_t* out) {
    if (B <= 0 || V <= 0) return -1;
    for (int b = 0; b < B; ++b) {
        float best = -INFINITY;
        int32_t idx = 0;
        for (int v = 0; v < V; ++v) {
            const float f = vo_bf16_to_f32(logits[(size_t)b * V + v]);
            if (f > best) {  /* strict: the first occurrence wins, NaN never */
                best = f;
                idx = v;
            }
        }
        out[b] = idx;
    }
    return 0;
}

/* ------------------------------------------------------------------ */
/* exact group dots                                                    */
/* ------------------------------------------------------------------ */

static int32_t group_dot(int qtype, const uint8_t* packed, int N, int K, int n, int g,
                         const int8_t* q /* xq row + g*G */) {
    int32_t s = 0;
    if (qtype == VO_Q4_G64) {
        const uint8_t* b = packed + (size_t)n * (K / 2) + (size_t)g * 32;
        for (int j = 0; j < 32; ++j) {
            s += ((int)(b[j] & 15u) - 8) * q[2 * j];
            s += ((int)(b[j] >> 4) - 8) * q[2 * j + 1];
        }
        return s;
    }
    if (qtype == VO_W8_G32) {
        const int8_t* b = (const int8_t*)packed + (size_t)n * K + (size_t)g * 32;
        for (int j = 0; j < 32; ++j) s += b[j] * q[j];
        return s;
    }
    const int G = 64;
    for (int j = 0; j < G; ++j) s += decode_one(qtype, packed, N, K, n, g * G + j) * q[j];
    return s;
}

int vo_group_dots(int qtype, const uint8_t* packed, int N, int K, const int8_t* xq, int M,
                  int32_t* D) {
    if (!shape_ok(qtype, N, K) || M <= 0) return -1;
    const int G = vo_group_size(qtype), ng = K / G;
    for (int m = 0; m < M; ++m)
        for (int n = 0; n < N; ++n)
            for (int g = 0; g < ng; ++g)
                D[((size_t)m * N + n) * ng + g] =
                    group_dot(qtype, packed, N, K, n, g, xq + (size_t)m * K + (size_t)g * G);
    return 0;
}

/* ------------------------------------------------------------------ */
/* full linear                                                         */
/* ------------------------------------------------------------------ */

static void linear_row(int qtype, const uint8_t* packed, const uint16_t* scales, int scale_enc,
                       int N, int K, const int8_t* xq, const float* xs, int m, int n,
                       const uint16_t* residual, uint16_t* y, float* y_f32, double* y_absterm) {
    const int G = vo_group_size(qtype), ng = K / G;
    float acc = 0.0f;
    double absterm = 0.0;
    for (int g = 0; g < ng; ++g) {
        int32_t d = group_dot(qtype, packed, N, K, n, g, xq + (size_t)m * K + (size_t)g * G);
        float f = vo_scale_to_f32(scales[(size_t)n * ng + g], scale_enc) * xs[(size_t)m * ng + g];
        float t = f * (float)d;
        acc += t;
        absterm += fabs((double)t);
    }
    if (residual) {
        float r = vo_bf16_to_f32(residual[(size_t)m * N + n]);
        acc += r;
        absterm += fabs((double)r);
    }
    y[(size_t)m * N + n] = vo_f32_to_bf16(acc);
    if (y_f32) y_f32[(size_t)m * N + n] = acc;
    if (y_absterm) y_absterm[(size_t)m * N + n] = absterm;
}

int vo_qlinear_prequant(int qtype, const uint8_t* packed, const uint16_t* scales, int scale_enc,
                        int N, int K, const int8_t* xq, const float* xs, int M,
                        const uint16_t* residual, uint16_t* y, float* y_f32, double* y_absterm) {
    if (!shape_ok(qtype, N, K) || M <= 0) return -1;
    for (int m = 0; m < M; ++m)
        for (int n = 0; n < N; ++n)
            linear_row(qtype, packed, scales, scale_enc, N, K, xq, xs, m, n, residual, y, y_f32,
                       y_absterm);
    return 0;
}

int vo_qlinear(int qtype, const uint8_t* packed, const uint16_t* scales, int scale_enc, int N,
               int K, const uint16_t* x, int M, const uint16_t* residual, uint16_t* y,
               float* y_f32, double* y_absterm) {
    if (!shape_ok(qtype, N, K) || M <= 0) return -1;
    const int G = vo_group_size(qtype);
    int8_t* xq = (int8_t*)malloc((size_t)M * K);
    float* xs = (float*)malloc(sizeof(float) * (size_t)M * (K / G));
    int rc = -2;
    if (xq && xs) {
        vo_quantize_act(x, M, K, G, xq, xs);
        rc = vo_qlinear_prequant(qtype, packed, scales, scale_enc, N, K, xq, xs, M, residual, y,
                                 y_f32, y_absterm);
    }
    free(xq);
    free(xs);
    return rc;
}

int vo_omp_max_threads(void) {
#ifdef _OPENMP
    return omp_get_max_threads();
#else
    return 1;
#endif
}

int vo_qlinear_omp(int qtype, const uint8_t* packed, const uint16_t* scales, int scale_enc,
                   int N, int K, const uint16_t* x, int M, const uint16_t* residual, uint16_t* y,
                   float* y_f32, double* y_absterm, int nthreads) {
    if (!shape_ok(qtype, N, K) || M <= 0) return -1;
    const int G = vo_group_size(qtype);
    int8_t* xq = (int8_t*)malloc((size_t)M * K);
    float* xs = (float*)malloc(sizeof(float) * (size_t)M * (K / G));
    if (!xq || !xs) {
        free(xq);
        free(xs);
        return -2;
    }
    vo_quantize_act(x, M, K, G, xq, xs);
#ifdef _OPENMP
    if (nthreads <= 0) nthreads = omp_get_max_threads();
#pragma omp parallel for num_threads(nthreads) schedule(static)
#endif
    for (int n = 0; n < N; ++n)
        for (int m = 0; m < M; ++m)
            linear_row(qtype, packed, scales, scale_enc, N, K, xq, xs, m, n, residual, y, y_f32,
                       y_absterm);
    (void)nthreads;
    free(xq);
    free(xs);
    return 0;
}

/* ------------------------------------------------------------------ */
/* exhaustive check of the exact-division identity                     */
/* ------------------------------------------------------------------ */

int64_t vo_check_markstein(int exp_lo, int exp_hi, int64_t* n_checked) {
    int64_t bad = 0, total = 0;
    if (exp_lo < 0) exp_lo = 0;
    if (exp_hi > 254) exp_hi = 254;
#ifdef _OPENMP
#pragma omp parallel for reduction(+ : bad, total) schedule(dynamic, 1)
#endif
    for (int ab = exp_lo << 7; ab < ((exp_hi + 1) << 7); ++ab) {
        const float amax = vo_bf16_to_f32((uint16_t)ab);
        const float s = fmaxf(amax / 127.0f, 1e-8f);
        const float r = 1.0f / s;
        for (int xb = 0; xb <= ab; ++xb) {
            const float x = vo_bf16_to_f32((uint16_t)xb);
            const float exact = x / s;
            const float q0 = x * r;
            const float e = fmaf(-q0, s, x);
            const float q1 = fmaf(e, r, q0);
            /* the quotient itself may differ by an ulp; the quantized
             * integer is the claim */
            bad += (rintf(q1) != rintf(exact));
            ++total;
        }
    }
    if (n_checked) *n_checked = total;
    return bad;
}
