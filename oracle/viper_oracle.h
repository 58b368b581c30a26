/*
 * CPU oracle for Viper's quantized linear path.  TEST INFRASTRUCTURE ONLY.
 *
 * This is a plain-C restatement of the reference's format and arithmetic
 * semantics, used as the checker for the HIP kernels.  Only tests/,
 * __graft_entry__.smoke() and bench.py's cpu_baseline leg may load it; the
 * product library (viper_amd/) never links or calls it.
 *
 * What each function restates (reference = itzrnvr/viper):
 *   vo_quantize_weights   tools/convert/convert.cpp:91-127 (Q4_G64: scale =
 *                         max|w|/7 floored at 1e-8, bf16 by truncation,
 *                         stored = clamp(round_half_away(w/scale)+8, 0, 15),
 *                         even k in the low nibble).  Q5/Q6/W8 generalise it.
 *   vo_quantize_act       kernels/ops/rmsnorm_quantize.cu:71-104,
 *                         swiglu_quantize.cu:45-78, linear_multim.cu:21-61:
 *                         per-row, per-group amax; scale = max(amax/127, 1e-8);
 *                         q = RNE(x / scale) with an IEEE divide; clamp +-127.
 *   vo_rmsnorm_bf16       kernels/ops/rmsnorm_quantize.cu:37-73 (phases 1-3):
 *                         inv = 1/sqrt(ss/H + eps) with ss = sum x^2, then
 *                         bf16_RNE((x * inv) * gamma) in fp32.  ss is summed in
 *                         double and rounded to fp32 once, and the square root
 *                         is exact; the reference sums in fp32 in a thread
 *                         order and uses rsqrtf, so outputs agree to 1 bf16 ulp.
 *   vo_swiglu_bf16        kernels/ops/swiglu_quantize.cu:35-41 (phase 1):
 *                         bf16_RNE(g / (1 + exp(-g)) * u) in fp32 with the libm
 *                         exp (the reference uses __expf; 1 bf16 ulp).
 *                         The quantize step after both is vo_quantize_act
 *                         (rmsnorm_quantize.cu:75-104, swiglu_quantize.cu:45-78).
 *   vo_linear_bf16        kernels/ops/linear_bf16_kernel.cu:15-54: y[m][n] =
 *                         bf16_RNE(sum_k f32(w[n][k]) * f32(x[m][k])); summed in
 *                         double here (the reference's fp32 order is its own),
 *                         with sum |w x| returned for the tolerance.
 *   vo_argmax_bf16        kernels/ops/sampling_kernel.cu:11-63: per row, the
 *                         smallest index of the largest f32(logit); NaN never
 *                         wins; a row with no value above -inf gives 0.
 *   vo_group_dots         the exact int32 group sum that dp4a_q4_kernel.cu:116-150
 *                         forms and dp4a_smem_kernel.cu:49-58 / linear_multim.cu:
 *                         92-112 split into 8-element dp4a partials.
 *   vo_qlinear*           dp4a_smem_kernel.cu:25-74 and linear_multim.cu:64-130:
 *                         y = bf16_RNE( sum_g (ws[n,g] * xs[m,g]) * D[m,n,g]
 *                                       [+ f32(residual)] ), fp32, g ascending.
 *
 * Parity pins (tests/test_oracle.py): the Q4 weight quantizer is compared
 * with the reference's own convert.cpp built from /root/reference
 * (oracle/_ref); the formats by brute force over every code; the activation
 * quantizer by closed-form special cases and invariants; the dots by an
 * independent numpy brute force, linearity and the all-0x88 zero-weight KAT;
 * bf16/fp16 conversions by numpy/ml_dtypes-free closed forms.
 *
 * Formats (packed buffer of one weight matrix with N rows, K columns):
 *   Q4_G64  [N][K/2] bytes; byte k/2 of a row holds k even in its low nibble
 *           and k odd in its high nibble; nibble u = w + 8, w in [-8, 7].
 *   Q5_G64  low plane  [N][K/2] = Q4-style nibbles of (u & 15), u = w + 16,
 *           then high plane [N][K/8]: one little-endian u32 per 32-weight
 *           chunk; weight k = 32c + 8i + 2b + p (i<4, b<4, p<2) keeps bit 4 of
 *           u at bit 8b + 2i + p.  w in [-16, 15].
 *   Q6_G64  low plane  [N][K/2] as above with u = w + 32, then high plane
 *           [N][K/4]: two u32 per chunk; word j = i/2 keeps bits 4..5 of u at
 *           bits 8b + 4(i%2) + 2p.  w in [-32, 31].
 *   W8_G32  [N][K] int8 two's complement, w in [-127, 127].
 *   Scales  [N][K/G] 16-bit, fp16 (scale_enc 0) or bf16 (scale_enc 1).
 *   Activation group G = 64 for Q4/Q5/Q6 and 32 for W8_G32.
 */
#ifndef VIPER_ORACLE_H
#define VIPER_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum { VO_BF16 = 0, VO_FP32 = 1, VO_Q4_G64 = 4, VO_Q5_G64 = 5, VO_Q6_G64 = 6, VO_W8_G32 = 8 };
enum { VO_SCALE_FP16 = 0, VO_SCALE_BF16 = 1 };

/* ---- scalar conversions ---- */
float vo_bf16_to_f32(uint16_t h);
uint16_t vo_f32_to_bf16(float f);         /* round to nearest even, NaN kept quiet */
float vo_f16_to_f32(uint16_t h);
uint16_t vo_f32_to_f16(float f);          /* round to nearest even, overflow -> inf */
float vo_scale_to_f32(uint16_t s, int scale_enc);

/* ---- format facts ---- */
int vo_group_size(int qtype);             /* 64, or 32 for W8_G32; 0 if unknown */
int vo_wmin(int qtype);
int vo_wmax(int qtype);
size_t vo_packed_bytes(int qtype, int64_t N, int64_t K);

/* ---- pack / unpack integer weights w[N][K] ---- */
int vo_pack(int qtype, const int8_t* w, int N, int K, uint8_t* packed);
int vo_unpack(int qtype, const uint8_t* packed, int N, int K, int8_t* w);

/* ---- seeded, portable synthetic inputs (SplitMix64 stream) ---- */
uint64_t vo_splitmix64(uint64_t* state);
uint64_t vo_substream(uint64_t seed, uint64_t stream_id);
/* integer weights uniform in the format's full range, packed; scales
 * log-uniform in [1e-3, 1e-2] encoded as fp16 or bf16 (RNE). */
int vo_gen_weights(int qtype, int N, int K, uint64_t seed, int scale_enc,
                   uint8_t* packed, uint16_t* scales);
/* bf16 activations ~ N(0,1) (Box-Muller); channels whose seeded hash falls
 * below outlier_frac are multiplied by outlier_mul before rounding. */
void vo_gen_act(int M, int K, uint64_t seed, double outlier_frac, float outlier_mul,
                uint16_t* x);

/* ---- weight quantizer (offline converter semantics) ---- */
int vo_quantize_weights(int qtype, const uint16_t* w_bf16, int N, int K, int scale_enc,
                        uint8_t* packed, uint16_t* scales);

/* ---- activation quantize: x[M][K] bf16 -> xq[M][K] int8, xs[M][K/G] fp32 ---- */
int vo_quantize_act(const uint16_t* x, int M, int K, int group, int8_t* xq, float* xs);

/* out[M][H] = rmsnorm(x) * gamma (bf16), per row; eps as the reference's cfg.rms_eps. */
int vo_rmsnorm_bf16(const uint16_t* x, const uint16_t* gamma, float eps, int M, int H, uint16_t* out);

/* y[M][N] (bf16) = x[M][K] w[N][K]^T, both bf16; y_f32 and absterm (may be NULL)
 * receive the unrounded sum and sum |w x|. */
int vo_linear_bf16(const uint16_t* w, const uint16_t* x, int M, int N, int K, uint16_t* y,
                   float* y_f32, double* absterm);

/* out[b] = greedy token of logits[b][V] (bf16). */
int vo_argmax_bf16(const uint16_t* logits, int B, int V, int32_t* out);

/* out[M][I] = silu(gate) * up (bf16). */
int vo_swiglu_bf16(const uint16_t* gate, const uint16_t* up, int M, int I, uint16_t* out);

/* ---- exact per-group int32 dots: D[m][n][g] ---- */
int vo_group_dots(int qtype, const uint8_t* packed, int N, int K, const int8_t* xq, int M,
                  int32_t* D);

/* ---- full linear.  y[M][N] bf16; optional y_f32 (pre-rounding fp32 value) and
 * y_absterm (sum of |terms| in double, for the condition-aware tolerance). */
int vo_qlinear_prequant(int qtype, const uint8_t* packed, const uint16_t* scales,
                        int scale_enc, int N, int K, const int8_t* xq, const float* xs,
                        int M, const uint16_t* residual, uint16_t* y, float* y_f32,
                        double* y_absterm);
int vo_qlinear(int qtype, const uint8_t* packed, const uint16_t* scales, int scale_enc,
               int N, int K, const uint16_t* x, int M, const uint16_t* residual,
               uint16_t* y, float* y_f32, double* y_absterm);
/* Same arithmetic and outputs as vo_qlinear, output rows split over OpenMP
 * threads (the CPU baseline, and the oracle for production-size checks). */
int vo_qlinear_omp(int qtype, const uint8_t* packed, const uint16_t* scales, int scale_enc,
                   int N, int K, const uint16_t* x, int M, const uint16_t* residual,
                   uint16_t* y, float* y_f32, double* y_absterm, int nthreads);
int vo_omp_max_threads(void);

/* ---- the division-free identity used by the GPU quantizer ----
 * Returns the number of (amax, x) bf16 pairs with 0 <= x <= amax, amax's
 * exponent field in [exp_lo, exp_hi], for which
 *     RNE(fma(fma(-q0, s, x), r, q0)),  q0 = x*r,
 * differs from RNE(x / s) (IEEE divide), where s = max(amax/127, 1e-8) and
 * r = 1/s (IEEE divide).  Over exponents 0..254 this covers every finite bf16
 * pair (negative x follows by symmetry: every step is odd in x).  The
 * fp32 quotients themselves differ by one ulp in ~0.2% of pairs; the rounded
 * integers never do. */
int64_t vo_check_markstein(int exp_lo, int exp_hi, int64_t* n_checked);

#ifdef __cplusplus
}
#endif
#endif
