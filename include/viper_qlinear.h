/*
 * viper_qlinear.h -- C ABI of the MI355X (gfx950) quantized linear path.
 *
 * This is the drop-in boundary under Viper's closed `linear()` switch.  Every
 * entry point is `extern "C"`, takes plain pointers and sizes, returns an int
 * equal to a viper::StatusCode value, never throws and allocates nothing.
 * All pointers are caller-owned device memory; calls are asynchronous and
 * ordered on `stream` (a hipStream_t, or NULL for the null stream).  Launch
 * errors are returned at once; device faults surface at the caller's next
 * synchronising call.  No entry point keeps state between calls, so calls
 * are re-entrant from any host thread.
 *
 * Reference interfaces replaced (itzrnvr/viper):
 *   viper_hip_qlinear               the Q4_G64 / Q5_G64|Q6_G64 / W8_G32 cases of
 *                                   ops::linear_forward (src/viper/linear.cpp:16-36,
 *                                   include/viper/ops.h:30-33), i.e. the
 *                                   quantize + dp4a GEMV pair the engine calls
 *                                   directly: rmsnorm_quantize_bf16 / quantize_to_q8
 *                                   + dp4a_smem_gemv{,_residual}
 *                                   (kernels/ops/dp4a_smem_kernel.h:10-20) and
 *                                   linear_q4_multim{,_residual}
 *                                   (kernels/ops/linear_multim.h:11-20).
 *   viper_hip_quantize_act          quantize_to_q8 (kernels/ops/linear_multim.h:24-26).
 *   viper_hip_qlinear_prequantized  dp4a_smem_gemv{,_residual}
 *                                   (kernels/ops/dp4a_smem_kernel.h:10-20) and
 *                                   linear_q4_dp4a_prequantized{,_residual}
 *                                   (kernels/ops/linear_multim.h:30-41).
 *   viper_hip_qlinear_fused2_prequantized
 *                                   dp4a_smem_gemv_fused2 (kernels/ops/dp4a_smem_kernel.cu:141-152,
 *                                   declared kernels/ops/dp4a_smem_kernel.h:22-27):
 *                                   two matrices of one shape (k and v, gate and up,
 *                                   include/viper/model_impl.cuh:652,725) on one
 *                                   quantized activation in one launch.
 *   viper_hip_qlinear_fused2        the same from bf16 x (quantize fused at M = 1).
 *   viper_hip_qlinear_m1            no single counterpart: one launch for what the engine
 *                                   does in two to four (include/viper/model_impl.cuh:650-652,
 *                                   719-720, 724-725, 727-728): the producer (rmsnorm+quantize,
 *                                   swiglu+quantize, quantize) folded into the GEMV prologue,
 *                                   and up to three matrices (q, k, v / gate, up) per launch.
 *   viper_hip_rmsnorm_quantize      rmsnorm_quantize_bf16 (kernels/ops/rmsnorm_quantize.cu:107-123,
 *                                   declared kernels/ops/rmsnorm_kernel.h), per row.
 *   viper_hip_swiglu_quantize       swiglu_quantize_bf16 (kernels/ops/swiglu_quantize.cu:81-96).
 *   viper_hip_rmsnorm_quantize_frag, viper_hip_swiglu_quantize_frag
 *                                   the same for M <= 16 rows in the matrix-core
 *                                   fragment order (the engine's verify step).
 *   viper_hip_qlinear_prequantized_frag, viper_hip_qlinear_fused2_prequantized_frag
 *                                   linear_q4_dp4a_prequantized / dp4a_smem_gemv_fused2
 *                                   at M = 2..16 from those fragments, one launch.
 *   viper_hip_linear_bf16           linear_bf16 (kernels/ops/linear_bf16_kernel.cu:57-70,
 *                                   declared kernels/ops/linear_bf16_kernel.h): the bf16 LM
 *                                   head GEMV (src/viper/model.cpp:300-304).
 *   viper_hip_sampling_greedy       sampling_greedy_bf16 (kernels/ops/sampling_kernel.cu:66-80).
 *   viper_hip_sampling_greedy_split the same, each row over many workgroups that meet in a
 *                                   caller workspace (no counterpart; the reference runs one
 *                                   block per row).
 *   viper_hip_qlinear_partials      no counterpart: the same kernels, also writing
 *                                   the exact per-group int32 dots for parity tests.
 *   viper_hip_qlinear_timeline      no counterpart: the M = 1 GEMV with per-wave
 *                                   timestamps (measurement).
 *   viper_hip_qlinear_frag_timeline no counterpart: the M = 2..16 matrix-core GEMM
 *                                   with per-wave timestamps (measurement).
 *   viper_hip_check_bf16_rounding   no counterpart: device self-check of the
 *                                   bf16 output rounding.
 *   viper_hip_check_quantizer       no counterpart: device self-check of the
 *                                   activation quantizer's rounding.
 *   viper_hip_stream_read           no counterpart: reads a buffer once with the
 *                                   M = 1 GEMV's load pattern and a given launch
 *                                   shape (measurement: the floor of one
 *                                   streaming dispatch).
 *   viper_hip_clock_stamp           no counterpart: a device-clock reading between
 *                                   launches (measurement).
 *   viper_hip_empty_dispatch        no counterpart: a launch that reads nothing
 *                                   (measurement: the fixed cost of a dispatch).
 *   viper_hip_prefetch              no counterpart: warms a weight range into the
 *                                   memory-side cache from a second stream.
 *
 * Formats (qtype values are viper::quant::QType, include/viper/quant.h:19-26):
 *   Q4_G64 (4)  packed [N][K/2]; k even in the low nibble; nibble = w + 8.
 *   Q5_G64 (5)  low plane [N][K/2] (nibbles of u = w + 16), then high plane
 *               [N][K/8]: per 32-weight chunk one u32 holding bit 4 of u for
 *               weight 8i+2b+p at bit 8b+2i+p.
 *   Q6_G64 (6)  low plane [N][K/2] (u = w + 32), then high plane [N][K/4]: per
 *               chunk two u32; word i/2 holds bits 4..5 of u at bit 8b+4(i%2)+2p.
 *   W8_G32 (8)  [N][K] int8, w in [-127, 127].
 *   Scales [N][K/G] 16-bit: fp16 (scale_enc 0) or bf16 (scale_enc 1).
 *   G = 64 for Q4/Q5/Q6, 32 for W8; activations are quantized per row and per
 *   G-group: s = max(amax/127, 1e-8), q = RNE(x/s) clamped to +-127.
 *   y[m][n] = bf16_RNE( sum_g ws[n][g] * xs[m][g] * D[m][n][g] [+ residual] ),
 *   D = exact int32 group dot.
 *
 * Alignment: w_packed, scales and x 16 bytes, xq 8 bytes, xs 4 bytes, y and
 * residual 2 bytes, partials 4 bytes.  Shapes: N, K, M > 0, K % G == 0,
 * M <= 16.
 */
#ifndef VIPER_QLINEAR_H
#define VIPER_QLINEAR_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Status codes: the numbering of viper::StatusCode (include/viper/status.h:12-21). */
#define VIPER_OK 0
#define VIPER_UNIMPLEMENTED 1
#define VIPER_INVALID_ARGUMENT 2
#define VIPER_DEVICE_ERROR 3 /* CUDA_ERROR in the reference */
#define VIPER_SHAPE_MISMATCH 4
#define VIPER_OUT_OF_MEMORY 5
#define VIPER_INTERNAL 99

/* QType values (include/viper/quant.h:19-26). */
#define VIPER_QTYPE_BF16 0
#define VIPER_QTYPE_FP32 1
#define VIPER_QTYPE_Q4_G64 4
#define VIPER_QTYPE_Q5_G64 5
#define VIPER_QTYPE_Q6_G64 6
#define VIPER_QTYPE_W8_G32 8

#define VIPER_SCALE_FP16 0
#define VIPER_SCALE_BF16 1

#define VIPER_QLINEAR_MAX_M 16
/* Longest K of the quantized entry points (a workgroup's block of weight
 * rows is addressed with 32-bit sizes and offsets); longer K is
 * INVALID_ARGUMENT. */
#define VIPER_QLINEAR_MAX_K (1 << 24)
/* Most output rows N of one matrix at M = 1 (the launch's row count shares a
 * word with flags); the M > 1 kernels take fewer than 2^27.  More is
 * INVALID_ARGUMENT. */
#define VIPER_QLINEAR_MAX_N ((1 << 30) - 1)
/* 7: the K split keeps its own per-block counters (no launch before it), so
 *    the fragment-input entry points take an optional workspace;
 *    viper_hip_qlinear_frag_workspace_bytes; the workspace layout's offsets
 *    changed (viper_hip_qlinear_workspace_layout).
 * 6: the M > 1 workspace is zero-filled before its first use and keeps the
 *    K split's control words at offset 0 (5 needed no initialisation).
 * 5: weight scales must be 16-byte aligned (4 accepted 2-byte aligned scales) */
#define VIPER_QLINEAR_ABI_VERSION 7

int viper_hip_abi_version(void);

/* Group size of a quantized qtype (64 or 32), 0 for anything else. */
int viper_hip_group_size(int qtype);

/* Bytes of caller workspace viper_hip_qlinear needs for this shape; 0 when
 * the activation quantize is fused into the GEMV (M == 1).  It holds the K
 * split's control words and block counters (the first 4352 bytes, for every
 * shape), for long K on the matrix cores (K of more than 20 quads of 4
 * groups) the K split's fp32 part sums, then the int8 activations and their
 * scales.  A workspace is zero-filled before its
 * first use (hipMemset, torch.zeros); after that it serves any sequence of
 * shapes and entry points that fit it with no clearing (each call leaves it
 * valid for the next), as long as nothing else writes it.  Calls that use
 * one workspace concurrently race. */
size_t viper_hip_qlinear_workspace_bytes(int qtype, int N, int K, int M);

/* The workspace's layout for this shape (no counterpart in the reference;
 * tests and debugging).  Returns viper_hip_qlinear_workspace_bytes() and,
 * when offsets is not NULL, writes six values (SIZE_MAX where the shape has
 * no such part):
 *   [0] the count of K-split sums that did not arrive within the kernel's
 *       bounded wait (uint32 at byte 4 for every shape; such outputs are
 *       NaN; the library never clears it, so a caller can check it stayed 0),
 *   [1] the K split's block counters (1024 uint32 from byte 256, for every
 *       shape: 64 * epoch + parts counted, a multiple of 64 between calls),
 *   [2] the K split's part sums (from byte 4352 for every shape: one record
 *       of 8 * 16 * 48 64-bit slots per row block),
 *   [3] xq, [4] xs,
 *   [5] the K split's row blocks (a count, not an offset; 0 without it). */
size_t viper_hip_qlinear_workspace_layout(int qtype, int N, int K, int M, size_t* offsets);

/* y[M][N] = linear(w, x) with x[M][K] bf16 quantized per row and group.
 * residual (may be NULL) is added in fp32 before the bf16 round.  group must
 * equal the format's group size.  workspace may be NULL when
 * viper_hip_qlinear_workspace_bytes() is 0. */
int viper_hip_qlinear(int qtype, const void* w_packed, const void* w_scales, int scale_enc,
                      int group, int N, int K, const void* x_bf16, int M, void* y_bf16,
                      const void* residual_bf16, void* workspace, size_t workspace_bytes,
                      void* stream);

/* xq[M][K] int8 and xs[M][K/group] fp32 from x[M][K] bf16 (group 64 or 32). */
int viper_hip_quantize_act(int group, const void* x_bf16, int M, int K, void* xq, void* xs,
                           void* stream);

/* y[M][N] from already quantized activations xq[M][K] (natural order) and
 * xs[M][K/group]. */
int viper_hip_qlinear_prequantized(int qtype, const void* w_packed, const void* w_scales,
                                   int scale_enc, int group, int N, int K, const void* xq,
                                   const void* xs, int M, void* y_bf16,
                                   const void* residual_bf16, void* stream);

/* y0 = linear(w0, x) and y1 = linear(w1, x) for two weight matrices of the
 * same qtype, scale encoding and shape, in one launch; no residual.  The
 * workspace is that of viper_hip_qlinear for (qtype, N, K, M). */
int viper_hip_qlinear_fused2(int qtype, const void* w0_packed, const void* w0_scales,
                             const void* w1_packed, const void* w1_scales, int scale_enc, int group,
                             int N, int K, const void* x_bf16, int M, void* y0_bf16, void* y1_bf16,
                             void* workspace, size_t workspace_bytes, void* stream);

/* viper_hip_qlinear_fused2 from already quantized activations (as
 * viper_hip_qlinear_prequantized). */
int viper_hip_qlinear_fused2_prequantized(int qtype, const void* w0_packed, const void* w0_scales,
                                          const void* w1_packed, const void* w1_scales,
                                          int scale_enc, int group, int N, int K, const void* xq,
                                          const void* xs, int M, void* y0_bf16, void* y1_bf16,
                                          void* stream);

/* Prologues of viper_hip_qlinear_m1 (what a and b hold). */
#define VIPER_PROLOGUE_BF16 0    /* a: x bf16 [K], quantized in the kernel */
#define VIPER_PROLOGUE_INT8 1    /* a: xq int8 [K], b: xs fp32 [K/group] (8- and 4-byte aligned) */
#define VIPER_PROLOGUE_RMSNORM 2 /* a: x bf16 [K], b: gamma bf16 [K]; v = bf16((x * rsqrt(sum x^2 / K + eps)) * gamma) */
#define VIPER_PROLOGUE_SWIGLU 3  /* a: gate bf16 [K], b: up bf16 [K]; v = bf16(gate / (1 + exp(-gate)) * up) */

/* M = 1: y_i[N_i] = linear(w_i, v) for n_out = 1..3 matrices of one qtype,
 * scale encoding and K (each with its own N_i), where v is the activation
 * row the prologue produces and quantizes (exactly as viper_hip_rmsnorm_quantize
 * / viper_hip_swiglu_quantize / viper_hip_quantize_act would), all in one
 * launch.  w_packed, w_scales, N and y_bf16 are host arrays of n_out entries.
 * residual (may be NULL, may alias y_bf16[0]) is added to output 0.
 * norm_out (RMSNORM only, may be NULL) receives the bf16 row v.  The
 * RMSNORM and SWIGLU prologues need K <= 20480 (Q4/Q5/Q6; the whole row is
 * held after one load round); a, b and norm_out 16-byte aligned unless
 * stated. */
int viper_hip_qlinear_m1(int qtype, int scale_enc, int group, int K, int prologue, const void* a, const void* b,
                         float eps, void* norm_out, int n_out, const void* const* w_packed,
                         const void* const* w_scales, const int* N, void* const* y_bf16,
                         const void* residual_bf16, void* stream);

/* M = 1 gate/up pair with the swiglu epilogue, one launch:
 *   g = linear(w_gate, v), u = linear(w_up, v)   two matrices of one qtype,
 *                                                scale encoding and shape N x K;
 *   h[n] = bf16(silu(g[n]) * u[n])               from the bf16-rounded g and u,
 * where v is the activation row of the BF16 or RMSNORM prologue (a, b, eps
 * and norm_out as viper_hip_qlinear_m1).  h equals, bit for bit, the bf16
 * output of viper_hip_swiglu_quantize applied to the two outputs of
 * viper_hip_qlinear_m1 for the same matrices.  gate_bf16 and up_bf16 (may be
 * NULL) receive g and u.  Replaces dp4a_smem_gemv_fused2(gate, up) followed by
 * swiglu_quantize_bf16's silu (include/viper/model_impl.cuh:724-727), with the
 * int8 quantize of h left to the down projection's prologue. */
int viper_hip_qlinear_m1_swiglu(int qtype, int scale_enc, int group, int K, int prologue, const void* a,
                                const void* b, float eps, void* norm_out, const void* w_gate,
                                const void* s_gate, const void* w_up, const void* s_up, int N, void* h_bf16,
                                void* gate_bf16, void* up_bf16, void* stream);

/* Producer-side activation quantize, per row m < M of H (or I) elements:
 *   rmsnorm: v = bf16_RNE((x * rsqrt(sum(x^2)/H + eps)) * gamma),
 *   swiglu:  v = bf16_RNE(gate / (1 + exp(-gate)) * up),
 * then xq[M][H] int8 and xs[M][H/group] fp32 from v exactly as
 * viper_hip_quantize_act.  out_bf16 (may be NULL) receives v; for swiglu it
 * may alias gate (the reference's engine passes gate as the output).  x,
 * gamma, gate, up and out 16-byte aligned; group 64 or 32. */
int viper_hip_rmsnorm_quantize(const void* x_bf16, const void* gamma_bf16, float eps, int M, int H,
                               int group, void* out_bf16, void* xq, void* xs, void* stream);
int viper_hip_swiglu_quantize(const void* gate_bf16, const void* up_bf16, int M, int I, int group,
                              void* out_bf16, void* xq, void* xs, void* stream);

/* LM head: y[M][N] = bf16_RNE(x[M][K] w[N][K]^T), w and x bf16, fp32
 * accumulation.  M <= 16, K % 8 == 0, M*K*2 <= 64 KiB; w and x 16-byte
 * aligned. */
int viper_hip_linear_bf16(const void* w_bf16, const void* x_bf16, void* y_bf16, int M, int N, int K,
                          void* stream);

/* out_token[b] = the smallest index of the largest logits[b][V] (bf16); NaN
 * never wins; a row with nothing above -inf gives 0. */
int viper_hip_sampling_greedy(const void* logits_bf16, int32_t* out_token, int B, int V, void* stream);

/* viper_hip_sampling_greedy with each row split over workgroups of 4096
 * logits (41 for a 166144-logit row instead of one), which meet through
 * workspace: viper_hip_sampling_greedy_workspace_bytes(B) bytes, 8-byte
 * aligned, zero before the first call; every call leaves it zero again, so
 * it is reused without clearing (two calls in flight on one workspace race).
 * Same result as viper_hip_sampling_greedy; rows that are not whole 16-byte
 * words (V % 8 != 0 or logits not 16-byte aligned) take that kernel and
 * leave the workspace alone.  No counterpart in the reference. */
size_t viper_hip_sampling_greedy_workspace_bytes(int B);
int viper_hip_sampling_greedy_split(const void* logits_bf16, int32_t* out_token, int B, int V, void* workspace,
                                    size_t workspace_bytes, void* stream);

/* viper_hip_qlinear without a workspace argument, for callers that cannot
 * allocate device memory (code under HIP graph capture, tight serving loops,
 * harnesses that forbid hipMalloc).  No counterpart in the reference.  The
 * workspace is a static device array of VIPER_QLINEAR_STATIC_SCRATCH_BYTES
 * per GPU (zero when the library is loaded), held until the process ends;
 * the call allocates nothing.  Shapes whose
 * viper_hip_qlinear_workspace_bytes() exceeds it return INVALID_ARGUMENT.
 * Every call on one GPU shares that GPU's array: calls that overlap on one
 * GPU (concurrent streams or host threads) race; calls ordered on one stream
 * do not.  Results equal viper_hip_qlinear's bit for bit. */
#define VIPER_QLINEAR_STATIC_SCRATCH_BYTES (8u << 20)
int viper_hip_qlinear_static(int qtype, const void* w_packed, const void* w_scales, int scale_enc,
                             int group, int N, int K, const void* x_bf16, int M, void* y_bf16,
                             const void* residual_bf16, void* stream);

/* viper_hip_qlinear, also writing D[M][N][K/group] int32 (test use). */
int viper_hip_qlinear_partials(int qtype, const void* w_packed, const void* w_scales,
                               int scale_enc, int group, int N, int K, const void* x_bf16, int M,
                               void* y_bf16, const void* residual_bf16, void* workspace,
                               size_t workspace_bytes, int32_t* partials, void* stream);

/* Device self-check of the fp32 -> bf16 rounding the kernels use (test
 * use): every fp32 bit pattern through the hardware conversion and through
 * the round-to-nearest-even statement (NaN kept quiet with its top payload
 * bits); adds the number of disagreements to *count (uint64, zeroed by the
 * caller). */
int viper_hip_check_bf16_rounding(unsigned long long* count, void* stream);

/* Device self-check of the division-free quantizer step (test use): for
 * every finite bf16 pair (amax, x) with 0 <= x <= amax and amax's exponent
 * field in [exp_lo, exp_hi] (0..254), compares the kernels' rounding with an
 * IEEE divide on the device.  counts[i] (int32, (exp_hi-exp_lo+1)*128
 * entries) receives the number of disagreements for amax bits
 * (exp_lo << 7) + i. */
int viper_hip_check_quantizer(int exp_lo, int exp_hi, int32_t* counts, void* stream);

/* Measurement entry point, no counterpart in the reference: the M = 1 GEMV
 * of viper_hip_qlinear (any quantized format, bf16 x, launch shapes whose
 * lanes tile a row exactly, e.g. K = 2560) with a per-wave timeline.  Lane 0 of every wave
 * writes 8 s_memrealtime readings (uint64, 100 MHz) to
 * stamps[(workgroup * waves + wave) * 8 + i]: wave start, activation and
 * weight-scale loads issued, weight loads issued, activation quantized into
 * LDS, workgroup barrier passed, first chunk dotted, last chunk dotted,
 * output stored.  *workgroups and *waves_per_workgroup (may be NULL) receive
 * the launch's grid; stamp_bytes must cover it.  y is the GEMV's output; the
 * readings cost the kernel about 0.2 us. */
int viper_hip_qlinear_timeline(int qtype, const void* w_packed, const void* w_scales, int scale_enc, int group,
                               int N, int K, const void* x_bf16, void* y_bf16, uint64_t* stamps, size_t stamp_bytes,
                               int* workgroups, int* waves_per_workgroup, void* stream);

/* Measurement probe, no counterpart in the reference: the floor of one
 * dispatch streaming `bytes` with the M = 1 GEMV's load pattern.  Each team
 * of 16 lanes reads one row of 16 * loads 16-byte chunks (lane l takes chunks
 * j * 16 + l), with non-temporal loads all issued at once; workgroups of
 * `threads` threads (64, 128, 256, 320, 512, 640 or 1024) cover threads / 16
 * rows each, in the GEMV's XCD-aware order; loads is 4, 5, 8, 10 or 16, and
 * bytes a multiple of threads * loads * 16 (16-byte aligned buffer).  With
 * side (16-byte aligned; NULL exactly when side_bytes is 0) every workgroup
 * first reads its own side_bytes (a multiple of 16, at most 16 * threads) at
 * side + workgroup * side_bytes, one 16-byte load per thread, as the GEMV
 * reads its block of weight scales.  With y_bf16 (may be NULL) every team
 * also stores one bf16 to y_bf16[row] (the GEMV's output pattern;
 * bytes / (256 * loads) entries).  Otherwise sink (4 bytes) is written only
 * if the folded data equals a fixed word. */
int viper_hip_stream_read(const void* buf, size_t bytes, int threads, int loads, const void* side, int side_bytes,
                          void* y_bf16, uint32_t* sink, void* stream);

/* Measurement entry point, no counterpart in the reference: the M = 2..16
 * matrix-core GEMM of viper_hip_qlinear_prequantized_frag (Q4_G64 or W8_G32,
 * K a multiple of 4 groups; at most 20 quads of 4 groups: one segment, or with a
 * workspace of viper_hip_qlinear_frag_workspace_bytes() (16-byte aligned)
 * the K split of a long K) with a per-wave timeline.  Lane 0 of every wave
 * writes 10 s_memrealtime readings (uint64, 100 MHz) to
 * stamps[(workgroup * waves + wave) * 10 + i]: wave start, activation and
 * scale loads issued, weight loads issued, staged scales in LDS, first group
 * scaled, last group scaled, cross-wave barrier passed, sums stored (y, or
 * the K split's slots), counted (the K split's block counter returned),
 * outputs stored (y by the K split's last part of a block); readings a
 * workgroup does not reach repeat its last one.  *workgroups and
 * *waves_per_workgroup (may be NULL) receive the grid; stamp_bytes must
 * cover it.  y equals the production call's bit for bit. */
int viper_hip_qlinear_frag_timeline(int qtype, const void* w_packed, const void* w_scales, int scale_enc, int group,
                                    int N, int K, const void* xfrag, const void* xsfrag, int M, void* y_bf16,
                                    uint64_t* stamps, size_t stamp_bytes, int* workgroups, int* waves_per_workgroup,
                                    void* workspace, size_t workspace_bytes, void* stream);

/* Warms `bytes` (a multiple of 16, 16-byte aligned) at buf into the GPU's
 * memory-side cache with plain loads, split over `workgroups` workgroups of
 * 256 threads; sink (4 bytes) is written only if the folded data equals a
 * fixed word.  For a second stream next to the one that runs the current
 * launches: the next launches' weights then come from the cache.  No
 * counterpart in the reference. */
int viper_hip_prefetch(const void* buf, size_t bytes, int workgroups, uint32_t* sink, void* stream);

/* Fragment order of 2..16 quantized activation rows: the matrix-core
 * operand layout the verify path's GEMM reads directly.  For G = 64,
 * xfrag [K/64][64 lanes][16 B]: lane 16 * kb + m of group g holds row m's
 * quarter qi = ((kb & 1) << 1) | (kb >> 1) of the group (k = 64g + 16qi ..
 * +15) as four 4-byte words: the even k of its first octet, the odd k of
 * that octet, then the same for the second octet.  For G = 32, xfrag
 * [K/32][4 kb][16 m][8 B]: row m's octet qi of group g in k order.  xsfrag
 * [K/G][16] fp32: the scale of row m's group g at g * 16 + m.  Rows M..15 are
 * never written and never used.  Both buffers 16-byte aligned, sized for 16
 * rows (K and 4 * K / G * 16 bytes). */

/* rmsnorm_quantize_bf16 / swiglu_quantize_bf16 (kernels/ops/rmsnorm_quantize.cu:107-123,
 * kernels/ops/swiglu_quantize.cu:81-96) for M <= 16 rows, writing the int8
 * rows and their scales in the fragment order above instead of [M][K] and
 * [M][K/G]: the same bytes and scales as viper_hip_rmsnorm_quantize /
 * viper_hip_swiglu_quantize, so the engine's verify step (M rows,
 * include/viper/model_impl.cuh:585-607) feeds its linears without a
 * quantize launch of their own. */
int viper_hip_rmsnorm_quantize_frag(const void* x_bf16, const void* gamma_bf16, float eps, int M, int H,
                                    int group, void* out_bf16, void* xfrag, void* xsfrag, void* stream);
int viper_hip_swiglu_quantize_frag(const void* gate_bf16, const void* up_bf16, int M, int I, int group,
                                   void* out_bf16, void* xfrag, void* xsfrag, void* stream);

/* linear_q4_dp4a_prequantized{,_residual} (kernels/ops/linear_multim.h:30-41)
 * and dp4a_smem_gemv_fused2 (kernels/ops/dp4a_smem_kernel.cu:141-152) at
 * M = 2..16 over activations in the fragment order above: one launch of the
 * matrix-core kernel.  K must be a multiple of 4 groups.  workspace (16-byte
 * aligned, may be NULL): with viper_hip_qlinear_frag_workspace_bytes() bytes
 * or more, long K is split over workgroups (the reference's hidden static
 * buffer, kernels/ops/linear_multim.cu:133-146, in the caller's hands); with
 * NULL, or for shapes that need none, each workgroup loops over all of K.
 * Same workspace rules as viper_hip_qlinear's (zero-filled before its first
 * use, then reused by any entry point without clearing; concurrent calls on
 * one workspace race).  The fused pair takes no workspace. */
size_t viper_hip_qlinear_frag_workspace_bytes(int qtype, int N, int K, int M);
int viper_hip_qlinear_prequantized_frag(int qtype, const void* w_packed, const void* w_scales, int scale_enc,
                                        int group, int N, int K, const void* xfrag, const void* xsfrag, int M,
                                        void* y_bf16, const void* residual_bf16, void* workspace,
                                        size_t workspace_bytes, void* stream);
int viper_hip_qlinear_fused2_prequantized_frag(int qtype, const void* w0_packed, const void* w0_scales,
                                               const void* w1_packed, const void* w1_scales, int scale_enc,
                                               int group, int N, int K, const void* xfrag, const void* xsfrag,
                                               int M, void* y0_bf16, void* y1_bf16, void* stream);

/* Measurement probe, no counterpart in the reference: one launch of one
 * wave that writes the GPU's constant 100 MHz counter (s_memrealtime) to
 * out[0] (uint64, 8-byte aligned).  Two of them around a sequence of
 * launches on one stream time the sequence on the device's clock. */
int viper_hip_clock_stamp(uint64_t* out, void* stream);

/* Measurement probe, no counterpart in the reference: one launch of
 * `workgroups` x `threads` (a multiple of 64, at most 1024) that reads
 * nothing.  With y_bf16 (2-byte aligned, workgroups * threads / 16 entries)
 * lane 0 of every 16-lane team stores one bf16 to y_bf16[row], the M = 1
 * GEMV's output pattern; with NULL nothing is stored.  Back-to-back launches
 * time the fixed cost of a dispatch. */
int viper_hip_empty_dispatch(int workgroups, int threads, void* y_bf16, void* stream);

#ifdef __cplusplus
}
#endif
#endif /* VIPER_QLINEAR_H */
