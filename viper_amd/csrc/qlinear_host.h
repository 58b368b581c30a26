// Host-side helpers and the launchers each kernel translation unit provides.
#pragma once

#include <hip/hip_runtime.h>

#include "qlinear_dev.h"

namespace vq {

// ------------------------------------------------------------------ host side

inline int status_of(hipError_t e) {
    if (e == hipSuccess) return VIPER_OK;
    if (e == hipErrorOutOfMemory) return VIPER_OUT_OF_MEMORY;
    return VIPER_DEVICE_ERROR;
}

inline int group_of(int qtype) {
    switch (qtype) {
        case VIPER_QTYPE_Q4_G64:
        case VIPER_QTYPE_Q5_G64:
        case VIPER_QTYPE_Q6_G64: return 64;
        case VIPER_QTYPE_W8_G32: return 32;
        default: return 0;
    }
}

inline size_t align16(size_t v) { return (v + 15) & ~(size_t)15; }

// LDS of the prequantized kernel for M rows
inline size_t lds_pre(int qtype, int M, int K) {
    const size_t G = (size_t)group_of(qtype);
    size_t b = (size_t)M * K + (size_t)M * (K / G) * 4;
    if (qtype != VIPER_QTYPE_W8_G32) b += (size_t)M * (K / 32) * 4;
    return b;
}

inline bool misaligned(const void* p, size_t a) { return ((uintptr_t)p % a) != 0; }

inline int validate_weights(int qtype, const void* w, const void* s, int senc, int group, int N,
                            int K, int M) {
    if (qtype == VIPER_QTYPE_BF16 || qtype == VIPER_QTYPE_FP32) return VIPER_UNIMPLEMENTED;
    const int G = group_of(qtype);
    if (G == 0) return VIPER_INVALID_ARGUMENT;
    if (w == nullptr || s == nullptr) return VIPER_INVALID_ARGUMENT;
    if (senc != VIPER_SCALE_FP16 && senc != VIPER_SCALE_BF16) return VIPER_INVALID_ARGUMENT;
    if (group != G) return VIPER_INVALID_ARGUMENT;
    if (N <= 0 || K <= 0 || M <= 0 || M > VIPER_QLINEAR_MAX_M || K > VIPER_QLINEAR_MAX_K) return VIPER_INVALID_ARGUMENT;
    if (K % G != 0) return VIPER_INVALID_ARGUMENT;
    if ((int64_t)M * K > INT32_MAX / 2) return VIPER_INVALID_ARGUMENT;
    // the kernels read scales in 8- and 16-byte loads (a workgroup's scale block at once)
    if (misaligned(w, 16) || misaligned(s, 16)) return VIPER_INVALID_ARGUMENT;
    return VIPER_OK;
}

inline void launch(const void* fn, unsigned grid, unsigned block, size_t lds, hipStream_t st, void** args) {
    (void)hipLaunchKernel(fn, dim3(grid), dim3(block), args, lds, st);
}

inline int device_cus() {
    int dev = 0, cus = 0;
    if (hipGetDevice(&dev) != hipSuccess) return 256;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0)
        return 256;
    return cus;
}

// LDS one workgroup may allocate on the current device (160 KB on gfx950).
// Most launch choices keep to LDS_MAX; the bf16-quantizing matrix-core mode
// stages a workgroup's activation fragments and uses the device's full budget.
inline int device_lds_max() {
    int dev = 0, lds = 0;
    if (hipGetDevice(&dev) != hipSuccess) return LDS_MAX;
    if (hipDeviceGetAttribute(&lds, hipDeviceAttributeMaxSharedMemoryPerBlock, dev) != hipSuccess || lds < LDS_MAX)
        return LDS_MAX;
    return lds;
}

// ---- launchers (one translation unit each)

// M = 1 (qgemv_m1.hip): one to three matrices of the same K (any N each)
// on one activation row produced by the prologue `pro` (PRO_BF16: x bf16,
// PRO_INT8: x int8 + xa scales, PRO_RMSNORM: x, xa = gamma, eps, xout,
// PRO_SWIGLU: x = gate, xa = up).  res and part belong to matrix 0.
enum { PRO_BF16 = 0, PRO_INT8 = 1, PRO_RMSNORM = 2, PRO_SWIGLU = 3 };
struct M1Out {
    const void* w;
    const void* s;
    void* y;
    int n;
};
size_t lds_m1(int qtype, int K);
bool m1_folded_ok(int qtype, int K, int N);
// M (1..4) activation rows: M > 1 needs one matrix, PRO_BF16 or PRO_INT8 and
// m1_rows_ok (x, y, res and part hold M rows).
int launch_m1(int qtype, int senc, int K, int pro, const void* x, const void* xa, float eps, void* xout,
              const M1Out* outs, int nouts, const void* res, int32_t* part, hipStream_t st, int M = 1);
bool m1_rows_ok(int qtype, int K, int M);
// m1_rows_ok and the bf16 rows are staged two octets per thread (Q4, exact
// tiling on 640 threads).
bool m1_rows_pair(int qtype, int K, int M);
// The M = 1 GEMV (bf16 x, exact tilings) with its per-wave timeline.
int launch_m1_timeline(int qtype, int senc, int K, const void* x, const void* w, const void* s, void* y, int N,
                       uint64_t* stamps, size_t stamp_bytes, int* workgroups, int* waves, hipStream_t st);
// M = 1 gate/up pair (one shape) with the swiglu epilogue: h = bf16(silu(g)
// * u) from the bf16-rounded outputs; g_out / u_out may be null.  Prologue
// PRO_BF16 or PRO_RMSNORM.
int launch_m1_swiglu(int qtype, int senc, int K, int pro, const void* x, const void* xa, float eps, void* xout,
                     const void* wg, const void* sg, const void* wu, const void* su, int N, void* h, void* g_out,
                     void* u_out, hipStream_t st);

// M <= 16 over prequantized activations, v_dot4 (qgemm_pre.hip).
int launch_pre(int qtype, const void* w, const void* s, int senc, int N, int K, const void* xq,
               const void* xs, int M, void* y, const void* res, int32_t* part, hipStream_t st);

// M = 2..16 on the i8 matrix cores (qgemm_mfma.hip): needs K a multiple of
// two groups and 4-byte aligned scales.  xnat: activations in the layout of
// viper_hip_quantize_act, else in the fragment order quantize_act_kernel<G,
// true> writes, which the shape must support (mfma_staged).
bool mfma_ok(int qtype, int K, int M, const void* s);

// M = 2..16, K a multiple of 4 groups (qgemm_rc.hip): row-contiguous weight
// loads moved into the matrix-core layout through LDS.  am (RC_FRAG, RC_NAT,
// RC_BF16 in qgemm_rc.h): reads the fragment order of the fragment quantize,
// the natural layout (xq, xs of viper_hip_quantize_act), or bf16 x [M][K]
// quantized by every workgroup (xq = x, xs unused; rc_bf16_ok must hold).
enum { RC_FRAG = 0, RC_NAT = 1, RC_BF16 = 2 };
bool rc_ok(int qtype, int K);
bool rc_bf16_ok(int qtype, int N, int K, int M, bool pair);
// K split of the fragment-input launch (long K): K in sk parts (2..RC_SK_MAX),
// one workgroup per (row block, part).  sc = the workspace's control words
// (offset 0 of every M > 1 workspace): sc[RC_CTL_MISS] counts sums that never
// arrived (their outputs are NaN; the library never clears it), and from
// sc[RC_CTL_CNT] one counter per row block (RC_CNT_MAX of them, reserved in
// every M > 1 layout so no other data lands there).  A counter holds
// 64 * epoch + the parts of the running call that have counted; the last part
// of a call (it counts sk - 1) adds 64 - sk, so every call starts on a
// multiple of 64 and the block's epoch (counter >> 6) grows by one per call.
// sp = the parts' sums as 64-bit {tag, fp32} slots in one record per row
// block (RC_REC_SLOTS slots at sp + block * RC_REC_SLOTS, the same place for
// every shape): a slot position is only ever written by its block, with the
// tag of that block's epoch.
constexpr int RC_SK_MAX = 8;      // parts of the K split
constexpr int RC_REC_ROWS = 48;   // rows of a row block (8 * rb, rb <= 6)
constexpr int RC_REC_SLOTS = RC_SK_MAX * VIPER_QLINEAR_MAX_M * RC_REC_ROWS;
constexpr int RC_CNT_MAX = 1024;  // row blocks a split launch may have
// Control words: the counters start a cache line of their own (byte 256).
constexpr int RC_CTL_MISS = 1, RC_CTL_CNT = 64;
constexpr size_t RC_CTL_BYTES = (size_t)RC_CTL_CNT * 4 + (size_t)RC_CNT_MAX * 4;
// The tag a call's slots carry: top byte 0x80 (no int8 activation byte, fp32
// activation scale or counter the workspace holds can have it), then the
// block's epoch, low 24 bits.
__host__ __device__ constexpr unsigned rc_tag(unsigned epoch) { return 0x80000000u | (epoch & 0x00FFFFFFu); }
// Split shape of a fragment-input launch (rows of both matrices, K): its row
// blocks (0 when K does not split); the sums' record bytes are
// blocks * RC_REC_SLOTS * 8.
int rc_split_blocks(int qtype, int N, int K);
int launch_rc(int qtype, const void* w, const void* s, int senc, int N, int K, const void* xq, const void* xs,
              int am, int M, void* y, const void* res, int32_t* part, const void* w1, const void* s1, void* y1,
              hipStream_t st, uint64_t* sp = nullptr, unsigned* sc = nullptr);
bool mfma_staged(int qtype, int N, int K);
int launch_rc_timeline(int qtype, const void* w, const void* s, int senc, int N, int K, const void* xq,
                       const void* xs, int M, void* y, uint64_t* stamps, size_t stamp_bytes, int* workgroups,
                       int* waves, unsigned* sc, hipStream_t st);
int launch_mfma(int qtype, const void* w, const void* s, int senc, int N, int K, const void* xq,
                const void* xs, bool xnat, int M, void* y, const void* res, int32_t* part,
                const void* w1, const void* s1, void* y1, hipStream_t st, uint64_t* sp = nullptr, unsigned* sc = nullptr);

}  // namespace vq
