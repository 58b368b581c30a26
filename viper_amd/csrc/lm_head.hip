// LM head: bf16 GEMV (the reference's linear_bf16,
// kernels/ops/linear_bf16_kernel.cu:15-70) and greedy argmax
// (sampling_greedy_bf16, kernels/ops/sampling_kernel.cu:11-80).
//
// GEMV: y[m][n] = bf16_RNE(sum_k w[n][k] * x[m][k]) with fp32 accumulation.
// The matrix (vocab x hidden, e.g. 166144 x 2560 = 850 MB) is streamed once
// from HBM: a team of TS lanes owns a row and each lane issues its 16-byte
// chunks of the row at once (non-temporal loads), after the activation loads
// (loads retire in issue order, so x is staged into LDS while the weights
// are in flight).  Each 16-byte chunk is 8 bf16 and costs 4 v_dot2_f32_bf16
// per activation row; teams are reduced with DPP in a fixed order.
//
// Argmax: one workgroup per logits row; every lane requests all of its
// 16-byte octets at once, keeps the first octet holding its largest value
// (octet maxima by v_max, compared with strict >, so NaN never wins and ties
// keep the smaller index), then finds the first element of that octet equal
// to it; lanes and waves combine by (value, then smaller index).

#include "qlinear_host.h"

namespace vq {

typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));

__device__ __forceinline__ float dot2_bf16(uint32_t a, uint32_t b, float c) {
    return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, a), __builtin_bit_cast(bf16x2, b), c,
                                           false);
}

constexpr int LH_CPL = 10;  // 16-byte chunk slots per lane per row segment
constexpr int LH_XS = 4;    // activation octets per thread loaded before the weights

template <int TS, int NTT, int MT, bool EXACT>
__global__ void __launch_bounds__(NTT)
gemv_bf16_kernel(const uint16_t* __restrict__ w, const uint16_t* x, uint16_t* __restrict__ y,
                 int M, int N, int K) {
    constexpr int ROWS = NTT / TS;
    extern __shared__ __align__(16) u32x4 lx[];  // [M][K/8]
    const int tid = (int)threadIdx.x;
    const int l = tid % TS;
    const int rr = tid / TS;
    // row blocks in XCD order (each XCD streams one contiguous range of rows):
    // 121.5 -> 117.3 us for the 166144 x 2560 head
    const int row0 = xcd_block((int)blockIdx.x, (int)gridDim.x) * ROWS;
    const int row = row0 + rr;
    const int nrows = min(ROWS, N - row0);
    const bool row_ok = rr < nrows;
    const int CPR = K / 8;
    const int nx = M * CPR;

    // 1. activation octets, then the weight chunks of the first segment
    const auto xr = buf(x, (uint32_t)nx * 16);
    u32x4 xv[LH_XS];
#pragma unroll
    for (int i = 0; i < LH_XS; ++i) xv[i] = bload16(xr, (tid + NTT * i) * 16);
    issue_fence();
    const uint32_t rbytes = (uint32_t)K * 2;
    const auto wr = buf(w + (size_t)row0 * K, (uint32_t)nrows * rbytes);
    const int segw = TS * LH_CPL;
    const int nseg = EXACT ? 1 : (CPR + segw - 1) / segw;
    u32x4 wv[LH_CPL];
    auto load_seg = [&](int seg) {
#pragma unroll
        for (int j = 0; j < LH_CPL; ++j) {
            const int c = seg * segw + j * TS + l;
            const bool in = EXACT || c < CPR;
            wv[j] = bload16<AUX_NT>(wr, in ? rr * (int)rbytes + c * 16 : OOB);
        }
    };
    load_seg(0);

    // 2. stage x into LDS
#pragma unroll
    for (int i = 0; i < LH_XS; ++i)
        if (tid + NTT * i < nx) lx[tid + NTT * i] = xv[i];
    for (int i = tid + NTT * LH_XS; i < nx; i += NTT) lx[i] = bload16(xr, i * 16);
    lds_barrier();

    // 3. dots
    float acc[MT];
#pragma unroll
    for (int m = 0; m < MT; ++m) acc[m] = 0.0f;
    for (int seg = 0; seg < nseg; ++seg) {
        if (seg) load_seg(seg);
#pragma unroll
        for (int j = 0; j < LH_CPL; ++j) {
            const int c = seg * segw + j * TS + l;
            const bool ok = EXACT || c < CPR;
            const int cc = EXACT ? c : min(c, CPR - 1);
#pragma unroll
            for (int m = 0; m < MT; ++m) {
                if (m < M) {
                    const u32x4 a = lx[m * CPR + cc];
                    float t = acc[m];
                    t = dot2_bf16(wv[j].x, a.x, t);
                    t = dot2_bf16(wv[j].y, a.y, t);
                    t = dot2_bf16(wv[j].z, a.z, t);
                    t = dot2_bf16(wv[j].w, a.w, t);
                    acc[m] = ok ? t : acc[m];  // a lane past the row adds nothing (not even 0 * inf)
                }
            }
        }
    }
#pragma unroll
    for (int m = 0; m < MT; ++m) {
        if (m < M) {
            const float v = team_sum<TS>(acc[m]);
            if (l == 0 && row_ok) y[(size_t)m * N + row] = f2bf(v);
        }
    }
}

// (value, index) order of the greedy pick: larger value, then smaller index
__device__ __forceinline__ void better(float& v, int& i, float ov, int oi) {
    if (ov > v || (ov == v && oi < i)) {
        v = ov;
        i = oi;
    }
}

constexpr int AM_NT = 1024;
constexpr int AM_PT = 24;  // octets per lane in flight at once (the whole 166144-logit row in one pass)

// Largest of the 8 bf16 values of an octet (v_max_f32 / v_max3_f32 return
// the non-NaN operand, so NaN never wins, as with the strict > scan).
__device__ __forceinline__ float octet_max(const u32x4& q) {
    const float f0 = __uint_as_float(q.x << 16), f1 = __uint_as_float(q.x & 0xffff0000u);
    const float f2 = __uint_as_float(q.y << 16), f3 = __uint_as_float(q.y & 0xffff0000u);
    const float f4 = __uint_as_float(q.z << 16), f5 = __uint_as_float(q.z & 0xffff0000u);
    const float f6 = __uint_as_float(q.w << 16), f7 = __uint_as_float(q.w & 0xffff0000u);
    return fmaxf(fmaxf(fmaxf(f0, f1), fmaxf(f2, f3)), fmaxf(fmaxf(f4, f5), fmaxf(f6, f7)));
}

__global__ void __launch_bounds__(AM_NT)
argmax_bf16_kernel(const uint16_t* logits, int32_t* __restrict__ out, int V) {
    __shared__ float sv[AM_NT / 64];
    __shared__ int si[AM_NT / 64];
    const int b = (int)blockIdx.x;
    const int tid = (int)threadIdx.x;
    const uint16_t* row = logits + (size_t)b * V;
    // octets (16-byte loads when the row is 16-byte aligned): per lane the
    // first octet holding its largest value (octets are visited in increasing
    // order per lane, strict >), all of a pass's loads in flight at once
    // (buffer loads: past the row they read zero and are skipped by the
    // index bound)
    const bool vec = ((((uintptr_t)row) & 15) == 0);
    const int noct = vec ? V / 8 : 0;
    const auto rr = buf(row, (uint32_t)noct * 16);
    float best = -__builtin_inff();
    int boct = -1;
    for (int o0 = tid; o0 < noct; o0 += AM_NT * AM_PT) {
        u32x4 q[AM_PT];
#pragma unroll
        for (int i = 0; i < AM_PT; ++i) q[i] = bload16(rr, (o0 + i * AM_NT) * 16);
#pragma unroll
        for (int i = 0; i < AM_PT; ++i) {
            const int o = o0 + i * AM_NT;
            const float m = octet_max(q[i]);
            if (o < noct && m > best) {
                best = m;
                boct = o;
            }
        }
    }
    // the first element of that octet equal to its maximum
    int idx = 0;
    if (boct >= 0) {
        const u32x4 q = bload16(rr, boct * 16);
        const uint32_t wd[4] = {q.x, q.y, q.z, q.w};
        idx = boct * 8 + 7;
#pragma unroll
        for (int j = 7; j >= 0; --j)
            if (bf16f((wd[j >> 1] >> (16 * (j & 1))) & 0xffffu) == best) idx = boct * 8 + j;
    }
    // elements past the last octet (or an unaligned row), one per lane
    for (int v = noct * 8 + tid; v < V; v += AM_NT) {
        const float f = bf16f(row[v]);
        if (f > best) {
            best = f;
            idx = v;
        }
    }
    // Indices increase per lane but interleave across lanes, so equal maxima
    // resolve in the combine below (larger value, then smaller index).
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) {
        const float ov = __shfl_xor(best, off, 64);
        const int oi = __shfl_xor(idx, off, 64);
        better(best, idx, ov, oi);
    }
    if ((tid & 63) == 0) {
        sv[tid >> 6] = best;
        si[tid >> 6] = idx;
    }
    __syncthreads();
    if (tid == 0) {
        for (int i = 1; i < AM_NT / 64; ++i) better(best, idx, sv[i], si[i]);
        out[b] = idx;
    }
}

// Split argmax: P workgroups per row, each over GR_OCT consecutive octets
// (GR_NT threads, GR_OCT / GR_NT octets each, all requested at once), meet
// through a 64-bit key per row in the caller's workspace:
//   key = (order(value) << 32) | (0xFFFFFFFF - index),
// where order maps floats to unsigned integers in the same order (+0 for
// both zeros, which compare equal), so the largest key is the largest value
// at its smallest index, the reference's (value, then smaller index) pick.
// Each workgroup takes the max into the row's key, then (after the max has
// returned, so it is performed first) counts itself on the row's counter;
// the workgroup that counts last swaps the key for 0, resets the counter and
// writes the index.  All four accesses are agent-scope atomics, performed in
// the order each workgroup issues them, so the last count sees every max.
// A workgroup with nothing above -inf offers (-inf, 0): a row with nothing
// above -inf gives 0, as the single-workgroup kernel does.
constexpr int GR_NT = 256;
constexpr int GR_OCT = 512;  // octets (4096 logits, 8 KB) per workgroup

__device__ __forceinline__ uint64_t greedy_key(float v, int i) {
    const uint32_t u = v == 0.0f ? 0u : __float_as_uint(v);
    const uint32_t o = (u & 0x80000000u) ? ~u : (u | 0x80000000u);
    return ((uint64_t)o << 32) | (uint64_t)(0xFFFFFFFFu - (uint32_t)i);
}

__global__ void __launch_bounds__(GR_NT)
argmax_split_kernel(const uint16_t* logits, int32_t* __restrict__ out, int V, int P, uint64_t* keys,
                    unsigned* cnt) {
    __shared__ float sv[GR_NT / 64];
    __shared__ int si[GR_NT / 64];
    constexpr int PT = GR_OCT / GR_NT;
    const int b = (int)blockIdx.x / P, p = (int)blockIdx.x % P;
    const int tid = (int)threadIdx.x;
    const int noct = V / 8;  // whole octets (the host takes this kernel for V % 8 == 0 only)
    const int o0 = p * GR_OCT;
    const int n = min(GR_OCT, noct - o0);
    const auto rr = buf(logits + (size_t)b * V + (size_t)o0 * 8, (uint32_t)n * 16);
    u32x4 q[PT];
#pragma unroll
    for (int i = 0; i < PT; ++i) q[i] = bload16(rr, (tid + i * GR_NT) * 16);
    float best = -__builtin_inff();
    int boct = -1;
#pragma unroll
    for (int i = 0; i < PT; ++i) {
        const int o = tid + i * GR_NT;
        const float m = octet_max(q[i]);
        if (o < n && m > best) {
            best = m;
            boct = o;
        }
    }
    int idx = 0;
    if (boct >= 0) {
        const u32x4 v = bload16(rr, boct * 16);
        const uint32_t wd[4] = {v.x, v.y, v.z, v.w};
        idx = (o0 + boct) * 8 + 7;
#pragma unroll
        for (int j = 7; j >= 0; --j)
            if (bf16f((wd[j >> 1] >> (16 * (j & 1))) & 0xffffu) == best) idx = (o0 + boct) * 8 + j;
    }
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) {
        const float ov = __shfl_xor(best, off, 64);
        const int oi = __shfl_xor(idx, off, 64);
        better(best, idx, ov, oi);
    }
    if ((tid & 63) == 0) {
        sv[tid >> 6] = best;
        si[tid >> 6] = idx;
    }
    __syncthreads();
    if (tid == 0) {
        for (int i = 1; i < GR_NT / 64; ++i) better(best, idx, sv[i], si[i]);
        const uint64_t prev =
            __hip_atomic_fetch_max(keys + b, greedy_key(best, idx), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        // the count depends on the returned max (no key is all ones), so it
        // is issued only after the max is performed
        const unsigned inc = 1u + (unsigned)(prev == ~0ull);
        const unsigned t = __hip_atomic_fetch_add(cnt + b, inc, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        if (t == (unsigned)(P - 1)) {
            const uint64_t k = __hip_atomic_exchange(keys + b, 0ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            __hip_atomic_store(cnt + b, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            out[b] = (int32_t)(0xFFFFFFFFu - (uint32_t)k);
        }
    }
}

// ---- host

typedef void (*lh_fn)(const uint16_t*, const uint16_t*, uint16_t*, int, int, int);

template <int TS, bool EXACT>
static lh_fn lh_pick_mt(int mt) {
    switch (mt) {
        case 1: return gemv_bf16_kernel<TS, 256, 1, EXACT>;
        case 4: return gemv_bf16_kernel<TS, 256, 4, EXACT>;
        default: return gemv_bf16_kernel<TS, 256, 16, EXACT>;
    }
}
template <int TS>
static lh_fn lh_pick(int mt, bool exact) {
    return exact ? lh_pick_mt<TS, true>(mt) : lh_pick_mt<TS, false>(mt);
}

}  // namespace vq

extern "C" int viper_hip_linear_bf16(const void* w_bf16, const void* x_bf16, void* y_bf16, int M, int N,
                                     int K, void* stream) {
    if (w_bf16 == nullptr || x_bf16 == nullptr || y_bf16 == nullptr) return VIPER_INVALID_ARGUMENT;
    if (M <= 0 || N <= 0 || K <= 0 || M > VIPER_QLINEAR_MAX_M || K % 8 != 0) return VIPER_INVALID_ARGUMENT;
    if (vq::misaligned(w_bf16, 16) || vq::misaligned(x_bf16, 16) || vq::misaligned(y_bf16, 2))
        return VIPER_INVALID_ARGUMENT;
    const size_t lds = (size_t)M * K * 2;
    if (lds > (size_t)vq::LDS_MAX || (size_t)K * 2 * 256 > (size_t)INT32_MAX) return VIPER_INVALID_ARGUMENT;
    const int cpr = K / 8;
    int ts = 8;
    while (ts < 64 && ts * vq::LH_CPL < cpr) ts *= 2;
    const bool exact = cpr == ts * vq::LH_CPL;
    const int mt = M == 1 ? 1 : M <= 4 ? 4 : 16;
    vq::lh_fn fn;
    switch (ts) {
        case 8: fn = vq::lh_pick<8>(mt, exact); break;
        case 16: fn = vq::lh_pick<16>(mt, exact); break;
        case 32: fn = vq::lh_pick<32>(mt, exact); break;
        default: fn = vq::lh_pick<64>(mt, exact); break;
    }
    const int rows = 256 / ts;
    const unsigned grid = (unsigned)((N + rows - 1) / rows);
    const uint16_t* a0 = (const uint16_t*)w_bf16;
    const uint16_t* a1 = (const uint16_t*)x_bf16;
    uint16_t* a2 = (uint16_t*)y_bf16;
    void* args[] = {&a0, &a1, &a2, &M, &N, &K};
    (void)hipLaunchKernel((const void*)fn, dim3(grid), dim3(256), args, lds, (hipStream_t)stream);
    return vq::status_of(hipGetLastError());
}

extern "C" int viper_hip_sampling_greedy(const void* logits_bf16, int32_t* out_token, int B, int V,
                                         void* stream) {
    if (logits_bf16 == nullptr || out_token == nullptr || B <= 0 || V <= 0) return VIPER_INVALID_ARGUMENT;
    if (vq::misaligned(logits_bf16, 2) || vq::misaligned(out_token, 4)) return VIPER_INVALID_ARGUMENT;
    const uint16_t* a0 = (const uint16_t*)logits_bf16;
    void* args[] = {&a0, &out_token, &V};
    (void)hipLaunchKernel((const void*)vq::argmax_bf16_kernel, dim3((unsigned)B), dim3(vq::AM_NT), args, 0,
                          (hipStream_t)stream);
    return vq::status_of(hipGetLastError());
}

extern "C" size_t viper_hip_sampling_greedy_workspace_bytes(int B) {
    return B > 0 ? (size_t)B * 16 : 0;
}

extern "C" int viper_hip_sampling_greedy_split(const void* logits_bf16, int32_t* out_token, int B, int V,
                                               void* workspace, size_t workspace_bytes, void* stream) {
    if (logits_bf16 == nullptr || out_token == nullptr || workspace == nullptr || B <= 0 || V <= 0)
        return VIPER_INVALID_ARGUMENT;
    if (vq::misaligned(logits_bf16, 2) || vq::misaligned(out_token, 4) || vq::misaligned(workspace, 8) ||
        workspace_bytes < viper_hip_sampling_greedy_workspace_bytes(B))
        return VIPER_INVALID_ARGUMENT;
    // rows that are not whole 16-byte octets take the one-workgroup kernel
    if (vq::misaligned(logits_bf16, 16) || V % 8 != 0)
        return viper_hip_sampling_greedy(logits_bf16, out_token, B, V, stream);
    int P = (V / 8 + vq::GR_OCT - 1) / vq::GR_OCT;
    if ((long)P * B > (long)INT32_MAX) return VIPER_INVALID_ARGUMENT;
    const uint16_t* a0 = (const uint16_t*)logits_bf16;
    uint64_t* keys = (uint64_t*)workspace;
    unsigned* cnt = (unsigned*)(keys + B);
    void* args[] = {&a0, &out_token, &V, &P, &keys, &cnt};
    (void)hipLaunchKernel((const void*)vq::argmax_split_kernel, dim3((unsigned)(P * B)), dim3(vq::GR_NT), args, 0,
                          (hipStream_t)stream);
    return vq::status_of(hipGetLastError());
}
