// Producers of the quantized activation: rmsnorm and swiglu, each followed by
// the per-group int8 quantize, in one kernel (the reference's
// rmsnorm_quantize_bf16, kernels/ops/rmsnorm_quantize.cu:21-123, and
// swiglu_quantize_bf16, kernels/ops/swiglu_quantize.cu:21-96).
//
//  * rmsnorm: ss = sum x^2 over the row (fp32, fixed reduction order),
//    inv = rsqrt(ss / H + eps), v = bf16_RNE((x * inv) * gamma).
//  * swiglu: v = bf16_RNE(g / (1 + exp(-g)) * u).
//  * then, per group of G: s = max(amax / 127, 1e-8), q = RNE(v / s), from
//    the bf16 values (the reference quantizes the rounded producer output).
//
// Layout of the work: a thread owns one octet (8 consecutive elements) per
// step, so a G-group is G/8 adjacent lanes and its amax is a DPP reduction.
// rmsnorm needs the whole row for ss, so one workgroup owns a row; swiglu is
// elementwise up to the group, so workgroups tile the row.

#include "qlinear_host.h"

namespace vq {

constexpr int PR_NT = 256;  // threads per workgroup of the tiled (swiglu) kernel

// Sum over the workgroup: DPP/permute butterfly in each wave, then the wave
// sums in wave order.  Every thread gets the same value.
__device__ __forceinline__ float block_sum(float v, float* red, int nthreads) {
    v += dpp_f<DPP_SWAP1>(v);
    v += dpp_f<DPP_SWAP2>(v);
    v += dpp_f<DPP_HALF_MIRROR>(v);
    v += dpp_f<DPP_MIRROR>(v);
    v += __shfl_xor(v, 16, 64);
    v += __shfl_xor(v, 32, 64);
    const int nw = nthreads >> 6;
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
    __syncthreads();
    float t = 0.0f;
    for (int i = 0; i < nw; ++i) t += red[i];
    return t;
}

__device__ __forceinline__ void unpack8(const u32x4& v, float* f) {
    f[0] = bf16f(v.x & 0xffffu);
    f[1] = bf16f(v.x >> 16);
    f[2] = bf16f(v.y & 0xffffu);
    f[3] = bf16f(v.y >> 16);
    f[4] = bf16f(v.z & 0xffffu);
    f[5] = bf16f(v.z >> 16);
    f[6] = bf16f(v.w & 0xffffu);
    f[7] = bf16f(v.w >> 16);
}

__device__ __forceinline__ u32x4 pack8(const float* f) {
    return u32x4{f2bf2(f[0], f[1]), f2bf2(f[2], f[3]), f2bf2(f[4], f[5]), f2bf2(f[6], f[7])};
}

// Quantize the bf16 octet v (octet o of row `row`) into xq/xs; all lanes of
// the wave call this together (the group amax is a DPP reduction).
// Natural layout (FRAG false): xq/xs point at the row, xq [K] int8 in k order,
// xs [K/G] fp32.  Fragment layout (FRAG true, at most 16 rows): the matrix-core
// operand order the fragment quantize writes, xq and xs the whole buffers --
// group g's quarter qi (16 values; G = 32: its octet qi) sits in k-slot
// kb = bit-swap(qi) of lane 16 * kb + row, 64-groups as [even k | odd k] per
// octet, 32-groups in k order; xs [K/G][16].
template <int G, bool FRAG>
__device__ __forceinline__ void quantize_store(const u32x4& v, bool ok, int o, int row, int8_t* xq, float* xs) {
    uint32_t d0, d1;
    float s;
    quantize_octet<G, FRAG && G == 64>(v, d0, d1, s);
    if (ok) {
        if constexpr (FRAG) {
            constexpr int Q = G == 64 ? 16 : 8;  // fragment bytes per lane and group
            const int k0 = o * 8, g = k0 / G, qi = (k0 % G) / Q;
            const int kb = ((qi & 1) << 1) | (qi >> 1);
            *(u32x2*)(xq + ((size_t)(g * 4 + kb) * 16 + row) * Q + k0 % Q) = u32x2{d0, d1};
            if ((o & (G / 8 - 1)) == 0) xs[g * 16 + row] = s;
        } else {
            *(u32x2*)(xq + (size_t)o * 8) = u32x2{d0, d1};
            if ((o & (G / 8 - 1)) == 0) xs[o / (G / 8)] = s;
        }
    }
}

// One workgroup per row; bd = the workgroup size, a multiple of 64 (an
// argument rather than blockDim.x, which is a hidden argument the wave would
// wait for before its first load).
template <int G, bool FRAG>
__global__ void __launch_bounds__(1024)
rmsnorm_quantize_kernel(const uint16_t* __restrict__ x, const uint16_t* __restrict__ gamma, float eps,
                        int H, uint16_t* out, int8_t* __restrict__ xq, float* __restrict__ xs, int bd) {
    __shared__ float red[16];
    const int row = (int)blockIdx.x;
    const int noct = H / 8;
    const int iters = (noct + bd - 1) / bd;
    const uint16_t* xr = x + (size_t)row * H;

    float ss = 0.0f;
    for (int it = 0; it < iters; ++it) {
        const int o = (int)threadIdx.x + it * bd;
        if (o < noct) {
            float f[8];
            unpack8(*(const u32x4*)(xr + (size_t)o * 8), f);
#pragma unroll
            for (int j = 0; j < 8; ++j) ss = __builtin_fmaf(f[j], f[j], ss);
        }
    }
    ss = block_sum(ss, red, bd);
    const float inv = __builtin_amdgcn_rsqf(ss / (float)H + eps);

    int8_t* qr = FRAG ? xq : xq + (size_t)row * H;
    float* sr = FRAG ? xs : xs + (size_t)row * (H / G);
    for (int it = 0; it < iters; ++it) {
        const int o = (int)threadIdx.x + it * bd;
        const bool ok = o < noct;
        u32x4 v = {0u, 0u, 0u, 0u};
        if (ok) {
            float f[8], g[8];
            unpack8(*(const u32x4*)(xr + (size_t)o * 8), f);
            unpack8(*(const u32x4*)(gamma + (size_t)o * 8), g);
#pragma unroll
            for (int j = 0; j < 8; ++j) f[j] = (f[j] * inv) * g[j];
            v = pack8(f);
            if (out != nullptr) *(u32x4*)(out + (size_t)row * H + (size_t)o * 8) = v;
        }
        quantize_store<G, FRAG>(v, ok, o, row, qr, sr);
    }
}

// Workgroups tile each row (blockIdx.y = row); in place (out == gate) is
// allowed: every element is read before the same thread writes it.
template <int G, bool FRAG>
__global__ void __launch_bounds__(PR_NT)
swiglu_quantize_kernel(const uint16_t* gate, const uint16_t* __restrict__ up, int I, uint16_t* out,
                       int8_t* __restrict__ xq, float* __restrict__ xs) {
    const int row = (int)blockIdx.y;
    const int noct = I / 8;
    const int o = (int)blockIdx.x * PR_NT + (int)threadIdx.x;
    const bool ok = o < noct;
    const size_t base = (size_t)row * I + (size_t)o * 8;
    u32x4 v = {0u, 0u, 0u, 0u};
    if (ok) {
        float g[8], u[8];
        unpack8(*(const u32x4*)(gate + base), g);
        unpack8(*(const u32x4*)(up + base), u);
#pragma unroll
        for (int j = 0; j < 8; ++j) g[j] = silu_mul(g[j], u[j]);
        v = pack8(g);
        if (out != nullptr) *(u32x4*)(out + base) = v;
    }
    if constexpr (FRAG) quantize_store<G, true>(v, ok, o, row, xq, xs);
    else quantize_store<G, false>(v, ok, o, row, xq + (size_t)row * I, xs + (size_t)row * (I / G));
}

static int check_producer(int group, int M, int K, const void* a, const void* b, const void* out,
                          const void* xq, const void* xs) {
    if (group != 64 && group != 32) return VIPER_INVALID_ARGUMENT;
    if (a == nullptr || b == nullptr || xq == nullptr || xs == nullptr) return VIPER_INVALID_ARGUMENT;
    if (M <= 0 || K <= 0 || K % group != 0) return VIPER_INVALID_ARGUMENT;
    if ((int64_t)M * K > INT32_MAX / 2) return VIPER_INVALID_ARGUMENT;
    if (misaligned(a, 16) || misaligned(b, 16) || misaligned(out, 16) || misaligned(xq, 8) ||
        misaligned(xs, 4))
        return VIPER_INVALID_ARGUMENT;
    return VIPER_OK;
}

}  // namespace vq

namespace vq {

static int rmsnorm_launch(const void* x_bf16, const void* gamma_bf16, float eps, int M, int H, int group,
                          void* out_bf16, void* xq, void* xs, bool frag, void* stream) {
    int rc = check_producer(group, M, H, x_bf16, gamma_bf16, out_bf16, xq, xs);
    if (rc != VIPER_OK) return rc;
    if (frag && (M > 16 || misaligned(xq, 16) || misaligned(xs, 16))) return VIPER_INVALID_ARGUMENT;
    const int noct = H / 8;
    const int bd64 = (noct + 63) / 64 * 64;
    const unsigned bd = (unsigned)(bd64 < 1024 ? bd64 : 1024);
    const uint16_t* a0 = (const uint16_t*)x_bf16;
    const uint16_t* a1 = (const uint16_t*)gamma_bf16;
    uint16_t* a4 = (uint16_t*)out_bf16;
    int8_t* a5 = (int8_t*)xq;
    float* a6 = (float*)xs;
    int bdi = (int)bd;
    void* args[] = {&a0, &a1, &eps, &H, &a4, &a5, &a6, &bdi};
    const void* fn = group == 64 ? (frag ? (const void*)rmsnorm_quantize_kernel<64, true>
                                         : (const void*)rmsnorm_quantize_kernel<64, false>)
                                 : (frag ? (const void*)rmsnorm_quantize_kernel<32, true>
                                         : (const void*)rmsnorm_quantize_kernel<32, false>);
    (void)hipLaunchKernel(fn, dim3((unsigned)M), dim3(bd), args, 0, (hipStream_t)stream);
    return status_of(hipGetLastError());
}

static int swiglu_launch(const void* gate_bf16, const void* up_bf16, int M, int I, int group, void* out_bf16,
                         void* xq, void* xs, bool frag, void* stream) {
    int rc = check_producer(group, M, I, gate_bf16, up_bf16, out_bf16, xq, xs);
    if (rc != VIPER_OK) return rc;
    if (frag && (M > 16 || misaligned(xq, 16) || misaligned(xs, 16))) return VIPER_INVALID_ARGUMENT;
    const unsigned gx = (unsigned)((I / 8 + PR_NT - 1) / PR_NT);
    const uint16_t* a0 = (const uint16_t*)gate_bf16;
    const uint16_t* a1 = (const uint16_t*)up_bf16;
    uint16_t* a3 = (uint16_t*)out_bf16;
    int8_t* a4 = (int8_t*)xq;
    float* a5 = (float*)xs;
    void* args[] = {&a0, &a1, &I, &a3, &a4, &a5};
    const void* fn = group == 64 ? (frag ? (const void*)swiglu_quantize_kernel<64, true>
                                         : (const void*)swiglu_quantize_kernel<64, false>)
                                 : (frag ? (const void*)swiglu_quantize_kernel<32, true>
                                         : (const void*)swiglu_quantize_kernel<32, false>);
    (void)hipLaunchKernel(fn, dim3(gx, (unsigned)M), dim3(PR_NT), args, 0, (hipStream_t)stream);
    return status_of(hipGetLastError());
}

}  // namespace vq

extern "C" int viper_hip_rmsnorm_quantize(const void* x_bf16, const void* gamma_bf16, float eps, int M,
                                          int H, int group, void* out_bf16, void* xq, void* xs,
                                          void* stream) {
    return vq::rmsnorm_launch(x_bf16, gamma_bf16, eps, M, H, group, out_bf16, xq, xs, false, stream);
}

extern "C" int viper_hip_swiglu_quantize(const void* gate_bf16, const void* up_bf16, int M, int I,
                                         int group, void* out_bf16, void* xq, void* xs, void* stream) {
    return vq::swiglu_launch(gate_bf16, up_bf16, M, I, group, out_bf16, xq, xs, false, stream);
}

extern "C" int viper_hip_rmsnorm_quantize_frag(const void* x_bf16, const void* gamma_bf16, float eps, int M,
                                               int H, int group, void* out_bf16, void* xfrag, void* xsfrag,
                                               void* stream) {
    return vq::rmsnorm_launch(x_bf16, gamma_bf16, eps, M, H, group, out_bf16, xfrag, xsfrag, true, stream);
}

extern "C" int viper_hip_swiglu_quantize_frag(const void* gate_bf16, const void* up_bf16, int M, int I,
                                              int group, void* out_bf16, void* xfrag, void* xsfrag, void* stream) {
    return vq::swiglu_launch(gate_bf16, up_bf16, M, I, group, out_bf16, xfrag, xsfrag, true, stream);
}
