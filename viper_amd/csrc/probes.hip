// Measurement probes (no counterpart in the reference): the floor of one
// dispatch that streams a buffer with the M = 1 GEMV's load pattern, and a
// reading of the device clock between launches.
#include "qlinear_host.h"

namespace vq {

// A team of 16 lanes reads one "row" of 16 * L 16-byte chunks, lane l taking
// chunks j * 16 + l (j < L) with 16-byte non-temporal loads, all issued at
// once: the GEMV's pattern (north star: 1280-byte rows, L = 5).  A workgroup
// of NTT threads covers NTT / 16 consecutive rows, workgroups in the
// XCD-aware order of the GEMV.  Nothing else happens to the data: the words
// are folded so the loads stay live.  With y, lane 0 of each team stores one
// bf16 (the fold) to y[row], the GEMV's output pattern; without it the fold
// reaches memory only in the (never expected) case that it equals a magic
// word.  With side (side_bytes per workgroup, a multiple of 16, at most
// 16 * NTT), threads t < side_bytes / 16 first load 16 bytes each of the
// workgroup's side block, as the GEMV loads its block of weight scales.
template <int NTT, int L>
__global__ void __launch_bounds__(NTT) stream_probe_kernel(const uint8_t* p, uint16_t* y, uint32_t* sink,
                                                           const uint8_t* side, int side_bytes) {
    constexpr int ROWS = NTT / 16, RB = 16 * L * 16;
    const int b = xcd_block((int)blockIdx.x, (int)gridDim.x);
    const int tid = (int)threadIdx.x, l = tid & 15, rr = tid >> 4;
    const auto sr = buf(side + (size_t)b * side_bytes, (uint32_t)side_bytes);
    const u32x4 sv = bload16(sr, tid * 16 < side_bytes ? tid * 16 : OOB);
    const auto r = buf(p + (size_t)b * ROWS * RB, (uint32_t)(ROWS * RB));
    u32x4 v[L];
#pragma unroll
    for (int j = 0; j < L; ++j) v[j] = bload16<AUX_NT>(r, rr * RB + (j * 16 + l) * 16);
    uint32_t f = sv.x ^ sv.y ^ sv.z ^ sv.w;
#pragma unroll
    for (int j = 0; j < L; ++j) f ^= v[j].x ^ v[j].y ^ v[j].z ^ v[j].w;
    if (y != nullptr) {
        if (l == 0) y[(size_t)b * ROWS + rr] = (uint16_t)f;
    } else if (f == 0x9E3779B9u) {
        sink[0] = f;
    }
}

typedef void (*probe_fn)(const uint8_t*, uint16_t*, uint32_t*, const uint8_t*, int);

template <int NTT>
static probe_fn probe_l(int loads) {
    switch (loads) {
        case 4: return stream_probe_kernel<NTT, 4>;
        case 5: return stream_probe_kernel<NTT, 5>;
        case 8: return stream_probe_kernel<NTT, 8>;
        case 10: return stream_probe_kernel<NTT, 10>;
        case 16: return stream_probe_kernel<NTT, 16>;
        default: return nullptr;
    }
}

static probe_fn probe_kernel(int threads, int loads) {
    switch (threads) {
        case 64: return probe_l<64>(loads);
        case 128: return probe_l<128>(loads);
        case 256: return probe_l<256>(loads);
        case 320: return probe_l<320>(loads);
        case 512: return probe_l<512>(loads);
        case 640: return probe_l<640>(loads);
        case 1024: return probe_l<1024>(loads);
        default: return nullptr;
    }
}

// One reading of the GPU's constant-rate 100 MHz counter (s_memrealtime)
// into out[0].  Placed on a stream before and after a sequence of launches,
// it times that sequence on the device's own clock.
__global__ void __launch_bounds__(64) clock_stamp_kernel(uint64_t* out) {
    const uint64_t t = __builtin_amdgcn_s_memrealtime();
    if (threadIdx.x == 0) out[0] = t;
}

// A dispatch that reads nothing: with y, lane 0 of every 16-lane team stores
// one bf16 (its row index) to y[row], the M = 1 GEMV's output pattern;
// without it nothing is stored.  Back-to-back launches time the fixed cost
// of a dispatch of the given grid, with and without the GEMV's row stores.
__global__ void __launch_bounds__(1024) empty_probe_kernel(uint16_t* y) {
    const int tid = (int)threadIdx.x;
    if (y != nullptr && (tid & 15) == 0) {
        const int row = ((int)blockIdx.x * (int)blockDim.x + tid) >> 4;
        y[row] = (uint16_t)row;
    }
}

// Warms a byte range into the memory-side cache (MALL): workgroup b reads
// chunk b of the range with plain (allocating) 16-byte loads, PF_LOADS per
// thread in flight per round, and folds the words so the loads stay live
// (the fold reaches memory only in the never-expected case that it equals a
// magic word).  Launched on its own stream next to the kernels that run now,
// it reads the weights the next launches will stream.
constexpr int PF_NT = 256, PF_LOADS = 16;
__global__ void __launch_bounds__(PF_NT) prefetch_kernel(const uint8_t* p, uint64_t bytes, uint64_t chunk,
                                                         uint32_t* sink) {
    const uint64_t lo = (uint64_t)blockIdx.x * chunk;
    const uint64_t hi = lo + chunk < bytes ? lo + chunk : bytes;
    uint32_t f = 0;
    for (uint64_t base = lo; base < hi; base += (uint64_t)PF_NT * PF_LOADS * 16) {
        const uint64_t n = hi - base;
        const auto r = buf(p + base, (uint32_t)(n < 0xFFFFFFF0ull ? n : 0xFFFFFFF0ull));
        u32x4 v[PF_LOADS];
#pragma unroll
        for (int j = 0; j < PF_LOADS; ++j) v[j] = bload16(r, (j * PF_NT + (int)threadIdx.x) * 16);
#pragma unroll
        for (int j = 0; j < PF_LOADS; ++j) f ^= v[j].x ^ v[j].y ^ v[j].z ^ v[j].w;
    }
    if (f == 0x9E3779B9u && sink != nullptr) sink[0] = f;
}

}  // namespace vq

extern "C" int viper_hip_prefetch(const void* buf, size_t bytes, int workgroups, uint32_t* sink, void* stream) {
    if (buf == nullptr || sink == nullptr || bytes == 0 || workgroups <= 0 || workgroups > 65536)
        return VIPER_INVALID_ARGUMENT;
    if (vq::misaligned(buf, 16) || vq::misaligned(sink, 4) || bytes % 16 != 0) return VIPER_INVALID_ARGUMENT;
    const uint8_t* a0 = (const uint8_t*)buf;
    uint64_t a1 = bytes;
    uint64_t chunk = (bytes + (uint64_t)workgroups - 1) / (uint64_t)workgroups;
    chunk = (chunk + 15) / 16 * 16;
    void* args[] = {&a0, &a1, &chunk, &sink};
    vq::launch((const void*)vq::prefetch_kernel, (unsigned)workgroups, vq::PF_NT, 0, (hipStream_t)stream, args);
    return vq::status_of(hipGetLastError());
}

extern "C" int viper_hip_empty_dispatch(int workgroups, int threads, void* y_bf16, void* stream) {
    if (workgroups <= 0 || workgroups > 65536 || threads <= 0 || threads > 1024 || threads % 64 != 0)
        return VIPER_INVALID_ARGUMENT;
    if (vq::misaligned(y_bf16, 2)) return VIPER_INVALID_ARGUMENT;
    uint16_t* a0 = (uint16_t*)y_bf16;
    void* args[] = {&a0};
    vq::launch((const void*)vq::empty_probe_kernel, (unsigned)workgroups, (unsigned)threads, 0, (hipStream_t)stream,
               args);
    return vq::status_of(hipGetLastError());
}

extern "C" int viper_hip_clock_stamp(uint64_t* out, void* stream) {
    if (out == nullptr || vq::misaligned(out, 8)) return VIPER_INVALID_ARGUMENT;
    void* args[] = {&out};
    vq::launch((const void*)vq::clock_stamp_kernel, 1, 64, 0, (hipStream_t)stream, args);
    return vq::status_of(hipGetLastError());
}

extern "C" int viper_hip_stream_read(const void* buf, size_t bytes, int threads, int loads, const void* side,
                                     int side_bytes, void* y_bf16, uint32_t* sink, void* stream) {
    const vq::probe_fn fn = vq::probe_kernel(threads, loads);
    if (fn == nullptr || buf == nullptr || sink == nullptr) return VIPER_INVALID_ARGUMENT;
    const size_t per_wg = (size_t)threads * (size_t)loads * 16;
    if (bytes == 0 || bytes % per_wg != 0 || bytes / per_wg > (size_t)INT32_MAX) return VIPER_INVALID_ARGUMENT;
    if (vq::misaligned(buf, 16) || vq::misaligned(sink, 4) || vq::misaligned(y_bf16, 2) || vq::misaligned(side, 16))
        return VIPER_INVALID_ARGUMENT;
    if (side_bytes < 0 || side_bytes % 16 != 0 || side_bytes > 16 * threads || (side_bytes > 0) != (side != nullptr))
        return VIPER_INVALID_ARGUMENT;
    const unsigned grid = (unsigned)(bytes / per_wg);
    const uint8_t* a0 = (const uint8_t*)buf;
    uint16_t* a1 = (uint16_t*)y_bf16;
    const uint8_t* a3 = (const uint8_t*)side;
    void* args[] = {&a0, &a1, &sink, &a3, &side_bytes};
    vq::launch((const void*)fn, grid, (unsigned)threads, 0, (hipStream_t)stream, args);
    return vq::status_of(hipGetLastError());
}
