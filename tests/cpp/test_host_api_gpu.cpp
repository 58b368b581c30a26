// GPU parity of the C++ host API (viper::ops) against the CPU oracle: every
// format and scale encoding through linear() at M = 1 (fused quantize) and
// M = 4 (workspace), quantize_activations() bit-exact, and
// linear_prequantized() with a residual.  bf16 outputs must be within 1 bf16
// ulp of the oracle or within 1e-5 * sum|group terms|.
#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdio>
#include <cstring>
#include <vector>

#include "artifact_writer.h"
#include "viper/artifact.h"
#include "viper/ops.h"
#include "viper_oracle.h"

using namespace viper;

static int failures = 0;
#define CHECK_HIP(x)                                                                        \
    do {                                                                                    \
        hipError_t e_ = (x);                                                                \
        if (e_ != hipSuccess) {                                                             \
            std::printf("HIP error %s at %s:%d\n", hipGetErrorString(e_), __FILE__, __LINE__); \
            return 2;                                                                       \
        }                                                                                   \
    } while (0)

template <typename T>
static T* upload(const std::vector<T>& h) {
    T* d = nullptr;
    if (hipMalloc(&d, h.size() * sizeof(T) + 16) != hipSuccess) return nullptr;
    if (hipMemcpy(d, h.data(), h.size() * sizeof(T), hipMemcpyHostToDevice) != hipSuccess) return nullptr;
    return d;
}

static double ulp_bf16(uint16_t h) {
    double f = std::fabs((double)vo_bf16_to_f32(h));
    double e = std::floor(std::log2(std::fmax(f, std::ldexp(1.0, -126))));
    return std::ldexp(1.0, (int)e - 7);
}

static bool close_bf16(const std::vector<uint16_t>& g, const std::vector<uint16_t>& r,
                       const std::vector<double>& absterm, const char* what) {
    int bad = 0;
    for (size_t i = 0; i < g.size(); ++i) {
        double d = std::fabs((double)vo_bf16_to_f32(g[i]) - (double)vo_bf16_to_f32(r[i]));
        double tol = std::fmax(std::fmax(ulp_bf16(r[i]), ulp_bf16(g[i])), 1e-5 * absterm[i]);
        if (!(d <= tol)) {
            if (bad < 3) std::printf("  %s[%zu]: gpu %g ref %g\n", what, i, vo_bf16_to_f32(g[i]), vo_bf16_to_f32(r[i]));
            ++bad;
        }
    }
    if (bad) std::printf("FAIL %s: %d of %zu outside tolerance\n", what, bad, g.size());
    return bad == 0;
}

static int run_case(int qt, int senc, int N, int K, int M, uint64_t seed) {
    const int G = vo_group_size(qt);
    std::vector<uint8_t> packed(vo_packed_bytes(qt, N, K));
    std::vector<uint16_t> scales((size_t)N * (K / G));
    vo_gen_weights(qt, N, K, seed, senc, packed.data(), scales.data());
    std::vector<uint16_t> x((size_t)M * K), res((size_t)M * N);
    vo_gen_act(M, K, seed + 1, 0.05, 20.0f, x.data());
    vo_gen_act(M, N, seed + 2, 0.0, 1.0f, res.data());
    std::vector<uint16_t> yref((size_t)M * N), yref_r((size_t)M * N);
    std::vector<float> yf((size_t)M * N);
    std::vector<double> ya((size_t)M * N), ya_r((size_t)M * N);
    vo_qlinear(qt, packed.data(), scales.data(), senc, N, K, x.data(), M, nullptr, yref.data(), yf.data(), ya.data());
    vo_qlinear(qt, packed.data(), scales.data(), senc, N, K, x.data(), M, res.data(), yref_r.data(), yf.data(), ya_r.data());

    uint8_t* dw = upload(packed);
    uint16_t* ds = upload(scales);
    uint16_t* dx = upload(x);
    uint16_t* dr = upload(res);
    uint16_t* dy = nullptr;
    CHECK_HIP(hipMalloc(&dy, (size_t)M * N * 2));
    if (!dw || !ds || !dx || !dr) return 2;

    quant::QuantizedWeight w{static_cast<quant::QType>(qt), dw, ds, N, K, G,
                             static_cast<quant::ScaleEnc>(senc)};
    Tensor tx = M == 1 ? Tensor(dx, DType::BF16, {K}) : Tensor(dx, DType::BF16, {M, K});
    Tensor ty = M == 1 ? Tensor(dy, DType::BF16, {N}) : Tensor(dy, DType::BF16, {M, N});
    Tensor tr = M == 1 ? Tensor(dr, DType::BF16, {N}) : Tensor(dr, DType::BF16, {M, N});
    const usize nws = ops::linear_workspace_bytes(w, M);
    void* dws = nullptr;
    if (nws) {
        CHECK_HIP(hipMalloc(&dws, nws));
        CHECK_HIP(hipMemset(dws, 0, nws));  // zero before first use
    }
    ops::LinearOptions opt;
    opt.workspace = dws;
    opt.workspace_bytes = nws;

    char what[96];
    std::snprintf(what, sizeof what, "linear q%d senc%d N%d K%d M%d", qt, senc, N, K, M);
    std::printf("case %s\n", what);
    std::fflush(stdout);
    Status st = ops::linear(w, tx, ty, opt);
    if (!st.ok()) {
        std::printf("FAIL %s: status %d %.*s\n", what, (int)st.code(), (int)st.message().size(), st.message().data());
        return 1;
    }
    CHECK_HIP(hipDeviceSynchronize());
    std::vector<uint16_t> yg((size_t)M * N);
    CHECK_HIP(hipMemcpy(yg.data(), dy, yg.size() * 2, hipMemcpyDeviceToHost));
    int fails = close_bf16(yg, yref, ya, what) ? 0 : 1;

    // residual through the same call
    opt.residual = &tr;
    st = ops::linear(w, tx, ty, opt);
    if (!st.ok()) return 1;
    CHECK_HIP(hipDeviceSynchronize());
    CHECK_HIP(hipMemcpy(yg.data(), dy, yg.size() * 2, hipMemcpyDeviceToHost));
    fails += close_bf16(yg, yref_r, ya_r, "linear+residual") ? 0 : 1;

    // quantize_activations bit-exact, then linear_prequantized
    std::vector<int8_t> xq_ref((size_t)M * K);
    std::vector<float> xs_ref((size_t)M * (K / G));
    vo_quantize_act(x.data(), M, K, G, xq_ref.data(), xs_ref.data());
    int8_t* dxq = nullptr;
    float* dxs = nullptr;
    CHECK_HIP(hipMalloc(&dxq, xq_ref.size()));
    CHECK_HIP(hipMalloc(&dxs, xs_ref.size() * 4));
    Tensor tq(dxq, DType::INT8, {M, K}), ts(dxs, DType::FP32, {M, K / G});
    st = ops::quantize_activations(tx, G, tq, ts);
    if (!st.ok()) return 1;
    CHECK_HIP(hipDeviceSynchronize());
    std::vector<int8_t> xq_g(xq_ref.size());
    std::vector<float> xs_g(xs_ref.size());
    CHECK_HIP(hipMemcpy(xq_g.data(), dxq, xq_g.size(), hipMemcpyDeviceToHost));
    CHECK_HIP(hipMemcpy(xs_g.data(), dxs, xs_g.size() * 4, hipMemcpyDeviceToHost));
    if (std::memcmp(xq_g.data(), xq_ref.data(), xq_g.size()) || std::memcmp(xs_g.data(), xs_ref.data(), xs_g.size() * 4)) {
        std::printf("FAIL quantize_activations not bit-exact\n");
        ++fails;
    }
    ops::LinearOptions po;
    po.residual = &tr;
    st = ops::linear_prequantized(w, tq, ts, ty, po);
    if (!st.ok()) return 1;
    CHECK_HIP(hipDeviceSynchronize());
    CHECK_HIP(hipMemcpy(yg.data(), dy, yg.size() * 2, hipMemcpyDeviceToHost));
    fails += close_bf16(yg, yref_r, ya_r, "linear_prequantized+residual") ? 0 : 1;

    for (void* p : {(void*)dw, (void*)ds, (void*)dx, (void*)dr, (void*)dy, (void*)dxq, (void*)dxs, dws})
        if (p) (void)hipFree(p);
    return fails;
}

// A synthetic .viper artifact with real Q4 data (oracle weights with bf16
// scales) is parsed and uploaded; linears run from the uploaded views and
// the bf16 sections read back byte for byte.
static int artifact_case() {
    namespace A = artifact;
    std::printf("case artifact upload\n");
    std::fflush(stdout);
    ArtifactDims d;
    auto fill = [&](const std::string& name, int layer, size_t bytes, std::vector<uint8_t>& out) {
        const bool scales = name.size() > 7 && name.compare(name.size() - 7, 7, ".scales") == 0;
        const std::string base = scales ? name.substr(0, name.size() - 7) : name;
        const bool linear = base != "embed" && base != "final_norm" && base != "input_layernorm" &&
                            base != "post_attention_layernorm";
        if (!linear) {
            hash_fill(name, layer, bytes, out);
            for (size_t i = 1; i < bytes; i += 2) out[i] &= 0x3f;  // finite bf16 bit patterns
            return;
        }
        // rows x cols from the byte counts: packed = rows*cols/2, scales = rows*(cols/64)*2
        int rows, cols;
        if (base == "q_proj") rows = 128, cols = 128;
        else if (base == "k_proj" || base == "v_proj") rows = 64, cols = 128;
        else if (base == "o_proj") rows = 128, cols = 128;
        else if (base == "gate_proj" || base == "up_proj") rows = 256, cols = 128;
        else if (base == "down_proj") rows = 128, cols = 256;
        else rows = 300, cols = 128;  // lm_head
        std::vector<uint8_t> packed((size_t)rows * cols / 2);
        std::vector<uint16_t> sc((size_t)rows * (cols / 64));
        const uint64_t seed = 0xA0000 + (uint64_t)(layer + 1) * 16 + (uint64_t)(base.size() * 131 + base[0]);
        vo_gen_weights(VO_Q4_G64, rows, cols, seed, VO_SCALE_BF16, packed.data(), sc.data());
        if (scales) out.assign((const uint8_t*)sc.data(), (const uint8_t*)sc.data() + sc.size() * 2);
        else out = packed;
        if (out.size() != bytes) std::printf("FAIL artifact writer size %s\n", name.c_str());
    };
    std::vector<uint8_t> f = write_artifact(d, fill);
    A::Index idx;
    Status st = A::parse(f.data(), f.size(), &idx);
    if (!st.ok()) {
        std::printf("FAIL artifact parse\n");
        return 1;
    }
    A::DeviceModel dm;
    st = A::upload(f.data(), idx, &dm);
    if (!st.ok()) {
        std::printf("FAIL artifact upload: %.*s\n", (int)st.message().size(), st.message().data());
        return 1;
    }
    int fails = 0;
    // every view 256-byte aligned
    for (auto& layer : dm.layers)
        for (auto& w : layer)
            if (((uintptr_t)w.data & 255) || ((uintptr_t)w.scales & 255)) ++fails;
    // linears from the uploaded views
    struct Pick {
        quant::QuantizedWeight w;
        const A::LinearBlob* b;
    };
    const Pick picks[] = {{dm.layers[0][A::Q], &idx.layers[0][A::Q]},
                          {dm.layers[1][A::DOWN], &idx.layers[1][A::DOWN]},
                          {dm.lm_head, &idx.lm_head}};
    for (const Pick& pk : picks) {
        const int N = pk.w.rows, K = pk.w.cols;
        std::vector<uint16_t> x(K), yref(N);
        std::vector<float> yf(N);
        std::vector<double> ya(N);
        vo_gen_act(1, K, 77 + N, 0.0, 1.0f, x.data());
        vo_qlinear(VO_Q4_G64, f.data() + pk.b->packed.offset, (const uint16_t*)(f.data() + pk.b->scales.offset),
                   VO_SCALE_BF16, N, K, x.data(), 1, nullptr, yref.data(), yf.data(), ya.data());
        uint16_t* dx = upload(x);
        uint16_t* dy = nullptr;
        CHECK_HIP(hipMalloc(&dy, (size_t)N * 2));
        Tensor tx(dx, DType::BF16, {K}), ty(dy, DType::BF16, {N});
        st = ops::linear(pk.w, tx, ty);
        if (!st.ok()) return 1;
        CHECK_HIP(hipDeviceSynchronize());
        std::vector<uint16_t> yg(N);
        CHECK_HIP(hipMemcpy(yg.data(), dy, (size_t)N * 2, hipMemcpyDeviceToHost));
        fails += close_bf16(yg, yref, ya, "artifact linear") ? 0 : 1;
        (void)hipFree(dx);
        (void)hipFree(dy);
    }
    // bf16 sections round trip
    auto same = [&](const void* dptr, const A::Blob& b) {
        std::vector<uint8_t> h(b.size);
        if (hipMemcpy(h.data(), dptr, b.size, hipMemcpyDeviceToHost) != hipSuccess) return false;
        return std::memcmp(h.data(), f.data() + b.offset, b.size) == 0;
    };
    if (!same(dm.embed, idx.embed) || !same(dm.final_norm, idx.final_norm) ||
        !same(dm.norms[1][0], idx.norms[1][0]) || !same(dm.norms[0][1], idx.norms[0][1])) {
        std::printf("FAIL artifact bf16 sections\n");
        ++fails;
    }
    if (!A::release(&dm).ok() || dm.arena != nullptr) ++fails;
    return fails;
}

// A weight described by the reference's six fields only (quant.h:34-41:
// qtype, data, scales, rows, cols, group_size) over bf16 scales, the
// converter's encoding (convert.cpp:109-113): the default encoding must
// decode them, for every format and both the fused M = 1 and multi-row paths.
int reference_fields_case(int qt, int M) {
    const int N = 257, K = 2560, G = vo_group_size(qt);
    std::vector<uint8_t> packed(vo_packed_bytes(qt, N, K));
    std::vector<uint16_t> scales((size_t)N * (K / G));
    vo_gen_weights(qt, N, K, 0xB16u + qt, VO_SCALE_BF16, packed.data(), scales.data());
    std::vector<uint16_t> x((size_t)M * K), yref((size_t)M * N);
    vo_gen_act(M, K, 0xB17u + qt, 0.0, 1.0f, x.data());
    std::vector<float> yf((size_t)M * N);
    std::vector<double> ya((size_t)M * N);
    vo_qlinear(qt, packed.data(), scales.data(), VO_SCALE_BF16, N, K, x.data(), M, nullptr, yref.data(), yf.data(),
               ya.data());
    uint8_t* dw = upload(packed);
    uint16_t* ds = upload(scales);
    uint16_t* dx = upload(x);
    uint16_t* dy = nullptr;
    CHECK_HIP(hipMalloc(&dy, (size_t)M * N * 2));
    quant::QuantizedWeight w;
    w.qtype = static_cast<quant::QType>(qt);
    w.data = dw;
    w.scales = ds;
    w.rows = N;
    w.cols = K;
    w.group_size = G;
    Tensor tx(dx, DType::BF16, {M, K}), ty(dy, DType::BF16, {M, N});
    ops::LinearOptions opt;
    opt.workspace_bytes = ops::linear_workspace_bytes(w, M);
    if (opt.workspace_bytes) {
        CHECK_HIP(hipMalloc(&opt.workspace, opt.workspace_bytes));
        CHECK_HIP(hipMemset(opt.workspace, 0, opt.workspace_bytes));  // zero before first use
    }
    char what[96];
    std::snprintf(what, sizeof what, "reference fields q%d M%d (bf16 scales)", qt, M);
    std::printf("case %s\n", what);
    std::fflush(stdout);
    if (!ops::linear(w, tx, ty, opt).ok()) return 1;
    CHECK_HIP(hipDeviceSynchronize());
    std::vector<uint16_t> yg((size_t)M * N);
    CHECK_HIP(hipMemcpy(yg.data(), dy, yg.size() * 2, hipMemcpyDeviceToHost));
    const int fails = close_bf16(yg, yref, ya, what) ? 0 : 1;
    (void)hipFree(dw);
    (void)hipFree(ds);
    (void)hipFree(dx);
    (void)hipFree(dy);
    if (opt.workspace) (void)hipFree(opt.workspace);
    return fails;
}

int main() {
    failures += artifact_case();
    for (int qt : {VO_Q4_G64, VO_Q5_G64, VO_Q6_G64, VO_W8_G32})
        for (int M : {1, 8}) failures += reference_fields_case(qt, M);
    const int qts[] = {VO_Q4_G64, VO_Q5_G64, VO_Q6_G64, VO_W8_G32};
    for (int qt : qts)
        for (int senc : {0, 1})
            for (int M : {1, 4}) failures += run_case(qt, senc, 300, 2560, M, 0x1234u + qt * 7 + senc + M);
    failures += run_case(VO_Q4_G64, 0, 2560, 10240, 1, 99);
    std::printf("%s (%d failures)\n", failures ? "FAILED" : "PASS", failures);
    return failures ? 1 : 0;
}
