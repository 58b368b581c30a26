// Host API checks that need no GPU: the closed registry (reference
// src/viper/quant.cpp:6-20, src/viper/tensor.cpp:8-40) and the Status codes
// linear() returns for bad arguments before any device work (reference
// src/viper/linear.cpp:16-36; argument rules as kernels/ops/linear_multim.cu:152).
#include <cstdio>
#include <string>
#include <unistd.h>

#include "artifact_writer.h"
#include "viper/artifact.h"
#include "viper/ops.h"
#include "viper/quant.h"
#include "viper/tensor.h"

using namespace viper;

static int failures = 0;
#define EXPECT(cond)                                                            \
    do {                                                                        \
        if (!(cond)) {                                                          \
            std::printf("FAIL %s:%d: %s\n", __FILE__, __LINE__, #cond);         \
            ++failures;                                                         \
        }                                                                       \
    } while (0)

int main() {
    using quant::QType;
    EXPECT(quant::qtype_name(QType::BF16) == "BF16");
    EXPECT(quant::qtype_name(QType::FP32) == "FP32");
    EXPECT(quant::qtype_name(QType::Q4_G64) == "Q4_G64");
    EXPECT(quant::qtype_name(QType::Q5_G64) == "Q5_G64");
    EXPECT(quant::qtype_name(QType::Q6_G64) == "Q6_G64");
    EXPECT(quant::qtype_name(QType::W8_G32) == "W8_G32");
    EXPECT(quant::qtype_name(static_cast<QType>(3)) == "UNKNOWN");
    EXPECT(quant::is_lossless(QType::BF16) && quant::is_lossless(QType::FP32));
    EXPECT(!quant::is_lossless(QType::Q4_G64) && !quant::is_lossless(QType::W8_G32));
    EXPECT(static_cast<int>(QType::Q4_G64) == 4 && static_cast<int>(QType::W8_G32) == 8);
    EXPECT(static_cast<int>(DType::Q4_G64) == 100 && static_cast<int>(DType::W8_G32) == 103);
    EXPECT(std::string(dtype_name(DType::Q6_G64)) == "Q6_G64");
    EXPECT(dtype_sizeof(DType::Q4_G64) == 1 && dtype_sizeof(DType::BF16) == 2);
    EXPECT(quant::group_size(QType::Q5_G64) == 64 && quant::group_size(QType::W8_G32) == 32);
    EXPECT(quant::packed_bytes(QType::Q4_G64, 10240, 2560) == 13107200);
    EXPECT(quant::packed_bytes(QType::Q5_G64, 4, 64) == 4 * 32 + 4 * 8);
    EXPECT(quant::packed_bytes(QType::Q6_G64, 4, 64) == 4 * 32 + 4 * 16);
    EXPECT(quant::packed_bytes(QType::W8_G32, 4, 64) == 256);
    EXPECT(quant::packed_bytes(QType::Q4_G64, 4, 96) == 0);

    // argument validation: pointers are fake and never dereferenced
    void* fake = reinterpret_cast<void*>(0x10000);
    quant::QuantizedWeight w{QType::Q4_G64, fake, fake, 64, 128, 64, quant::ScaleEnc::FP16};
    Tensor x(fake, DType::BF16, {128});
    Tensor y(fake, DType::BF16, {64});
    auto code = [&](const quant::QuantizedWeight& ww, const Tensor& xx, Tensor& yy) {
        return ops::linear(ww, xx, yy).code();
    };
    quant::QuantizedWeight wb = w;
    wb.qtype = QType::BF16;
    EXPECT(code(wb, x, y) == StatusCode::UNIMPLEMENTED);
    wb.qtype = static_cast<QType>(7);
    EXPECT(code(wb, x, y) == StatusCode::INVALID_ARGUMENT);
    wb = w;
    wb.group_size = 32;
    EXPECT(code(wb, x, y) == StatusCode::INVALID_ARGUMENT);
    wb = w;
    wb.cols = 96;
    Tensor x96(fake, DType::BF16, {96});
    EXPECT(code(wb, x96, y) == StatusCode::SHAPE_MISMATCH);
    wb = w;
    wb.data = nullptr;
    EXPECT(code(wb, x, y) == StatusCode::INVALID_ARGUMENT);
    Tensor xf(fake, DType::FP32, {128});
    EXPECT(code(w, xf, y) == StatusCode::INVALID_ARGUMENT);
    Tensor xw(fake, DType::BF16, {100});
    EXPECT(code(w, xw, y) == StatusCode::SHAPE_MISMATCH);
    Tensor y2(fake, DType::BF16, {2, 64});
    EXPECT(code(w, x, y2) == StatusCode::SHAPE_MISMATCH);
    Tensor x17(fake, DType::BF16, {17, 128});
    Tensor y17(fake, DType::BF16, {17, 64});
    EXPECT(code(w, x17, y17) == StatusCode::INVALID_ARGUMENT);
    Tensor x4(fake, DType::BF16, {4, 128});
    Tensor y4(fake, DType::BF16, {4, 64});
    EXPECT(code(w, x4, y4) == StatusCode::INVALID_ARGUMENT);  // no workspace
    EXPECT(ops::linear_workspace_bytes(w, 1) == 0);
    EXPECT(ops::linear_workspace_bytes(w, 4) == 256 + 4 * 1024 + 16 * 128 + 2 * 16 * 4);  // control words and counters, xq, xs for 16 rows
    Tensor misaligned(reinterpret_cast<void*>(0x10008), DType::BF16, {128});
    EXPECT(code(w, misaligned, y) == StatusCode::INVALID_ARGUMENT);
    // lossy dtypes through the Tensor overload: UNIMPLEMENTED, as the
    // reference's switch returns (src/viper/linear.cpp:26-32)
    for (DType dt : {DType::Q4_G64, DType::Q5_G64, DType::Q6_G64, DType::W8_G32}) {
        Tensor wt(fake, dt, {64, 128});
        EXPECT(ops::linear_forward(wt, Tensor(), x, y).code() == StatusCode::UNIMPLEMENTED);
    }
    // the six fields of the reference's QuantizedWeight leave the encoding at
    // bf16, what its converter writes
    {
        quant::QuantizedWeight r;
        EXPECT(r.scale_enc == quant::ScaleEnc::BF16);
    }
    Tensor wbf(fake, DType::BF16, {64, 128});
    EXPECT(ops::linear_forward(wbf, Tensor(), x, y).code() == StatusCode::UNIMPLEMENTED);
    Tensor wi(fake, DType::INT32, {64, 128});
    EXPECT(ops::linear_forward(wi, Tensor(), x, y).code() == StatusCode::INVALID_ARGUMENT);
    Tensor xq(fake, DType::INT8, {128}), xs(fake, DType::FP32, {2});
    EXPECT(ops::quantize_activations(x, 48, xq, xs).code() == StatusCode::INVALID_ARGUMENT);
    EXPECT(ops::quantize_activations(x, 64, xq, y).code() == StatusCode::INVALID_ARGUMENT);

    // .viper v1 artifact: index, offsets and every rejection path
    {
        namespace A = artifact;
        ArtifactDims d;
        std::vector<uint8_t> f = write_artifact(d, hash_fill);
        A::Index idx;
        EXPECT(A::parse(f.data(), f.size(), &idx).ok());
        EXPECT(idx.header.version == 1 && idx.header.n_layers == 2 && idx.header.hidden == 128 &&
               idx.header.vocab == 300);
        EXPECT(idx.layers.size() == 2 && idx.norms.size() == 2);
        EXPECT(idx.layers[1][A::DOWN].rows == 128 && idx.layers[1][A::DOWN].cols == 256);
        EXPECT(idx.layers[0][A::K].rows == 64 && idx.layers[0][A::O].cols == 128);
        EXPECT(idx.layers[0][A::Q].packed.offset == A::kHeaderBytes + 8);
        std::vector<uint8_t> want;
        hash_fill("up_proj.scales", 1, 256 * 2 * 2, want);
        const A::Blob& b = idx.layers[1][A::UP].scales;
        EXPECT(b.size == want.size() && std::memcmp(f.data() + b.offset, want.data(), want.size()) == 0);
        hash_fill("post_attention_layernorm", 0, 256, want);
        EXPECT(std::memcmp(f.data() + idx.norms[0][1].offset, want.data(), 256) == 0);
        hash_fill("lm_head", -1, 300 * 64, want);
        EXPECT(std::memcmp(f.data() + idx.lm_head.packed.offset, want.data(), want.size()) == 0);

        std::vector<uint8_t> g = f;
        g[2] = 'x';
        EXPECT(A::parse(g.data(), g.size(), &idx).code() == StatusCode::INVALID_ARGUMENT);
        g = write_artifact(d, hash_fill, 2);
        EXPECT(A::parse(g.data(), g.size(), &idx).code() == StatusCode::INVALID_ARGUMENT);
        EXPECT(A::parse(f.data(), f.size() - 1, &idx).code() == StatusCode::IO_ERROR);
        EXPECT(A::parse(f.data(), 40, &idx).code() == StatusCode::IO_ERROR);
        g = f;
        g.push_back(0);
        EXPECT(A::parse(g.data(), g.size(), &idx).code() == StatusCode::IO_ERROR);
        // one section a byte short (of the right total length): its size field disagrees
        auto short_fill = [](const std::string& name, int layer, size_t bytes, std::vector<uint8_t>& out) {
            hash_fill(name, layer, bytes, out);
            if (name == "k_proj.scales" && layer == 1) out.pop_back();
        };
        g = write_artifact(d, short_fill);
        EXPECT(A::parse(g.data(), g.size(), &idx).code() == StatusCode::INVALID_ARGUMENT);
        // header products past INT32_MAX (n_heads * head_dim here): a wrapped
        // section size would let a few-KB file parse into views ~137 GB past
        // its end; the parser rejects the header instead
        {
            std::vector<uint8_t> bad(A::kHeaderBytes + 8192, 0);
            std::memcpy(bad.data(), "VIPER", 5);
            const uint32_t hdr[10] = {1, 1, 1, 192, 64, 1596634768u, 1596634768u, 3851171736u, 64, 16};
            std::memcpy(bad.data() + 16, hdr, sizeof hdr);
            EXPECT(A::parse(bad.data(), bad.size(), &idx).code() == StatusCode::INVALID_ARGUMENT);
            const uint32_t big[10] = {1, 1, 1, 0x80000000u, 64, 1, 1, 64, 64, 16};  // hidden > INT32_MAX
            std::memcpy(bad.data() + 16, big, sizeof big);
            EXPECT(A::parse(bad.data(), bad.size(), &idx).code() == StatusCode::INVALID_ARGUMENT);
        }
        // untrusted layer / pass counts: a bare 56-byte header (and one with a
        // few KB after it) claiming 2^32 - 1 layers must come back as a
        // Status before anything is sized by that count (no throw)
        {
            const uint32_t many[10] = {1, 0xFFFFFFFFu, 1, 128, 256, 2, 1, 64, 300, 16};
            const uint32_t passes[10] = {1, 2, 0xFFFFFFFFu, 128, 256, 2, 1, 64, 300, 16};
            for (const uint32_t* h : {many, passes})
                for (const size_t extra : {(size_t)0, (size_t)8192}) {
                    std::vector<uint8_t> bad(A::kHeaderBytes + extra, 0);
                    std::memcpy(bad.data(), "VIPER", 5);
                    std::memcpy(bad.data() + 16, h, 40);
                    bool threw = false;
                    StatusCode c = StatusCode::OK;
                    try {
                        c = A::parse(bad.data(), bad.size(), &idx).code();
                    } catch (...) {
                        threw = true;
                    }
                    EXPECT(!threw && c == StatusCode::IO_ERROR);
                    EXPECT(idx.layers.empty() && idx.norms.empty());
                }
        }
        ArtifactDims odd = d;
        odd.hidden = 96;  // not a multiple of the 64-group
        g = write_artifact(odd, hash_fill);
        EXPECT(A::parse(g.data(), g.size(), &idx).code() == StatusCode::INVALID_ARGUMENT);

        char path[] = "/tmp/viper_artifact_XXXXXX";
        const int fd = mkstemp(path);
        EXPECT(fd >= 0 && write(fd, f.data(), f.size()) == (ssize_t)f.size());
        close(fd);
        {
            A::MappedFile mf;
            EXPECT(mf.open(path).ok() && mf.size() == f.size());
            EXPECT(A::parse(mf.data(), mf.size(), &idx).ok());
        }
        unlink(path);
        A::MappedFile missing;
        EXPECT(missing.open("/nonexistent/model.viper").code() == StatusCode::IO_ERROR);
    }

    std::printf("%s (%d failures)\n", failures ? "FAILED" : "PASS", failures);
    return failures ? 1 : 0;
}
