// Format registry helpers (reference src/viper/quant.cpp:6-20, plus the
// layout facts this build freezes for Q5/Q6/W8).
#include "viper/quant.h"

namespace viper::quant {

std::string_view qtype_name(QType q) noexcept {
    switch (q) {
        case QType::BF16: return "BF16";
        case QType::FP32: return "FP32";
        case QType::Q4_G64: return "Q4_G64";
        case QType::Q5_G64: return "Q5_G64";
        case QType::Q6_G64: return "Q6_G64";
        case QType::W8_G32: return "W8_G32";
    }
    return "UNKNOWN";
}

bool is_lossless(QType q) noexcept { return q == QType::BF16 || q == QType::FP32; }

i32 group_size(QType q) noexcept {
    switch (q) {
        case QType::Q4_G64:
        case QType::Q5_G64:
        case QType::Q6_G64: return 64;
        case QType::W8_G32: return 32;
        default: return 0;
    }
}

usize packed_bytes(QType q, i64 rows, i64 cols) noexcept {
    const i32 g = group_size(q);
    if (g == 0 || rows <= 0 || cols <= 0 || cols % g != 0) return 0;
    const usize n = static_cast<usize>(rows) * static_cast<usize>(cols);
    switch (q) {
        case QType::Q4_G64: return n / 2;
        case QType::Q5_G64: return n / 2 + n / 8;
        case QType::Q6_G64: return n / 2 + n / 4;
        case QType::W8_G32: return n;
        default: return 0;
    }
}

DType dtype_of(QType q) noexcept {
    switch (q) {
        case QType::BF16: return DType::BF16;
        case QType::FP32: return DType::FP32;
        case QType::Q4_G64: return DType::Q4_G64;
        case QType::Q5_G64: return DType::Q5_G64;
        case QType::Q6_G64: return DType::Q6_G64;
        case QType::W8_G32: return DType::W8_G32;
    }
    return DType::FP32;
}

}  // namespace viper::quant
