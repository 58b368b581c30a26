// dtype helpers (reference src/viper/tensor.cpp:8-40).
#include "viper/tensor.h"

namespace viper {

const char* dtype_name(DType d) noexcept {
    switch (d) {
        case DType::FP32: return "FP32";
        case DType::BF16: return "BF16";
        case DType::FP16: return "FP16";
        case DType::INT8: return "INT8";
        case DType::UINT8: return "UINT8";
        case DType::INT32: return "INT32";
        case DType::UINT32: return "UINT32";
        case DType::Q4_G64: return "Q4_G64";
        case DType::Q5_G64: return "Q5_G64";
        case DType::Q6_G64: return "Q6_G64";
        case DType::W8_G32: return "W8_G32";
    }
    return "UNKNOWN";
}

usize dtype_sizeof(DType d) noexcept {
    switch (d) {
        case DType::FP32:
        case DType::INT32:
        case DType::UINT32: return 4;
        case DType::BF16:
        case DType::FP16: return 2;
        case DType::INT8:
        case DType::UINT8:
        // packed formats: one byte per storage unit, per-element size varies
        case DType::Q4_G64:
        case DType::Q5_G64:
        case DType::Q6_G64:
        case DType::W8_G32: return 1;
    }
    return 0;
}

}  // namespace viper
