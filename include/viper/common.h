// Scalar aliases of the Viper host API (reference include/viper/common.h:23-37),
// without any GPU runtime header: 16-bit floats travel as their bit patterns.
#pragma once

#include <cstddef>
#include <cstdint>

#include "viper/status.h"

namespace viper {

using i8 = std::int8_t;
using i16 = std::int16_t;
using i32 = std::int32_t;
using i64 = std::int64_t;
using u8 = std::uint8_t;
using u16 = std::uint16_t;
using u32 = std::uint32_t;
using u64 = std::uint64_t;
using usize = std::size_t;
using f32 = float;
using f64 = double;

// bf16 / fp16 values are carried as raw bits on the host side.
using bf16_bits = std::uint16_t;
using fp16_bits = std::uint16_t;

}  // namespace viper
