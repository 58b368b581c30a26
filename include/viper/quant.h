// Closed weight-format registry.  linear() is a switch on w.qtype, never a
// generic backend (reference include/viper/quant.h:1-50).
//
// Lossless: BF16, FP32.  Lossy: Q4_G64, Q5_G64, Q6_G64, W8_G32.
//
// Packed layouts (device memory, one matrix of `rows` outputs x `cols`
// inputs; the reference fixes Q4_G64 in tools/convert/convert.cpp:91-127 and
// leaves Q5/Q6/W8 undefined, so this build freezes them):
//   Q4_G64  [rows][cols/2]: k even in the low nibble, k odd in the high one;
//           nibble = w + 8, w in [-8, 7].
//   Q5_G64  low plane [rows][cols/2] of (w+16) & 15 as Q4, then high plane
//           [rows][cols/8]: per 32-weight chunk a little-endian u32 holding
//           bit 4 of (w+16) for weight 8i+2b+p at bit 8b+2i+p.
//   Q6_G64  low plane as Q5 with w+32, then high plane [rows][cols/4]: per
//           chunk two u32; word i/2 holds bits 4..5 at bit 8b+4(i%2)+2p.
//   W8_G32  [rows][cols] int8, w in [-127, 127].
//   scales  [rows][cols/group_size] 16-bit per group, fp16 or bf16
//           (scale_enc); the reference's converter writes bf16 by
//           truncation (convert.cpp:109-113), its headers say fp16.
#pragma once

#include <string_view>

#include "viper/common.h"
#include "viper/tensor.h"

namespace viper::quant {

enum class QType : int {
    BF16 = 0,    // lossless
    FP32 = 1,    // lossless
    Q4_G64 = 4,  // lossy
    Q5_G64 = 5,  // lossy
    Q6_G64 = 6,  // lossy
    W8_G32 = 8,  // lossy
};

enum class ScaleEnc : int { FP16 = 0, BF16 = 1 };

std::string_view qtype_name(QType q) noexcept;
bool is_lossless(QType q) noexcept;

// Quantization group of a lossy format (64, or 32 for W8_G32); 0 otherwise.
i32 group_size(QType q) noexcept;
// Bytes of the packed weight array for rows x cols (0 for lossless or an
// invalid shape).
usize packed_bytes(QType q, i64 rows, i64 cols) noexcept;
// The tensor dtype that names a format (Q4_G64 -> DType::Q4_G64, ...).
DType dtype_of(QType q) noexcept;

// Device view of one quantized matrix (reference quant.h:34-41) plus the
// scale encoding, which the reference leaves implicit.  The encoding defaults
// to bf16, what the reference's converter writes (convert.cpp:109-113) and
// its engine decodes (dp4a_smem_kernel.cu:27,61), so a caller that fills only
// the reference's six fields over reference-converted weights decodes them
// correctly; fp16 scales (BASELINE's synthetic weights) must be stated.
struct QuantizedWeight {
    QType qtype = QType::BF16;
    void* data = nullptr;    // device pointer to packed weights
    void* scales = nullptr;  // device pointer to per-group scales
    i32 rows = 0;            // output channels (N)
    i32 cols = 0;            // input channels (K)
    i32 group_size = 64;     // 64 for Q*_G64, 32 for W8_G32
    ScaleEnc scale_enc = ScaleEnc::BF16;
};

// Lossy-vs-lossless delta report (reference quant.h:44-50).
struct QualityDelta {
    f64 max_abs_err = 0.0;
    f64 mean_abs_err = 0.0;
    f64 kl_divergence = 0.0;
    i32 oracle_vocab = 166144;
    i32 oracle_tokens = 0;
};

}  // namespace viper::quant
