// Viper operator API for the quantized linear path.  Every op returns Status
// and never throws (reference include/viper/ops.h:1-33).
//
// All tensors are caller-owned device memory (bf16 activations as DType::BF16,
// int8 activations as DType::INT8, scales as DType::FP32).  Calls are
// asynchronous on `stream` (a hipStream_t or nullptr for the null stream)
// and allocate nothing.
#pragma once

#include "viper/common.h"
#include "viper/quant.h"
#include "viper/tensor.h"

namespace viper::ops {

struct LinearOptions {
    const Tensor* residual = nullptr;  // [M, N] bf16 added in fp32 before the bf16 round
    void* workspace = nullptr;         // device scratch for M > 1 (see linear_workspace_bytes), zero-filled
                                       // before its first use, then reused without clearing
    usize workspace_bytes = 0;
    void* stream = nullptr;
};

// y[M, N] = x[M, K] through w: a closed switch on w.qtype.  x and y are bf16
// of shape [K] / [N] (M = 1) or [M, K] / [M, N] with M <= 16.  BF16/FP32
// weights are not on this path (UNIMPLEMENTED).
Status linear(const quant::QuantizedWeight& w, const Tensor& x, Tensor& y);
Status linear(const quant::QuantizedWeight& w, const Tensor& x, Tensor& y,
              const LinearOptions& opt);

// Workspace linear() needs for M activation rows (0 when M == 1).
usize linear_workspace_bytes(const quant::QuantizedWeight& w, i64 M) noexcept;

// xq[M, K] int8 + xs[M, K/group] fp32 from x[M, K] bf16 (reference
// quantize_to_q8, kernels/ops/linear_multim.h:24-26).
Status quantize_activations(const Tensor& x, i32 group, Tensor& xq, Tensor& xs,
                            void* stream = nullptr);

// y from already quantized activations (reference dp4a_smem_gemv /
// linear_q4_dp4a_prequantized, kernels/ops/dp4a_smem_kernel.h:10-20).
Status linear_prequantized(const quant::QuantizedWeight& w, const Tensor& xq, const Tensor& xs,
                           Tensor& y, const LinearOptions& opt = {});

// The reference's entry (src/viper/linear.cpp:11-37): a Tensor cannot carry
// the per-group scales, so the quantized dtypes are routed to linear() and
// this overload only reports which call to use.
Status linear_forward(const Tensor& w, const Tensor& b, const Tensor& x, Tensor& y);

}  // namespace viper::ops
