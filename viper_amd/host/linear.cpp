// The linear() switch: the host side of the quantized path.  A closed switch
// on w.qtype (reference src/viper/linear.cpp:16-36) whose lossy cases call
// the gfx950 kernels through the C ABI (include/viper_qlinear.h).  Shapes and
// dtypes are checked here so the messages can name the offending argument;
// the C ABI re-checks everything it dereferences.
#include <string>

#include "viper/ops.h"
#include "viper_qlinear.h"

namespace viper::ops {
namespace {

Status from_code(int rc, const char* what) {
    switch (rc) {
        case VIPER_OK: return Status::Ok();
        case VIPER_UNIMPLEMENTED: return Status(StatusCode::UNIMPLEMENTED, what);
        case VIPER_INVALID_ARGUMENT: return Status(StatusCode::INVALID_ARGUMENT, std::string(what) + ": invalid argument");
        case VIPER_DEVICE_ERROR: return Status(StatusCode::CUDA_ERROR, std::string(what) + ": device error");
        case VIPER_SHAPE_MISMATCH: return Status(StatusCode::SHAPE_MISMATCH, std::string(what) + ": shape mismatch");
        case VIPER_OUT_OF_MEMORY: return Status(StatusCode::OUT_OF_MEMORY, std::string(what) + ": out of memory");
        default: return Status(StatusCode::INTERNAL, std::string(what) + ": internal error");
    }
}

Status bad(StatusCode c, const std::string& m) { return Status(c, "linear: " + m); }

// Rows M of an activation tensor of width K ([K] or [M, K]).
Status rows_of(const Tensor& t, i64 width, const char* name, i64& M) {
    const Shape& s = t.shape();
    if (s.rank() == 1) {
        M = 1;
        if (s[0] != width) return bad(StatusCode::SHAPE_MISMATCH, std::string(name) + " width");
        return Status::Ok();
    }
    if (s.rank() == 2) {
        M = s[0];
        if (s[1] != width) return bad(StatusCode::SHAPE_MISMATCH, std::string(name) + " width");
        return Status::Ok();
    }
    return bad(StatusCode::SHAPE_MISMATCH, std::string(name) + " must be [K] or [M, K]");
}

Status check_weight(const quant::QuantizedWeight& w) {
    switch (w.qtype) {
        case quant::QType::BF16:
            return Status::Unimplemented("linear BF16: lossless weights are not on the quantized path");
        case quant::QType::FP32:
            return Status::Unimplemented("linear FP32: lossless weights are not on the quantized path");
        case quant::QType::Q4_G64:
        case quant::QType::Q5_G64:
        case quant::QType::Q6_G64:
        case quant::QType::W8_G32: break;
        default: return bad(StatusCode::INVALID_ARGUMENT, "bad weight qtype");
    }
    if (w.data == nullptr || w.scales == nullptr) return bad(StatusCode::INVALID_ARGUMENT, "null weight data or scales");
    if (w.rows <= 0 || w.cols <= 0) return bad(StatusCode::INVALID_ARGUMENT, "non-positive weight shape");
    if (w.group_size != quant::group_size(w.qtype))
        return bad(StatusCode::INVALID_ARGUMENT, "group_size does not match the format");
    if (w.cols % w.group_size != 0) return bad(StatusCode::SHAPE_MISMATCH, "cols is not a multiple of the group");
    return Status::Ok();
}

Status check_out(const Tensor& y, i64 M, i64 N, const char* name) {
    if (y.dtype() != DType::BF16) return bad(StatusCode::INVALID_ARGUMENT, std::string(name) + " must be BF16");
    i64 My = 0;
    Status s = rows_of(y, N, name, My);
    if (!s.ok()) return s;
    if (My != M) return bad(StatusCode::SHAPE_MISMATCH, std::string(name) + " rows differ from x rows");
    return Status::Ok();
}

}  // namespace

usize linear_workspace_bytes(const quant::QuantizedWeight& w, i64 M) noexcept {
    if (M <= 0 || M > VIPER_QLINEAR_MAX_M) return 0;
    return viper_hip_qlinear_workspace_bytes(static_cast<int>(w.qtype), w.rows, w.cols, static_cast<int>(M));
}

Status linear(const quant::QuantizedWeight& w, const Tensor& x, Tensor& y) {
    return linear(w, x, y, LinearOptions{});
}

Status linear(const quant::QuantizedWeight& w, const Tensor& x, Tensor& y, const LinearOptions& opt) {
    Status s = check_weight(w);
    if (!s.ok()) return s;
    if (x.dtype() != DType::BF16) return bad(StatusCode::INVALID_ARGUMENT, "x must be BF16");
    i64 M = 0;
    s = rows_of(x, w.cols, "x", M);
    if (!s.ok()) return s;
    if (M <= 0 || M > VIPER_QLINEAR_MAX_M) return bad(StatusCode::INVALID_ARGUMENT, "x rows must be in [1, 16]");
    s = check_out(y, M, w.rows, "y");
    if (!s.ok()) return s;
    const void* res = nullptr;
    if (opt.residual != nullptr) {
        s = check_out(*opt.residual, M, w.rows, "residual");
        if (!s.ok()) return s;
        res = opt.residual->data();
    }
    const usize need = linear_workspace_bytes(w, M);
    if (need > opt.workspace_bytes || (need > 0 && opt.workspace == nullptr))
        return bad(StatusCode::INVALID_ARGUMENT,
                   "M > 1 needs a workspace of " + std::to_string(need) + " bytes (linear_workspace_bytes)");
    const int rc = viper_hip_qlinear(static_cast<int>(w.qtype), w.data, w.scales,
                                     static_cast<int>(w.scale_enc), w.group_size, w.rows, w.cols,
                                     x.data(), static_cast<int>(M), y.data(), res, opt.workspace,
                                     opt.workspace_bytes, opt.stream);
    return from_code(rc, "linear");
}

Status quantize_activations(const Tensor& x, i32 group, Tensor& xq, Tensor& xs, void* stream) {
    if (x.dtype() != DType::BF16) return Status(StatusCode::INVALID_ARGUMENT, "quantize_activations: x must be BF16");
    if (xq.dtype() != DType::INT8 || xs.dtype() != DType::FP32)
        return Status(StatusCode::INVALID_ARGUMENT, "quantize_activations: xq must be INT8 and xs FP32");
    if (group != 64 && group != 32) return Status(StatusCode::INVALID_ARGUMENT, "quantize_activations: group must be 64 or 32");
    const Shape& s = x.shape();
    if (s.rank() < 1) return Status(StatusCode::SHAPE_MISMATCH, "quantize_activations: x has no shape");
    const i64 K = s[s.rank() - 1];
    const i64 M = x.numel() / (K > 0 ? K : 1);
    if (K <= 0 || K % group != 0) return Status(StatusCode::SHAPE_MISMATCH, "quantize_activations: K % group != 0");
    if (xq.numel() != M * K || xs.numel() != M * (K / group))
        return Status(StatusCode::SHAPE_MISMATCH, "quantize_activations: xq/xs sizes");
    const int rc = viper_hip_quantize_act(group, x.data(), static_cast<int>(M), static_cast<int>(K), xq.data(),
                                          xs.data(), stream);
    return from_code(rc, "quantize_activations");
}

Status linear_prequantized(const quant::QuantizedWeight& w, const Tensor& xq, const Tensor& xs, Tensor& y,
                           const LinearOptions& opt) {
    Status s = check_weight(w);
    if (!s.ok()) return s;
    if (xq.dtype() != DType::INT8 || xs.dtype() != DType::FP32)
        return bad(StatusCode::INVALID_ARGUMENT, "xq must be INT8 and xs FP32");
    i64 M = 0;
    s = rows_of(xq, w.cols, "xq", M);
    if (!s.ok()) return s;
    if (M <= 0 || M > VIPER_QLINEAR_MAX_M) return bad(StatusCode::INVALID_ARGUMENT, "xq rows must be in [1, 16]");
    if (xs.numel() != M * (w.cols / w.group_size)) return bad(StatusCode::SHAPE_MISMATCH, "xs size");
    s = check_out(y, M, w.rows, "y");
    if (!s.ok()) return s;
    const void* res = nullptr;
    if (opt.residual != nullptr) {
        s = check_out(*opt.residual, M, w.rows, "residual");
        if (!s.ok()) return s;
        res = opt.residual->data();
    }
    const int rc = viper_hip_qlinear_prequantized(static_cast<int>(w.qtype), w.data, w.scales,
                                                  static_cast<int>(w.scale_enc), w.group_size, w.rows, w.cols,
                                                  xq.data(), xs.data(), static_cast<int>(M), y.data(), res,
                                                  opt.stream);
    return from_code(rc, "linear_prequantized");
}

Status linear_forward(const Tensor& w, const Tensor& b, const Tensor& x, Tensor& y) {
    (void)b;  // Viper's linears are bias-free
    (void)x;
    (void)y;
    switch (w.dtype()) {
        case DType::BF16:
            return Status::Unimplemented("linear_forward BF16: lossless weights are not on the quantized path");
        case DType::FP32:
            return Status::Unimplemented("linear_forward FP32: lossless weights are not on the quantized path");
        // The reference returns UNIMPLEMENTED for every lossy case
        // (src/viper/linear.cpp:26-32); so does this overload, since a Tensor
        // cannot carry the group scales: the quantized path is
        // ops::linear(quant::QuantizedWeight, x, y).
        case DType::Q4_G64:
            return Status::Unimplemented(
                "linear_forward Q4_G64: a Tensor cannot carry the group scales; use ops::linear(QuantizedWeight, x, y)");
        case DType::Q5_G64:
        case DType::Q6_G64:
            return Status::Unimplemented(
                "linear_forward Q5/Q6: a Tensor cannot carry the group scales; use ops::linear(QuantizedWeight, x, y)");
        case DType::W8_G32:
            return Status::Unimplemented(
                "linear_forward W8_G32: a Tensor cannot carry the group scales; use ops::linear(QuantizedWeight, x, y)");
        default: return Status(StatusCode::INVALID_ARGUMENT, "linear_forward: bad weight dtype");
    }
}

}  // namespace viper::ops
