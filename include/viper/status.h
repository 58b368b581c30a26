// Status value type of the Viper host API.
//
// Same StatusCode numbering and Status surface as the reference
// (itzrnvr/viper include/viper/status.h:12-42): every public call returns a
// Status, never throws, and Status::Ok() is the success value.  The C ABI
// (include/viper_qlinear.h) returns these codes as plain ints.
#pragma once

#include <string>
#include <string_view>
#include <utility>

namespace viper {

enum class StatusCode : int {
    OK = 0,
    UNIMPLEMENTED = 1,
    INVALID_ARGUMENT = 2,
    CUDA_ERROR = 3,  // device (HIP) error; the reference's name is kept
    SHAPE_MISMATCH = 4,
    OUT_OF_MEMORY = 5,
    IO_ERROR = 6,
    INTERNAL = 99,
};

class Status {
  public:
    Status() = default;
    explicit Status(StatusCode code, std::string message = "")
        : code_(code), message_(std::move(message)) {}

    StatusCode code() const noexcept { return code_; }
    bool ok() const noexcept { return code_ == StatusCode::OK; }
    explicit operator bool() const noexcept { return ok(); }
    std::string_view message() const noexcept { return message_; }

    static Status Ok() { return Status(StatusCode::OK); }
    static Status Unimplemented(std::string_view what = "") {
        return Status(StatusCode::UNIMPLEMENTED, std::string(what));
    }

  private:
    StatusCode code_ = StatusCode::OK;
    std::string message_;
};

}  // namespace viper
