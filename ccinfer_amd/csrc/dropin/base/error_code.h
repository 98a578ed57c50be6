// Error codes of the drop-in C++ layer. The enumerators and their numeric order are the
// reference's interface (src/base/error_code.h:8-45) so callers switch on the same values;
// the C ABI (include/ccinfer_attn.h) returns these numbers as int.
#pragma once

#include <cstdint>
#include <string_view>

namespace ccinfer {

enum class ErrorCode : uint16_t {
    Ok = 0,
    CudaOutOfMemory,
    CudaLaunchFailed,
    CudaInvalidValue,
    CudaRuntimeError,
    CublasError,
    InvalidArgument,
    ModelLoadFailed,
    ModelConfigInvalid,
    ModelShapeMismatch,
    ModelUnsupportedArch,
    ModelUnsupportedDType,
    KVBlockExhausted,
    KVBlockDoubleFree,
    KVInvalidBlockTable,
    KVBlockHashCollision,
    RequestTooLong,
    RequestCancelled,
    RequestTimeout,
    ServerShuttingDown,
    MaxSequencesReached,
    BatchTranslationFailed,
    ChannelClosed,
    ChannelCancelled,
    ChannelError,
    NetworkBindFailed,
    Unsupported,
    InternalError,
};

// The device-side codes keep the reference's names; on this build "Cuda*" denotes the
// corresponding HIP runtime condition.
inline constexpr std::string_view error_message(ErrorCode c) noexcept {
    switch (c) {
        case ErrorCode::Ok: return "ok";
        case ErrorCode::CudaOutOfMemory: return "device out of memory";
        case ErrorCode::CudaLaunchFailed: return "kernel launch failed";
        case ErrorCode::CudaInvalidValue: return "device invalid value";
        case ErrorCode::CudaRuntimeError: return "device runtime error";
        case ErrorCode::CublasError: return "BLAS error";
        case ErrorCode::InvalidArgument: return "invalid argument";
        case ErrorCode::Unsupported: return "unsupported operation";
        case ErrorCode::InternalError: return "internal error";
        default: return "error";
    }
}

}  // namespace ccinfer
