// The engine's status type, restated so the hip backend compiles on its own.
// Same namespace, enumerator order and Status API as the reference
// (core/engine/error.h:12-77): the numeric codes are wire-stable there, and a
// drop-in backend must return exactly these values.
#pragma once

#include <cstdint>
#include <map>
#include <string>
#include <string_view>

namespace lykuro::nie {

enum class ErrorCode : int32_t {
    kOk = 0,
    kInvalidRequest,
    kAuthenticationFailed,
    kModelNotLoaded,
    kUnsupportedModel,
    kArtifactVerificationFailed,
    kContextLengthExceeded,
    kResourceExhausted,
    kCapacityExhausted,
    kDeadlineRejected,
    kDeadlineExceeded,
    kRequestCancelled,
    kEngineDraining,
    kGpuOom,
    kGpuUnhealthy,
    kInferenceFailed,
    kStreamConsumerSlow,
    kInternalError,
    kMetalBackendUnavailable,
    kMetalDeviceUnsupported,
    kMetalLibraryInvalid,
    kMetalPipelineCreationFailed,
    kMetalCommandFailed,
    kMetalMemoryPressure,
    kMetalOutOfMemory,
    kMetalExecutionTimeout,
    kMacProfileNotCertified,
    kBackendAbiMismatch,
};

std::string_view ErrorCodeName(ErrorCode code);
bool IsRetryable(ErrorCode code);

// Content-free status: a static message, the reporting component, and
// numeric details.
class Status {
public:
    Status() = default;
    Status(ErrorCode code, std::string message, std::string component = {})
        : code_(code), message_(std::move(message)), component_(std::move(component)) {}

    static Status Ok() { return Status(); }

    bool ok() const { return code_ == ErrorCode::kOk; }
    ErrorCode code() const { return code_; }
    const std::string& message() const { return message_; }
    const std::string& component() const { return component_; }
    bool retryable() const { return IsRetryable(code_); }

    Status& WithDetail(std::string_view key, int64_t value) {
        details_[std::string(key)] = value;
        return *this;
    }
    const std::map<std::string, int64_t>& details() const { return details_; }

private:
    ErrorCode code_ = ErrorCode::kOk;
    std::string message_;
    std::string component_;
    std::map<std::string, int64_t> details_;
};

}  // namespace lykuro::nie
