// Error model of the tbn host runtime: the reference's ErrorCode values and
// exception classes (tbn-runtime/include/tbn/utils/errors.hpp:10-93), plus the
// mapping from the C ABI's integer status codes to those exceptions.
#pragma once

#include <stdexcept>
#include <string>

namespace tbn {

enum class ErrorCode {
    SUCCESS = 0,
    INVALID_ARGUMENT = -1,
    OUT_OF_MEMORY = -2,
    NOT_IMPLEMENTED = -3,
    INVALID_MODEL = -4,
    RUNTIME_ERROR = -5,
    QUANTIZATION_ERROR = -6,
    INVALID_SHAPE = -7,
    DEVICE_NOT_SUPPORTED = -8,
    ONNX_PARSE_ERROR = -9,
    OPERATOR_NOT_SUPPORTED = -10
};

class TBNError : public std::exception {
public:
    TBNError(ErrorCode code, std::string message) : code_(code), message_(std::move(message)) {}
    const char* what() const noexcept override { return message_.c_str(); }
    ErrorCode code() const noexcept { return code_; }

private:
    ErrorCode code_;
    std::string message_;
};

#define TBN_DEFINE_ERROR(Name, Code)                                          \
    class Name : public TBNError {                                            \
    public:                                                                   \
        explicit Name(const std::string& msg) : TBNError(ErrorCode::Code, msg) {} \
    };

TBN_DEFINE_ERROR(InvalidArgumentError, INVALID_ARGUMENT)
TBN_DEFINE_ERROR(OutOfMemoryError, OUT_OF_MEMORY)
TBN_DEFINE_ERROR(NotImplementedError, NOT_IMPLEMENTED)
TBN_DEFINE_ERROR(InvalidModelError, INVALID_MODEL)
TBN_DEFINE_ERROR(RuntimeError, RUNTIME_ERROR)
TBN_DEFINE_ERROR(QuantizationError, QUANTIZATION_ERROR)
TBN_DEFINE_ERROR(InvalidShapeError, INVALID_SHAPE)
TBN_DEFINE_ERROR(DeviceNotSupportedError, DEVICE_NOT_SUPPORTED)
TBN_DEFINE_ERROR(OperatorNotSupportedError, OPERATOR_NOT_SUPPORTED)

#undef TBN_DEFINE_ERROR

// Throws the exception class matching a non-zero C ABI status; `what` names
// the operation and the library's last-error message is appended.
[[noreturn]] void throw_status(int status, const std::string& what);

// Checks a C ABI status.
inline void check_status(int status, const char* what) {
    if (status != 0) throw_status(status, what);
}

}  // namespace tbn

#define TBN_CHECK(cond, ErrorType, msg)  \
    do {                                 \
        if (!(cond)) throw ErrorType(msg); \
    } while (0)
