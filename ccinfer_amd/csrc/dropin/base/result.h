// Result<T>: the reference's error-as-value convention (src/base/result.h:9-10,
// std::expected<T, ErrorCode>). libstdc++ 11 in this image has no <expected>, so a small
// expected-like type is provided when the standard one is missing; both spell
// `return unexpected(ErrorCode::X);` / `r.has_value()` / `r.error()` the same way.
#pragma once

#include <utility>
#include <version>

#include "base/error_code.h"

#if defined(__cpp_lib_expected) && __cpp_lib_expected >= 202202L
#include <expected>
namespace ccinfer {
template <typename T>
using Result = std::expected<T, ErrorCode>;
inline std::unexpected<ErrorCode> unexpected(ErrorCode e) { return std::unexpected<ErrorCode>(e); }
}  // namespace ccinfer
#else
namespace ccinfer {

struct Unexpected {
    ErrorCode code;
};
inline Unexpected unexpected(ErrorCode e) { return Unexpected{e}; }

template <typename T>
class Result {
public:
    Result(T v) : ok_(true), value_(std::move(v)) {}
    Result(Unexpected u) : ok_(false), err_(u.code) {}
    bool has_value() const noexcept { return ok_; }
    explicit operator bool() const noexcept { return ok_; }
    T& value() { return value_; }
    const T& value() const { return value_; }
    T& operator*() { return value_; }
    T* operator->() { return &value_; }
    ErrorCode error() const noexcept { return err_; }

private:
    bool ok_;
    T value_{};
    ErrorCode err_ = ErrorCode::Ok;
};

template <>
class Result<void> {
public:
    Result() = default;
    Result(Unexpected u) : err_(u.code) {}
    bool has_value() const noexcept { return err_ == ErrorCode::Ok; }
    explicit operator bool() const noexcept { return has_value(); }
    ErrorCode error() const noexcept { return err_; }

private:
    ErrorCode err_ = ErrorCode::Ok;
};

}  // namespace ccinfer
#endif
