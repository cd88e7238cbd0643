#pragma once

// Errors as values, with the reference's error codes (src/core/expected.h:10-52): a call that
// can fail returns Expected<T>, holding either the value or an Error{code, message}.

#include <string>
#include <utility>
#include <variant>

namespace axon {

enum class ErrorCode { InvalidArgument, Unsupported, OutOfRange, Io, Corrupt, Device };

struct Error {
  ErrorCode code;
  std::string message;
};

inline Error make_error(ErrorCode code, std::string message) { return Error{code, std::move(message)}; }

template <class T>
class Expected {
public:
  Expected(T value) : v_(std::move(value)) {}  // NOLINT(google-explicit-constructor)
  Expected(Error error) : v_(std::move(error)) {}  // NOLINT(google-explicit-constructor)
  explicit operator bool() const noexcept { return v_.index() == 0; }
  T& operator*() { return std::get<0>(v_); }
  const T& operator*() const { return std::get<0>(v_); }
  T* operator->() { return &std::get<0>(v_); }
  const T* operator->() const { return &std::get<0>(v_); }
  const Error& error() const { return std::get<1>(v_); }

private:
  std::variant<T, Error> v_;
};

}  // namespace axon
